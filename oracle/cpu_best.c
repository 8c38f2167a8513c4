/* CPU-C, the best-effort host baseline of the W4A16 decode GEMV (test infrastructure, timed by
 * bench.py's CPU-baseline leg only; it is not the parity checker: cf_oracle.c is).
 *
 * y[n] = sum_k x[k] * (q[n, k] - z[n, g]) * s[n, g] over the canonical INT4 g128 arrays (codes
 * u32 [N, K/8], f16 scales [N, GP], u4 zero points [N, ceil(G/8)]), the semantics of
 * codegen/eval.rs:1465-1507 over the dequantized weight.  Built -O3 with AVX2 / FMA / F16C and
 * OpenMP: rows split over the threads, each group's products summed in f32 vector lanes with
 * the zero point folded out, y = sum_g s_g * (sum_i x_i q_i - z_g * sum_i x_i).  Its rounding is
 * not the reference's sequential f32 loop (the port in cf_oracle.c keeps that one). */
#include <immintrin.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>

static float f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }

/* x: f32 [k]; threads <= 0: OpenMP's default. */
void cpub_gemv_w4a16(const float *x, int64_t n, int64_t k, const uint32_t *codes, const uint16_t *scales_f16,
                     const uint32_t *zeros, float *y, int threads) {
    const int64_t G = k / 128, GP = (G + 7) / 8 * 8, ZW = (G + 7) / 8, KW = k / 8;
    float *xs = (float *)malloc(sizeof(float) * (size_t)(G > 0 ? G : 1));
    for (int64_t g = 0; g < G; ++g) {
        float s = 0.0f;
        for (int i = 0; i < 128; ++i) s += x[g * 128 + i];
        xs[g] = s;
    }
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        const uint32_t *cw = codes + r * KW;
        float acc = 0.0f;
        for (int64_t g = 0; g < G; ++g) {
            const float *xg = x + g * 128;
            const uint32_t *wg = cw + g * 16;
            float dot[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int w = 0; w < 16; ++w) {
                const uint32_t v = wg[w];
#pragma omp simd
                for (int j = 0; j < 8; ++j) dot[j] += xg[8 * w + j] * (float)((v >> (4 * j)) & 15u);
            }
            const float d = ((dot[0] + dot[1]) + (dot[2] + dot[3])) + ((dot[4] + dot[5]) + (dot[6] + dot[7]));
            const float z = (float)((zeros[r * ZW + g / 8] >> (4 * (g % 8))) & 15u);
            acc += f16_to_f32(scales_f16[r * GP + g]) * (d - z * xs[g]);
        }
        y[r] = acc;
    }
    free(xs);
}
