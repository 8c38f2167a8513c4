/* CPU-B, the "codegen-faithful" host baseline of the W4A16 decode GEMV (test infrastructure,
 * timed by bench.py's CPU-baseline leg only; cf_oracle.c is the parity checker).
 *
 * The reference's Rust emitter lowers `castforge.fused_qmatmul` to one loop nest with the dequant
 * inline (codegen/targets/rust_composites.rs:176-244; the plain matmul at rust.rs:1061-1076):
 *
 *     for m in 0..M { for n in 0..N { let mut acc = 0.0_f32;
 *         for k in 0..K { let w_val = ((w[n * K + k] as i32 - zp) as f32) * scale; acc += a[m * K + k] * w_val; }
 *         out[m * N + n] = acc; } }
 *
 * and its JIT builds that text with `rustc -C opt-level=3` and no target-cpu (autotune.rs:636-645):
 * x86-64 baseline code, no fused multiply-add (Rust never contracts), and no vectorised f32
 * reduction (the sum order is fixed).  This is that loop nest for the INT4 g128 format, whose
 * zero point and scale are per (row, group) instead of per tensor: the nibble, zero point and
 * scale are read inside the k loop, as the emitted code reads its i8 code.  Built -O3 without
 * -march and with -ffp-contract=off, one thread (the emitted code has none). */
#include <stdint.h>

static float f16_bits_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    union { uint32_t u; float f; } v;
    if (e == 0) {  /* zero or subnormal: m * 2^-24, exact in f32 */
        v.f = (float)m * 5.9604644775390625e-8f;
        v.u |= s;
        return v.f;
    }
    v.u = e == 31 ? (s | 0x7F800000u | (m << 13)) : (s | ((e + 112u) << 23) | (m << 13));
    return v.f;
}

/* x: f32 [m, k] (the activations the emitted code reads), y: f32 [m, n]. */
void cpcg_gemv_w4a16(const float *x, int64_t m, int64_t n, int64_t k, const uint32_t *codes,
                     const uint16_t *scales_f16, const uint32_t *zeros, float *y) {
    const int64_t G = k / 128, GP = (G + 7) / 8 * 8, ZW = (G + 7) / 8, KW = k / 8;
    for (int64_t mi = 0; mi < m; ++mi)
        for (int64_t ni = 0; ni < n; ++ni) {
            float acc = 0.0f;
            for (int64_t ki = 0; ki < k; ++ki) {
                const int64_t g = ki / 128;
                const int32_t q = (int32_t)((codes[ni * KW + ki / 8] >> (4 * (ki % 8))) & 15u);
                const int32_t zp = (int32_t)((zeros[ni * ZW + g / 8] >> (4 * (g % 8))) & 15u);
                const float w_val = (float)(q - zp) * f16_bits_to_f32(scales_f16[ni * GP + g]);
                acc += x[mi * k + ki] * w_val;
            }
            y[mi * n + ni] = acc;
        }
}
