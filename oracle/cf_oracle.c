/*
 * CPU oracle for the quantized-weight hot path — TEST INFRASTRUCTURE ONLY (see cf_oracle.h).
 *
 * Compiled with -O2 -ffp-contract=off and without fast-math: every f32 multiply, add and
 * divide rounds on its own, as the reference's Rust code does (Rust never contracts a*b+c).
 * Citations are to sungdomo/CastForge.
 */
#include "cf_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Rust `x as u8` / `x as i8` / `x as i32`: saturating, NaN -> 0. */
static inline int rust_as_sat(float x, int lo, int hi) {
    if (isnan(x)) return 0;
    if (x <= (float)lo) return lo;
    if (x >= (float)hi) return hi;
    return (int)x; /* truncation toward zero */
}

/* Rust f32::round (half away from zero) or IEEE round-half-even. */
static inline float round_mode_f(float x, int mode) {
    return mode == ORC_ROUND_HALF_EVEN ? nearbyintf(x) : roundf(x);
}

/* Rust f32::clamp: NaN stays NaN. */
static inline float rust_clamp(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* ============================ scalar converters ========================================= */

/* tensor_store.rs:109-111: bf16 by truncation of the low 16 bits */
uint16_t orc_f32_to_bf16_trunc(float v) { return (uint16_t)(f2u(v) >> 16); }

/* tensor_store.rs:84-102: f16 by mantissa truncation, overflow -> Inf, underflow -> signed 0 */
uint16_t orc_f32_to_f16_trunc(float v) {
    uint32_t bits = f2u(v);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    int32_t exp = (int32_t)((bits >> 23) & 0xff);
    uint32_t mant = bits & 0x007fffff;
    if (exp == 255) return sign | 0x7c00 | (mant != 0 ? 0x0200 : 0);
    int32_t new_exp = exp - 127 + 15;
    if (new_exp >= 31) return sign | 0x7c00;
    if (new_exp <= 0) return sign;
    return sign | (uint16_t)(new_exp << 10) | (uint16_t)(mant >> 13);
}

/* tensor_store.rs:59-82: exact f16 -> f32 including subnormals */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, out;
    if (exp == 0) {
        if (mant == 0) {
            out = sign << 31;
        } else {
            uint32_t m = mant, e = 127 - 14;
            while ((m & 0x400u) == 0) { m <<= 1; e -= 1; }
            m &= 0x3ffu;
            out = (sign << 31) | (e << 23) | (m << 13);
        }
    } else if (exp == 0x1f) {
        out = (sign << 31) | 0x7f800000u | (mant << 13);
    } else {
        out = (sign << 31) | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    return u2f(out);
}

/* tensor_store.rs:104-107 */
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* IEEE RNE f32 -> bf16; NaN stays a quiet NaN of the same sign. */
uint16_t orc_f32_to_bf16_rne(float v) {
    uint32_t u = f2u(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* IEEE RNE f32 -> f16 with subnormals, overflow to Inf, NaN -> quiet NaN. Written from the
 * binary16 definition: the value is rounded once, at the f16 precision of its binade. */
uint16_t orc_f32_to_f16_rne(float v) {
    uint32_t u = f2u(v);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7e00u;
    if (a >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to Inf */
    int32_t e = (int32_t)(a >> 23) - 127;
    if (e < -25) return sign; /* < 2^-25: below half of the smallest subnormal */
    uint32_t m = (a & 0x7fffffu) | 0x800000u; /* 24-bit significand, value m * 2^(e-23) */
    if (e < -14) {
        /* subnormal: result = RNE(value / 2^-24) = RNE(m * 2^(e-23+24)) */
        int shift = -(e + 1); /* 23-24-e... = -e-1, in [14, 24] */
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return sign | (uint16_t)q; /* q may reach 0x400 = smallest normal, still correct */
    }
    uint32_t q = (m >> 13) & 0x3ffu, rem = m & 0x1fffu;
    uint32_t he = (uint32_t)(e + 15);
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) {
        q++;
        if (q == 0x400u) { q = 0; he++; }
    }
    if (he >= 31) return sign | 0x7c00u;
    return sign | (uint16_t)((he << 10) | q);
}

/* ================================ E4M3FN codec ========================================== */

/* mutable_loads.rs:367-411 restated step by step (log2/floor exponent, RNE mantissa). */
uint8_t orc_f32_to_e4m3fn(float v) {
    if (isnan(v)) return 0x7F;
    uint8_t sign = signbit(v) ? 0x80 : 0x00;
    float abs_v = fabsf(v);
    if (abs_v == 0.0f) return sign;
    if (abs_v >= 448.0f) return sign | 0x7E;
    const float min_normal = 1.0f / 64.0f;
    if (abs_v < min_normal) {
        float scaled = abs_v * 512.0f;
        float fl = floorf(scaled);
        float diff = scaled - fl;
        uint8_t mant = (uint8_t)rust_as_sat(fl, 0, 255);
        if (diff > 0.5f || (diff == 0.5f && (mant & 1) == 1)) mant += 1;
        return sign | mant;
    }
    int32_t exp_unbiased = rust_as_sat(floorf(log2f(abs_v)), -2147483647 - 1, 2147483647);
    uint8_t exp_biased = (uint8_t)(exp_unbiased + 7);
    float norm = abs_v / ldexpf(1.0f, exp_unbiased) - 1.0f; /* powi(2, e) is exact */
    float scaled_m = norm * 8.0f;
    float floor_m = floorf(scaled_m);
    float diff_m = scaled_m - floor_m;
    uint8_t mant = (uint8_t)rust_as_sat(floor_m, 0, 255);
    if (diff_m > 0.5f || (diff_m == 0.5f && (mant & 1) == 1)) mant += 1;
    uint8_t e = exp_biased, m = mant;
    if (m == 8) { m = 0; e += 1; }
    if (e > 15 || (e == 15 && m >= 7)) return sign | 0x7E;
    return (uint8_t)(sign | (e << 3) | m);
}

/* mutable_loads.rs:415-432 */
float orc_e4m3fn_to_f32(uint8_t b) {
    float sign = (b & 0x80) ? -1.0f : 1.0f;
    uint8_t exp = (b >> 3) & 0x0F, mant = b & 0x07;
    if (exp == 0x0F && mant == 0x07) return NAN;
    if (exp == 0) {
        if (mant == 0) return sign < 0.0f ? -0.0f : 0.0f;
        return sign * ((float)mant / 512.0f);
    }
    float scale = ldexpf(1.0f, (int)exp - 7);
    return sign * (1.0f + (float)mant / 8.0f) * scale;
}

/* Independent encoder: pure integer RNE on the f32 bit pattern with saturation at 448. */
uint8_t orc_f32_to_e4m3fn_int(float v) {
    uint32_t b = f2u(v);
    uint8_t s = (uint8_t)((b >> 24) & 0x80u);
    uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7F;
    if (a >= 0x43e00000u) return s | 0x7E; /* |v| >= 448 (incl. Inf) */
    int32_t E = (int32_t)(a >> 23) - 127;
    uint32_t m = a & 0x7fffffu;
    if (E < -6) {
        /* e4m3 subnormal: q = RNE(|v| * 2^9) */
        uint32_t sig = (a >> 23) ? (m | 0x800000u) : m;
        int32_t Eeff = (a >> 23) ? E : -126;
        int32_t shift = 14 - Eeff; /* value = sig * 2^(Eeff-23); * 2^9 -> >> (14 - Eeff) */
        if (shift >= 32) return s;
        uint32_t q = sig >> shift, rem = sig & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint8_t)(s | q);
    }
    uint32_t q = m >> 20, rem = m & 0xfffffu;
    uint32_t eb = (uint32_t)(E + 7);
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) {
        q++;
        if (q == 8) { q = 0; eb++; }
    }
    if (eb > 15 || (eb == 15 && q >= 7)) return s | 0x7E;
    return (uint8_t)(s | (eb << 3) | q);
}

/* The reference codec takes the exponent from floorf(log2f(|v|)).  For 16 positive inputs
 * just below a power of two, log2f rounds up to the integer, the mantissa term goes negative,
 * saturates to 0 and is then bumped to 1 (mutable_loads.rs:390-401), so the reference returns
 * code+1 where a true RNE encoder returns code.  The set, found by scanning every positive
 * f32 with glibc's log2f, is: f32 exponent field e in [0x79, 0x86] with mantissa >= the
 * threshold below (0 = no quirk in that binade). */
static const uint32_t E4M3_QUIRK_MIN_MANT[14] = {
    0x7ffffe, 0x7ffffe, 0x7fffff, 0x7fffff, 0, 0, 0, 0,
    0x7fffff, 0x7fffff, 0x7ffffe, 0x7ffffe, 0x7ffffe, 0x7ffffe};

uint8_t orc_f32_to_e4m3fn_fast(float v) {
    uint8_t c = orc_f32_to_e4m3fn_int(v);
    uint32_t a = f2u(v) & 0x7fffffffu, e = a >> 23, m = a & 0x7fffffu;
    if (e >= 0x79 && e <= 0x86) {
        uint32_t t = E4M3_QUIRK_MIN_MANT[e - 0x79];
        if (t != 0 && m >= t) c = (uint8_t)(c + 1);
    }
    return c;
}

int64_t orc_e4m3_crosscheck(uint32_t lo, uint32_t hi, uint32_t stride, int use_fast,
                            uint32_t *first_bad) {
    int64_t bad = 0;
    uint64_t first = UINT64_MAX;
    if (stride == 0) stride = 1;
    int64_t count = ((int64_t)hi - (int64_t)lo + stride - 1) / stride;
#pragma omp parallel for reduction(+ : bad) reduction(min : first) schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        uint32_t x = lo + (uint32_t)i * stride;
        float f = u2f(x);
        uint8_t other = use_fast ? orc_f32_to_e4m3fn_fast(f) : orc_f32_to_e4m3fn_int(f);
        if (orc_f32_to_e4m3fn(f) != other) {
            bad++;
            if (x < first) first = x;
        }
    }
    if (first_bad) *first_bad = bad ? (uint32_t)first : 0;
    return bad;
}

/* ============================ reference quantizers ====================================== */

/* formats.rs:654-660 */
void orc_int_bounds(int bits, int *eff_bits, float *qmin, float *qmax) {
    if (bits == 4) { *eff_bits = 4; *qmin = -8.0f; *qmax = 7.0f; }
    else { *eff_bits = 8; *qmin = -128.0f; *qmax = 127.0f; }
}

/* formats.rs:670-677: amax = fold(0, f32::max(acc, |v|)); scale = amax<1e-12 ? 1 : amax/qmax;
 * q = (v/scale).round().clamp(qmin,qmax) as i8 */
float orc_quantize_symmetric(const float *v, int64_t n, int bits, int round_mode, int8_t *q) {
    int eb; float qmin, qmax;
    orc_int_bounds(bits, &eb, &qmin, &qmax);
    float amax = 0.0f;
    for (int64_t i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(v[i]));
    float scale = amax < 1e-12f ? 1.0f : amax / qmax;
    for (int64_t i = 0; i < n; ++i) {
        float r = rust_clamp(round_mode_f(v[i] / scale, round_mode), qmin, qmax);
        q[i] = (int8_t)rust_as_sat(r, -128, 127);
    }
    return scale;
}

/* formats.rs:680-688: format!("{:.6}") then trim '0' then trim '.', append ".0" if no dot.
 * glibc printf("%.6f") rounds the exact binary value half-to-even, as Rust's formatter does. */
void orc_scale_string(float scale, char *buf, int buflen) {
    char tmp[128];
    snprintf(tmp, sizeof tmp, "%.6f", (double)scale);
    size_t len = strlen(tmp);
    while (len > 0 && tmp[len - 1] == '0') tmp[--len] = 0;
    while (len > 0 && tmp[len - 1] == '.') tmp[--len] = 0;
    if (!strchr(tmp, '.')) { tmp[len++] = '.'; tmp[len++] = '0'; tmp[len] = 0; }
    snprintf(buf, (size_t)buflen, "%s", tmp);
}

/* descending order under Rust's f32::total_cmp (positive NaN sorts above +Inf) */
static int cmp_total_desc(const void *pa, const void *pb) {
    uint32_t a = f2u(*(const float *)pa), b = f2u(*(const float *)pb);
    int32_t ka = (int32_t)(a ^ (((uint32_t)((int32_t)a >> 31)) >> 1));
    int32_t kb = (int32_t)(b ^ (((uint32_t)((int32_t)b >> 31)) >> 1));
    return (ka < kb) - (ka > kb);
}

/* schemes.rs:485-549 */
int64_t orc_quantize_groupwise(const float *v, int64_t n, int bits, int64_t group_size,
                               int awq_salient, float salient_ratio, int round_mode,
                               float *deq, float *scales, float *salient_thresh) {
    int eb; float qmin, qmax;
    orc_int_bounds(bits, &eb, &qmin, &qmax);
    int64_t gs = group_size < 2 ? 2 : group_size;
    float ratio = rust_clamp(salient_ratio, 0.001f, 0.5f);
    float *sorted = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    for (int64_t i = 0; i < n; ++i) sorted[i] = fabsf(v[i]);
    qsort(sorted, (size_t)n, sizeof(float), cmp_total_desc);
    float cnt_f = ceilf((float)n * ratio);
    int64_t salient_count = (int64_t)rust_as_sat(cnt_f, 0, 2147483647);
    if (salient_count < 1) salient_count = 1;
    if (salient_count > n) salient_count = n;
    float thresh = (n > 0 && salient_count >= 1) ? sorted[salient_count - 1] : 0.0f;
    free(sorted);
    if (salient_thresh) *salient_thresh = thresh;
    int64_t g = 0;
    for (int64_t c0 = 0; c0 < n; c0 += gs, ++g) {
        int64_t c1 = c0 + gs < n ? c0 + gs : n;
        float gmax = 0.0f;
        for (int64_t i = c0; i < c1; ++i) gmax = fmaxf(gmax, fabsf(v[i]));
        float scale = gmax < 1e-12f ? 1.0f : gmax / qmax;
        if (scales) scales[g] = scale;
        for (int64_t i = c0; i < c1; ++i) {
            float eff = (awq_salient && fabsf(v[i]) >= thresh) ? scale * 0.5f : scale;
            float q = rust_clamp(round_mode_f(v[i] / eff, round_mode), qmin, qmax);
            deq[i] = q * eff;
        }
    }
    return salient_count;
}

/* schemes.rs:681-713 */
void orc_quantize_fp8_grid(const float *v, int64_t n, int e5m2, int mxfp8, int64_t block_size,
                           float *deq) {
    float fp8_max = e5m2 ? 57344.0f : 448.0f;
    float grid_steps = e5m2 ? 15.0f : 31.0f;
    int64_t bs = block_size < 4 ? 4 : block_size;
    for (int64_t c0 = 0; c0 < n; c0 += bs) {
        int64_t c1 = c0 + bs < n ? c0 + bs : n;
        float amax = 0.0f;
        for (int64_t i = c0; i < c1; ++i) amax = fmaxf(amax, fabsf(v[i]));
        float raw = amax < 1e-12f ? 1.0f : amax / fp8_max;
        float scale = mxfp8 ? powf(2.0f, ceilf(log2f(raw))) : raw;
        float step = fmaxf(fp8_max / grid_steps, 1e-6f);
        for (int64_t i = c0; i < c1; ++i) {
            float scaled = rust_clamp(v[i] / scale, -fp8_max, fp8_max);
            float q = roundf(scaled / step) * step;
            deq[i] = q * scale;
        }
    }
}

/* Closed form of ceilf(log2f(raw)) for a positive normal f32, the MX exponent of
 * schemes.rs:706: e for raw = 2^e, else e + 1 unless log2f's f32 rounding lands exactly on e,
 * which happens for raw = 2^e (1 + m 2^-23) with m below (2^h - 1) 2^23, h the half-spacing
 * of f32 values next to e (below |e| when e < 0).  The GPU kernel computes the exponent this
 * way; orc_mx_scale_crosscheck compares it with glibc's log2f. */
int orc_mx_scale_exp_model(float raw) {
    uint32_t b = f2u(raw);
    int e = (int)((b >> 23) & 0xffu) - 127;
    uint32_t m = b & 0x7fffffu;
    if (m == 0) return e;
    if (e == 0) return 1;
    int a = e > 0 ? e : -e;
    int fl = 31 - __builtin_clz((unsigned)a);
    double h = (e < 0 && (a & (a - 1)) == 0) ? ldexp(1.0, fl - 25) : ldexp(1.0, fl - 24);
    double thr = (exp2(h) - 1.0) * 8388608.0;
    return (double)m < thr ? e : e + 1;
}

/* Counts f32 bit patterns x in [lo, hi) (positive normals) where ceilf(log2f(x)) differs from
 * the closed form. */
int64_t orc_mx_scale_crosscheck(uint32_t lo, uint32_t hi, uint32_t *first_bad) {
    int64_t bad = 0;
    uint64_t first = UINT64_MAX;
    int64_t count = (int64_t)hi - (int64_t)lo;
#pragma omp parallel for reduction(+ : bad) reduction(min : first) schedule(static)
    for (int64_t i = 0; i < count; ++i) {
        uint32_t x = lo + (uint32_t)i;
        float f = u2f(x);
        if ((int)ceilf(log2f(f)) != orc_mx_scale_exp_model(f)) {
            bad++;
            if (x < first) first = x;
        }
    }
    if (first_bad) *first_bad = bad ? (uint32_t)first : 0;
    return bad;
}

/* ======================= BASELINE schemes (written spec) ================================ */

/* Per-output-channel symmetric: formats.rs:670-677 applied to every row of [n, k]. */
void orc_quantize_int8_rows(const float *v, int64_t n, int64_t k, int bits, int round_mode,
                            int8_t *q, float *scales) {
    for (int64_t r = 0; r < n; ++r)
        scales[r] = orc_quantize_symmetric(v + r * k, k, bits, round_mode, q + r * k);
}

/* INT4 asymmetric, groups of `group` along K (last group may be short), K % 8 == 0.
 *   mx/mn = NaN-ignoring max/min of the group; range = mx - mn (f32)
 *   range >= 1e-12 ? h = f16_rne(range / 15) : h = f16(1.0);  h == +0 -> 0x0001; h == Inf -> 0x7BFF
 *   s = f32(h);  z = clamp(rne(-mn / s), 0, 15)  (NaN -> 0)
 *   q = clamp(rne(v / s) [NaN -> 0] + z, 0, 15)
 * codes[n][k/8] u32: element k at bits 4*(k%8); scales[n][GP] f16 bits with GP = 8*ceil(G/8)
 * (rows padded to whole 8-group blocks, pad entries 0, so 8 scales load as one aligned 16 B);
 * zeros[n][GP/8] u32: zero of group g at bits 4*(g%8). */
static inline uint16_t int4_scale_bits(float mx, float mn) {
    float range = mx - mn;
    uint16_t h;
    if (range >= 1e-12f) h = orc_f32_to_f16_rne(range / 15.0f);
    else h = 0x3C00;
    if (h == 0) h = 0x0001;
    if (h == 0x7C00) h = 0x7BFF;
    return h;
}

void orc_quantize_int4g(const float *v, int64_t n, int64_t k, int64_t group, uint32_t *codes,
                        uint16_t *scales_f16, uint32_t *zeros) {
    int64_t G = (k + group - 1) / group, ZW = (G + 7) / 8, GP = ZW * 8, KW = k / 8;
    for (int64_t r = 0; r < n; ++r) {
        const float *row = v + r * k;
        for (int64_t w = 0; w < KW; ++w) codes[r * KW + w] = 0;
        for (int64_t w = 0; w < ZW; ++w) zeros[r * ZW + w] = 0;
        for (int64_t g = 0; g < GP; ++g) scales_f16[r * GP + g] = 0;
        for (int64_t g = 0; g < G; ++g) {
            int64_t k0 = g * group, k1 = k0 + group < k ? k0 + group : k;
            float mx = -INFINITY, mn = INFINITY;
            for (int64_t i = k0; i < k1; ++i) { mx = fmaxf(mx, row[i]); mn = fminf(mn, row[i]); }
            uint16_t h = int4_scale_bits(mx, mn);
            float s = orc_f16_to_f32(h);
            float zf = nearbyintf(-mn / s);
            if (isnan(zf)) zf = 0.0f;
            zf = fminf(fmaxf(zf, 0.0f), 15.0f);
            uint32_t z = (uint32_t)zf;
            scales_f16[r * GP + g] = h;
            zeros[r * ZW + g / 8] |= z << (4 * (g % 8));
            for (int64_t i = k0; i < k1; ++i) {
                float t = nearbyintf(row[i] / s);
                if (isnan(t)) t = 0.0f;
                float qf = fminf(fmaxf(t + zf, 0.0f), 15.0f);
                codes[r * KW + i / 8] |= ((uint32_t)qf) << (4 * (i % 8));
            }
        }
    }
}

/* AWQ-style pre-scale: quantize W'[r][c] = f32(W[r][c] * s[c]). */
void orc_quantize_int4g_awq(const float *v, const float *s, int64_t n, int64_t k, int64_t group,
                            uint32_t *codes, uint16_t *scales_f16, uint32_t *zeros) {
    float *t = (float *)malloc(sizeof(float) * (size_t)(n * k > 0 ? n * k : 1));
    for (int64_t r = 0; r < n; ++r)
        for (int64_t c = 0; c < k; ++c) t[r * k + c] = v[r * k + c] * s[c];
    orc_quantize_int4g(t, n, k, group, codes, scales_f16, zeros);
    free(t);
}

void orc_dequantize_int4g(const uint32_t *codes, const uint16_t *scales_f16,
                          const uint32_t *zeros, int64_t n, int64_t k, int64_t group, float *out) {
    int64_t G = (k + group - 1) / group, ZW = (G + 7) / 8, GP = ZW * 8, KW = k / 8;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) {
            int64_t g = i / group;
            int32_t q = (int32_t)((codes[r * KW + i / 8] >> (4 * (i % 8))) & 0xFu);
            int32_t z = (int32_t)((zeros[r * ZW + g / 8] >> (4 * (g % 8))) & 0xFu);
            out[r * k + i] = (float)(q - z) * orc_f16_to_f32(scales_f16[r * GP + g]);
        }
}

/* NF4: the 16-entry normal-float table of QLoRA (Dettmers et al. 2023), as f32. */
const float ORC_NF4_TABLE[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

/* code = #{i : x > mid_i}, mid_i = 0.5f * (T[i] + T[i+1]) in f32; a tie goes to the lower
 * code; NaN -> code 7 (the 0.0 entry). */
uint8_t orc_nf4_code(float x) {
    if (isnan(x)) return 7;
    uint8_t c = 0;
    for (int i = 0; i < 15; ++i) {
        float mid = 0.5f * (ORC_NF4_TABLE[i] + ORC_NF4_TABLE[i + 1]);
        if (x > mid) c++;
    }
    return c;
}

/* absmax = fold(0, max(acc,|v|)) per block of `block` along K; stored = absmax<1e-12 ? 1 : absmax;
 * code = nf4_code(v / stored); dequant = T[code] * stored. */
void orc_quantize_nf4(const float *v, int64_t n, int64_t k, int64_t block, uint32_t *codes,
                      float *absmax) {
    int64_t B = (k + block - 1) / block, KW = k / 8;
    for (int64_t r = 0; r < n; ++r) {
        const float *row = v + r * k;
        for (int64_t w = 0; w < KW; ++w) codes[r * KW + w] = 0;
        for (int64_t b = 0; b < B; ++b) {
            int64_t k0 = b * block, k1 = k0 + block < k ? k0 + block : k;
            float am = 0.0f;
            for (int64_t i = k0; i < k1; ++i) am = fmaxf(am, fabsf(row[i]));
            float st = am < 1e-12f ? 1.0f : am;
            absmax[r * B + b] = st;
            for (int64_t i = k0; i < k1; ++i)
                codes[r * KW + i / 8] |= ((uint32_t)orc_nf4_code(row[i] / st)) << (4 * (i % 8));
        }
    }
}

void orc_dequantize_nf4(const uint32_t *codes, const float *absmax, int64_t n, int64_t k,
                        int64_t block, float *out) {
    int64_t B = (k + block - 1) / block, KW = k / 8;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) {
            uint32_t c = (codes[r * KW + i / 8] >> (4 * (i % 8))) & 0xFu;
            out[r * k + i] = ORC_NF4_TABLE[c] * absmax[r * B + i / block];
        }
}

/* FP8 per row: amax = fold(0, max(acc,|v|)); scale = amax<1e-12 ? 1 : amax/448;
 * code = e4m3fn(v / scale) with the codec of mutable_loads.rs:367-411. */
void orc_quantize_fp8_rows(const float *v, int64_t rows, int64_t cols, uint8_t *codes,
                           float *scales) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *row = v + r * cols;
        float am = 0.0f;
        for (int64_t i = 0; i < cols; ++i) am = fmaxf(am, fabsf(row[i]));
        float s = am < 1e-12f ? 1.0f : am / 448.0f;
        scales[r] = s;
        for (int64_t i = 0; i < cols; ++i) codes[r * cols + i] = orc_f32_to_e4m3fn(row[i] / s);
    }
}

void orc_quantize_fp8_rows_bf16(const uint16_t *v, int64_t rows, int64_t cols, uint8_t *codes,
                                float *scales) {
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *row = v + r * cols;
        float am = 0.0f;
        for (int64_t i = 0; i < cols; ++i) am = fmaxf(am, fabsf(orc_bf16_to_f32(row[i])));
        float s = am < 1e-12f ? 1.0f : am / 448.0f;
        scales[r] = s;
        for (int64_t i = 0; i < cols; ++i)
            codes[r * cols + i] = orc_f32_to_e4m3fn(orc_bf16_to_f32(row[i]) / s);
    }
}

/* ============================== evaluator GEMM ========================================== */

/* eval.rs:1465-1507 */
void orc_matmul_2d(const float *a, const float *b, int64_t m, int64_t n, int64_t k,
                   int packed_rhs, float *out) {
    for (int64_t row = 0; row < m; ++row)
        for (int64_t col = 0; col < n; ++col) {
            float acc = 0.0f;
            for (int64_t kk = 0; kk < k; ++kk) {
                float bv = packed_rhs ? b[col * k + kk] : b[kk * n + col];
                float p = a[row * k + kk] * bv;
                acc = acc + p;
            }
            out[row * n + col] = acc;
        }
}

/* eval.rs:1733-1735 */
static float gelu_scalar(float x) {
    float inner = 0.7978846f * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

/* eval.rs:1151-1176 */
void orc_epilogue(float *out, int64_t len, const float *bias, int64_t bias_len, const float *z,
                  int64_t z_len, int mode) {
    if (mode == 0) return;
    int64_t bl = bias_len > 0 ? bias_len : 1, zl = z_len > 0 ? z_len : 1;
    for (int64_t i = 0; i < len; ++i) {
        float val = out[i] + (bias_len > 0 ? bias[i % bl] : 0.0f);
        float zz = z_len > 0 ? z[i % zl] : 0.0f;
        switch (mode) {
        case 2: val = fmaxf(val, zz); break;
        case 3: val = tanhf(val); break;
        case 4: val = val / (1.0f + expf(-val)); break;
        case 5: val = gelu_scalar(val); break;
        case 6: val = val * zz; break;
        default: break;
        }
        out[i] = val;
    }
}

static float *bf16_to_f32_buf(const uint16_t *x, int64_t len) {
    float *a = (float *)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
    for (int64_t i = 0; i < len; ++i) a[i] = orc_bf16_to_f32(x[i]);
    return a;
}

/* eval.rs:305-319 dequant ((q - zp) as f32 * scale) then eval.rs:1465-1507 packed matmul */
void orc_gemm_w8a16(const uint16_t *x, int64_t m, int64_t n, int64_t k, const int8_t *codes,
                    const float *scales, float *out) {
    float *a = bf16_to_f32_buf(x, m * k);
    float *w = (float *)malloc(sizeof(float) * (size_t)(n * k > 0 ? n * k : 1));
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) w[r * k + i] = (float)codes[r * k + i] * scales[r];
    orc_matmul_2d(a, w, m, n, k, 1, out);
    free(a); free(w);
}

void orc_gemm_w4a16(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                    const uint32_t *codes, const uint16_t *scales_f16, const uint32_t *zeros,
                    float *out) {
    float *a = bf16_to_f32_buf(x, m * k);
    float *w = (float *)malloc(sizeof(float) * (size_t)(n * k > 0 ? n * k : 1));
    orc_dequantize_int4g(codes, scales_f16, zeros, n, k, group, w);
    orc_matmul_2d(a, w, m, n, k, 1, out);
    free(a); free(w);
}

void orc_gemm_nf4(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t block,
                  const uint32_t *codes, const float *absmax, float *out) {
    float *a = bf16_to_f32_buf(x, m * k);
    float *w = (float *)malloc(sizeof(float) * (size_t)(n * k > 0 ? n * k : 1));
    orc_dequantize_nf4(codes, absmax, n, k, block, w);
    orc_matmul_2d(a, w, m, n, k, 1, out);
    free(a); free(w);
}

void orc_gemm_fp8(const uint8_t *qa, const float *sa, int64_t m, const uint8_t *qw,
                  const float *sw, int64_t n, int64_t k, float *out) {
    float *a = (float *)malloc(sizeof(float) * (size_t)(m * k > 0 ? m * k : 1));
    float *w = (float *)malloc(sizeof(float) * (size_t)(n * k > 0 ? n * k : 1));
    for (int64_t r = 0; r < m; ++r)
        for (int64_t i = 0; i < k; ++i) a[r * k + i] = orc_e4m3fn_to_f32(qa[r * k + i]) * sa[r];
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) w[r * k + i] = orc_e4m3fn_to_f32(qw[r * k + i]) * sw[r];
    orc_matmul_2d(a, w, m, n, k, 1, out);
    free(a); free(w);
}

double orc_now_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* codegen/eval.rs:1369-1382, castforge.static_quantize with its scale attribute resolved to f32
 * (> 0) and bits: qmax = bits == 4 ? 7 : 127; y = clamp(round(x / sc), -qmax, qmax) * sc with
 * Rust's round (half away from zero) and clamp (NaN passes). */
void orc_static_quantize(const float *x, int64_t n, float sc, int bits, float *y) {
    const float qmax = bits == 4 ? 7.0f : 127.0f;
    for (int64_t i = 0; i < n; ++i) y[i] = rust_clamp(roundf(x[i] / sc), -qmax, qmax) * sc;
}

/* ---- GGUF tensor payloads ---------------------------------------------------------------- */
/* gguf.rs:486-550 (decode_ggml_tensor): F32 / F16 / BF16 element arrays and the 32-element
 * blocks Q4_0 (f16 d, then 16 bytes: element 2j = low nibble of byte j, 2j+1 = high nibble,
 * value (nibble - 8) * d) and Q8_0 (f16 d, then 32 int8: value q * d).  Blocks run over the
 * flattened tensor; the last block's elements past num_elems are dropped.  Returns the payload
 * bytes read, or -1 for an unknown type. */
int64_t orc_gguf_decode(int type, const uint8_t *raw, int64_t num_elems, float *out) {
    switch (type) {
    case ORC_GGML_F32:
        for (int64_t i = 0; i < num_elems; ++i) {
            uint32_t u = (uint32_t)raw[4 * i] | ((uint32_t)raw[4 * i + 1] << 8) |
                         ((uint32_t)raw[4 * i + 2] << 16) | ((uint32_t)raw[4 * i + 3] << 24);
            out[i] = u2f(u);
        }
        return num_elems * 4;
    case ORC_GGML_F16:
    case ORC_GGML_BF16:
        for (int64_t i = 0; i < num_elems; ++i) {
            uint16_t h = (uint16_t)(raw[2 * i] | (raw[2 * i + 1] << 8));
            out[i] = type == ORC_GGML_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
        }
        return num_elems * 2;
    case ORC_GGML_Q4_0: {
        const int64_t blocks = (num_elems + 31) / 32;
        int64_t o = 0;
        for (int64_t b = 0; b < blocks; ++b) {
            const uint8_t *blk = raw + 18 * b;
            const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            for (int j = 2; j < 18; ++j) {
                if (o < num_elems) out[o++] = (float)((int32_t)(blk[j] & 0x0f) - 8) * d;
                if (o < num_elems) out[o++] = (float)((int32_t)((blk[j] >> 4) & 0x0f) - 8) * d;
            }
        }
        return blocks * 18;
    }
    case ORC_GGML_Q8_0: {
        const int64_t blocks = (num_elems + 31) / 32;
        int64_t o = 0;
        for (int64_t b = 0; b < blocks; ++b) {
            const uint8_t *blk = raw + 34 * b;
            const float d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
            for (int j = 2; j < 34; ++j)
                if (o < num_elems) out[o++] = (float)(int8_t)blk[j] * d;
        }
        return blocks * 34;
    }
    default:
        return -1;
    }
}

/* gguf.rs:283-296: a QuantizedI8 tensor (n int8 codes, one f32 scale) as Q8_0 blocks: every
 * block repeats f32_to_f16_bits(scale) (tensor_store.rs:84-102, truncating) and the codes of its
 * 32 elements, zero past n; max(n, 1) elements make ceil(max(n,1) / 32) blocks.  Returns the
 * bytes written. */
int64_t orc_gguf_encode_q8_0(const int8_t *codes, int64_t n, float scale, uint8_t *out) {
    const int64_t blocks = ((n > 1 ? n : 1) + 31) / 32;
    const uint16_t h = orc_f32_to_f16_trunc(scale);
    for (int64_t b = 0; b < blocks; ++b) {
        uint8_t *blk = out + 34 * b;
        blk[0] = (uint8_t)(h & 0xff);
        blk[1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; ++j) {
            const int64_t i = 32 * b + j;
            blk[2 + j] = (uint8_t)(i < n ? codes[i] : 0);
        }
    }
    return blocks * 34;
}

/* ---- outlier suppression ----------------------------------------------------------------- */
/* formats.rs:301-327 (RotateHadamardPass::run): w is a [k, n] constant; b =
 * next_power_of_two(block_size).min(k).max(2); when k % b == 0, every column's blocks of b
 * consecutive rows go through the butterfly stages h = 1, 2, .., b/2 (buf[j] = x + y,
 * buf[j+h] = x - y) and are written back times norm = 1 / sqrt(b); otherwise w is unchanged.
 * Returns b, or -1 when b is not a power of two (the reference's butterfly then indexes past
 * its buffer and panics). */
int64_t orc_rotate_hadamard(float *w, int64_t k, int64_t n, int64_t block_size) {
    int64_t p = 1;
    while (p < block_size) p <<= 1;
    int64_t b = p < k ? p : k;
    if (b < 2) b = 2;
    if (k % b != 0) return b;
    if ((b & (b - 1)) != 0) return -1;
    const float norm = 1.0f / sqrtf((float)b);
    float *buf = (float *)malloc(sizeof(float) * (size_t)b);
    for (int64_t col = 0; col < n; ++col) {
        for (int64_t kb = 0; kb < k; kb += b) {
            for (int64_t i = 0; i < b; ++i) buf[i] = w[(kb + i) * n + col];
            for (int64_t h = 1; h < b; h *= 2)
                for (int64_t i = 0; i < b; i += 2 * h)
                    for (int64_t j = i; j < i + h; ++j) {
                        const float x = buf[j], y = buf[j + h];
                        buf[j] = x + y;
                        buf[j + h] = x - y;
                    }
            for (int64_t i = 0; i < b; ++i) w[(kb + i) * n + col] = buf[i] * norm;
        }
    }
    free(buf);
    return b;
}

static float rust_maxf(float a, float b) { return isnan(a) ? b : (isnan(b) ? a : (a > b ? a : b)); }

/* schemes.rs:188-238 (run_smoothquant) for one constant of n elements with act_max its
 * calibrated bound (as f32): alpha clamped to [0.05, 0.95]; w_max = max over |w| (NaN
 * skipped), at least 1e-5; s = max(max(act_max, 1e-4)^alpha / w_max^(1 - alpha), 1e-4);
 * e = max(w_max * s / qmax, 1e-6); w[i] = (clamp(round(w[i] * s / e), qmin, qmax) * e) / s.
 * scales_out (may be NULL) receives s and e. */
void orc_smoothquant(float *w, int64_t n, float act_max, float alpha, int bits, float *scales_out) {
    int eff_bits;
    float qmin, qmax;
    orc_int_bounds(bits, &eff_bits, &qmin, &qmax);
    alpha = rust_clamp(alpha, 0.05f, 0.95f);
    float w_max = 0.0f;
    for (int64_t i = 0; i < n; ++i) w_max = rust_maxf(w_max, fabsf(w[i]));
    w_max = rust_maxf(w_max, 1e-5f);
    const float s = rust_maxf(powf(rust_maxf(act_max, 1e-4f), alpha) / powf(w_max, 1.0f - alpha), 1e-4f);
    const float e = rust_maxf(w_max * s / qmax, 1e-6f);
    for (int64_t i = 0; i < n; ++i) {
        const float migrated = w[i] * s;
        const float q = rust_clamp(roundf(migrated / e), qmin, qmax);
        w[i] = (q * e) / s;
    }
    if (scales_out) {
        scales_out[0] = s;
        scales_out[1] = e;
    }
}
