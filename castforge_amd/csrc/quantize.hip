// Quantize / dequantize kernels for gfx950 and their C-ABI entry points.
//
// All kernels are HBM-bound streaming passes: 16-byte loads, wave64 butterfly reductions
// for absmax/min/max, packed stores (4 int8 codes or 8 nibble codes per 32-bit store).
// The arithmetic gives the bytes of the CPU reference's f32 sequence: x / scale as the correctly
// rounded f32 quotient (hipcc's IEEE division, or div_by_scale's reciprocal and correction
// where that is shown to give the same quotient), no contraction (this file is built with
// -ffp-contract=off), round-half-even via rintf or half-away via roundf, NaN -> 0 as in Rust's
// `as i8`.
#include <algorithm>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

constexpr int kBlock = 256;  // 4 waves
#ifndef CFH_INT4Q16
#define CFH_INT4Q16 1  // 0: the 8-codes-per-thread INT4 kernel for every group size
#endif
#ifndef CFH_INT4Q16_AWQ_ROWS
#define CFH_INT4Q16_AWQ_ROWS 4  // rows per thread of the 16-codes INT4 kernel with an AWQ pre-scale
#endif

__device__ __forceinline__ float round_sel(float x, int mode) {
    return mode == CFH_ROUND_HALF_EVEN ? rintf(x) : roundf(x);
}

// RN(x / s) from y = RN(1 / s), Markstein's correction step:
//     q = fma(fma(-RN(x y), s, x), y, RN(x y)).
// The remainder fma(-q0, s, x) is exact when q0 is within an ulp of x / s and nothing over- or
// underflows, and then q is the correctly rounded quotient, bit for bit the IEEE division
// (about 10 instructions) that it replaces.  For denormal x both quotients round to codes of
// 0.  q0 is first clamped to [-lim, lim]: callers pick lim so that every |x / s| > lim gives
// the same code, and the clamp keeps the remainder finite when RN(x y) overflows (inf x still
// yields inf, NaN x NaN).  An infinite s (y = 0) gives NaN, not x / s = +-0: the callers check
// that case.  Validated on the CPU against x / s for every positive finite f16 scale (INT4
// group scales, lim 64) and for random f32 scales amax / 7, amax / 127 (both rounding modes,
// lim 256) and amax / 448 (E4M3 codes, lim 1024), with random x, exact ties and ties +- 3 ulp:
// no code differs.
__device__ __forceinline__ float div_by_scale(float x, float s, float y, float lim) {
    const float q0 = fminf(fmaxf(x * y, -lim), lim);
    return __builtin_fmaf(__builtin_fmaf(-q0, s, x), y, q0);
}

// formats.rs:676: (v / scale).round().clamp(qmin, qmax) as i8 — NaN maps to 0.
__device__ __forceinline__ uint32_t quant_sym_byte(float v, float scale, float qmin, float qmax,
                                                   int mode) {
    float r = round_sel(v / scale, mode);
    if (r != r) return 0u;
    r = fminf(fmaxf(r, qmin), qmax);
    return static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu;
}

// Same code with the quotient from div_by_scale (|qmin|, qmax <= 128, so lim 256 is safe; an
// infinite scale yields NaN -> 0, which is also the code of v / inf = +-0 and inf / inf).
__device__ __forceinline__ uint32_t quant_sym_byte_y(float v, float scale, float y, float qmin,
                                                     float qmax, int mode) {
    float r = round_sel(div_by_scale(v, scale, y, 256.0f), mode);
    if (r != r) return 0u;
    r = fminf(fmaxf(r, qmin), qmax);
    return static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xffu;
}

// Block-wide max of non-negative values (fmaxf ignores NaN like Rust's f32::max).
__device__ __forceinline__ float block_max(float v, float *red) {
    v = wave_max<64>(v);
    const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kBlock / 64; ++i) r = fmaxf(r, red[i]);
    return r;
}

// Up to kQSets matrices with the same column count, quantized by one launch: their rows are
// concatenated in launch order and each workgroup finds its matrix from its row.
constexpr int kQSets = 8;
template <class T>
struct RowSets {
    const T *src[kQSets];
    const float *in_scale[kQSets];  // INT4: AWQ per-column pre-scale, or null
    void *codes[kQSets];
    void *scales[kQSets];
    uint32_t *zeros[kQSets];        // INT4
    int64_t row_end[kQSets];        // rows of matrices 0..i
    int count;
    // matrix of launch row r, and r's row within it
    __device__ __forceinline__ int find(int64_t r, int64_t &local) const {
        int p = 0;
#pragma unroll
        for (int i = 1; i < kQSets; ++i)
            if (i < count && r >= row_end[i - 1]) p = i;
        local = r - (p > 0 ? row_end[p - 1] : 0);
        return p;
    }
};

template <class T>
RowSets<T> one_set(const T *src, const float *in_scale, void *codes, void *scales, uint32_t *zeros,
                   int64_t rows) {
    RowSets<T> s{};
    s.src[0] = src;
    s.in_scale[0] = in_scale;
    s.codes[0] = codes;
    s.scales[0] = scales;
    s.zeros[0] = zeros;
    s.row_end[0] = rows;
    s.count = 1;
    return s;
}

struct F32x4Src {
    using elem = float;
    const float *p;
    __device__ __forceinline__ float4 load4(int64_t i) const {
        return reinterpret_cast<const float4 *>(p)[i];
    }
    __device__ __forceinline__ float load1(int64_t i) const { return p[i]; }
};

struct Bf16x4Src {
    using elem = uint16_t;
    const uint16_t *p;
    __device__ __forceinline__ float4 load4(int64_t i) const {
        uint2 u = reinterpret_cast<const uint2 *>(p)[i];
        return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                           __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    }
    __device__ __forceinline__ float load1(int64_t i) const { return bf16_to_f32(p[i]); }
};

// Encoders: how one value becomes one byte, given the row's absmax.  enc() divides; enc_y()
// takes y = RN(1 / scale) and is used when fast_ok(y) says it yields the same byte.
struct SymEnc {
    float qmin, qmax;
    int mode;
    __device__ __forceinline__ float scale_of(float amax) const {
        return amax < 1e-12f ? 1.0f : amax / qmax;
    }
    __device__ __forceinline__ uint32_t enc(float v, float scale) const {
        return quant_sym_byte(v, scale, qmin, qmax, mode);
    }
    __device__ __forceinline__ bool fast_ok(float) const { return true; }
    __device__ __forceinline__ uint32_t enc_y(float v, float scale, float y) const {
        return quant_sym_byte_y(v, scale, y, qmin, qmax, mode);
    }
    __device__ __forceinline__ uint32_t enc4_y(float4 v, float scale, float y) const {
        return enc_y(v.x, scale, y) | (enc_y(v.y, scale, y) << 8) | (enc_y(v.z, scale, y) << 16) |
               (enc_y(v.w, scale, y) << 24);
    }
    static constexpr bool finite_path() { return false; }
};

// Low bytes of four i32 -> one word (byte i = value i).
__device__ __forceinline__ uint32_t pack_low_bytes(int32_t a, int32_t b, int32_t c, int32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(static_cast<uint32_t>(b), static_cast<uint32_t>(a), 0x0c0c0400u);
    const uint32_t cd = __builtin_amdgcn_perm(static_cast<uint32_t>(d), static_cast<uint32_t>(c), 0x04000c0cu);
    return ab | cd;
}

// SymEnc with the rounding mode fixed at compile time, and a path for rows that hold neither
// NaN nor an infinity (rows_quant_reg_kernel checks that from the bit patterns).  There
// amax is finite, so |v * y| <= qmax (1 + 2^-22): div_by_scale's clamp never acts, the quotient
// is never NaN and its rounding already lies in [qmin, qmax] (qmin <= -qmax - 1), so the code
// is the rounded quotient itself.
template <int MODE>
struct SymEncM : SymEnc {
    __device__ __forceinline__ float rnd(float q) const {
        return MODE == CFH_ROUND_HALF_EVEN ? rintf(q) : roundf(q);
    }
    __device__ __forceinline__ uint32_t enc(float v, float scale) const {
        return quant_sym_byte(v, scale, qmin, qmax, MODE);
    }
    __device__ __forceinline__ uint32_t enc_y(float v, float scale, float y) const {
        return quant_sym_byte_y(v, scale, y, qmin, qmax, MODE);
    }
    __device__ __forceinline__ uint32_t enc4_y(float4 v, float scale, float y) const {
        return enc_y(v.x, scale, y) | (enc_y(v.y, scale, y) << 8) | (enc_y(v.z, scale, y) << 16) |
               (enc_y(v.w, scale, y) << 24);
    }
    static constexpr bool finite_path() { return true; }
    __device__ __forceinline__ uint32_t enc4_finite(float4 v, float scale, float y) const {
        auto q = [&](float x) {
            const float q0 = x * y;
            return static_cast<int32_t>(rnd(__builtin_fmaf(__builtin_fmaf(-q0, scale, x), y, q0)));
        };
        return pack_low_bytes(q(v.x), q(v.y), q(v.z), q(v.w));
    }
};

// Calls f with e as the SymEncM of its rounding mode.
template <class F>
void with_round_mode(const SymEnc &e, F &&f) {
    if (e.mode == CFH_ROUND_HALF_EVEN) f(SymEncM<CFH_ROUND_HALF_EVEN>{e});
    else f(SymEncM<CFH_ROUND_HALF_AWAY>{e});
}

// E4M3 bytes of four values (byte i = value i).  gfx950's v_cvt_pk_fp8_f32 (OCP E4M3FN, round
// to nearest even) gives f32_to_e4m3fn's byte for every f32 except NaN (the reference's 0x7F
// for either sign), |v| >= 464 (the conversion's NaN where the reference saturates to
// 0x7E / 0xFE) and the reference's 32 log2-quirk inputs (mantissa 0x7ffffe / 0x7fffff just
// below a power of two): an exhaustive comparison over all 2^32 f32 patterns on the GPU
// found no other difference.  Lanes holding such a candidate (NaN, |v| >= 448, or a mantissa
// of 0x7ffffe / 0x7fffff) take the exact encoder; the others, nearly all, take two
// conversions instead of ~30 instructions per value.
__device__ __forceinline__ bool e4m3_special(float v) {
    const uint32_t a = __float_as_uint(v) & 0x7fffffffu;
    return a >= 0x43e00000u || (a & 0x7ffffeu) == 0x7ffffeu;
}
__device__ __forceinline__ uint32_t e4m3x4(float v0, float v1, float v2, float v3) {
    // one test of the OR of the four flags (no short-circuit branches)
    if (static_cast<int>(e4m3_special(v0)) | static_cast<int>(e4m3_special(v1)) |
        static_cast<int>(e4m3_special(v2)) | static_cast<int>(e4m3_special(v3)))
        return f32_to_e4m3fn(v0) | (f32_to_e4m3fn(v1) << 8) | (f32_to_e4m3fn(v2) << 16) |
               (static_cast<uint32_t>(f32_to_e4m3fn(v3)) << 24);
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, lo, true));
}

struct Fp8Enc {
    __device__ __forceinline__ float scale_of(float amax) const {
        return amax < 1e-12f ? 1.0f : amax / 448.0f;
    }
    __device__ __forceinline__ uint32_t enc(float v, float scale) const {
        return f32_to_e4m3fn(v / scale);
    }
    // E4M3 keeps the sign of v / inf = -0 and codes NaN as 0x7F, so an infinite scale divides.
    __device__ __forceinline__ bool fast_ok(float y) const { return y != 0.0f; }
    // div_by_scale turns -0 into +0 (the remainder fma rounds -0 + +0 to +0); scale > 0, so
    // the quotient's sign is v's, and OR-ing v's sign bit back in restores 0x80 for -0.
    __device__ __forceinline__ float quot(float v, float scale, float y) const {
        const float q = div_by_scale(v, scale, y, 1024.0f);
        return __uint_as_float(__float_as_uint(q) | (__float_as_uint(v) & 0x80000000u));
    }
    __device__ __forceinline__ uint32_t enc_y(float v, float scale, float y) const {
        return f32_to_e4m3fn(quot(v, scale, y));
    }
    __device__ __forceinline__ uint32_t enc4_y(float4 v, float scale, float y) const {
        return e4m3x4(quot(v.x, scale, y), quot(v.y, scale, y), quot(v.z, scale, y), quot(v.w, scale, y));
    }
    // Rows without NaN or infinity (amax finite): |v * y| <= 448.0001, so no clamp is needed,
    // the quotient is never NaN and stays below the conversion's NaN range (464), and only
    // the log2-quirk mantissas (0x7ffffe / 0x7fffff) need the exact encoder.  The quotient
    // q0 - (q0 * scale - v) * y is div_by_scale's with the residual's sign flipped: the same
    // magnitudes, and the sign of a zero quotient (v = -0, or a negative quotient that
    // underflows) kept without the OR that quot() needs.
    static constexpr bool finite_path() { return true; }
    __device__ __forceinline__ uint32_t enc4_finite(float4 v, float scale, float y) const {
        const float x[4] = {v.x, v.y, v.z, v.w};
        float q[4];
        uint32_t f = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float q0 = x[j] * y;
            q[j] = __builtin_fmaf(-__builtin_fmaf(q0, scale, -x[j]), y, q0);
            f = max(f, __builtin_amdgcn_ubfe(__float_as_uint(q[j]), 1, 22));
        }
        if (f == 0x3fffffu)
            return f32_to_e4m3fn(q[0]) | (f32_to_e4m3fn(q[1]) << 8) | (f32_to_e4m3fn(q[2]) << 16) |
                   (static_cast<uint32_t>(f32_to_e4m3fn(q[3])) << 24);
        return static_cast<uint32_t>(
            __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false), true));
    }
};

__device__ __forceinline__ float amax4(float a, float4 v) {
    a = fmaxf(a, fabsf(v.x));
    a = fmaxf(a, fabsf(v.y));
    a = fmaxf(a, fabsf(v.z));
    a = fmaxf(a, fabsf(v.w));
    return a;
}

// One workgroup per row; the row stays in registers (VPT float4 per thread), so HBM sees
// each input byte once.  Requires cols % 4 == 0 and 16-byte aligned rows.
template <int VPT, class Src, class Enc>
__global__ __launch_bounds__(kBlock) void rows_quant_reg_kernel(RowSets<typename Src::elem> sets,
                                                                 int64_t cols, Enc e) {
    __shared__ float red[kBlock / 64];
    int64_t row;
    const int set = sets.find(blockIdx.x, row);
    const Src src{sets.src[set]};
    uint8_t *__restrict__ codes = static_cast<uint8_t *>(sets.codes[set]);
    float *__restrict__ scales = static_cast<float *>(sets.scales[set]);
    const int64_t nv = cols >> 2;
    const int64_t base = row * nv;
    // Threads past the row's end load its last 4 values again: an index clamp rather than a
    // branch, since a load under a divergent branch gets a wait of its own and the loads would
    // run one after another.  A repeated element leaves the absmax unchanged; those threads
    // store nothing.
    float4 v[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) v[i] = src.load4(base + min(threadIdx.x + static_cast<int64_t>(i) * kBlock, nv - 1));
    uint32_t *out = reinterpret_cast<uint32_t *>(codes + row * cols);
    if constexpr (Enc::finite_path()) {
        // the largest magnitude bit pattern: below 0x7f800000 the row is finite and it is the
        // absmax itself (non-NaN floats order like their magnitude bits)
        uint32_t mb = 0;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const uint32_t a = __float_as_uint(v[i].x) & 0x7fffffffu, b = __float_as_uint(v[i].y) & 0x7fffffffu;
            const uint32_t c = __float_as_uint(v[i].z) & 0x7fffffffu, d = __float_as_uint(v[i].w) & 0x7fffffffu;
            mb = max(max(mb, max(a, b)), max(c, d));
        }
        mb = wave_umax<64>(mb);
        __syncthreads();
        if ((threadIdx.x & 63) == 0) reinterpret_cast<uint32_t *>(red)[threadIdx.x >> 6] = mb;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) mb = max(mb, reinterpret_cast<const uint32_t *>(red)[w]);
        if (mb < 0x7f800000u) {  // uniform over the workgroup (one row)
            const float scale = e.scale_of(__uint_as_float(mb));
            const float y = 1.0f / scale;
#pragma unroll
            for (int i = 0; i < VPT; ++i) {
                const int64_t idx = threadIdx.x + static_cast<int64_t>(i) * kBlock;
                const uint32_t w = e.enc4_finite(v[i], scale, y);
                if (idx < nv) out[idx] = w;
            }
            if (threadIdx.x == 0) scales[row] = scale;
            return;
        }
    }
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) am = amax4(am, v[i]);
    am = block_max(am, red);
    const float scale = e.scale_of(am);
    const float y = 1.0f / scale;
    if (e.fast_ok(y)) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int64_t idx = threadIdx.x + static_cast<int64_t>(i) * kBlock;
            if (idx < nv) out[idx] = e.enc4_y(v[i], scale, y);
        }
    } else {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int64_t idx = threadIdx.x + static_cast<int64_t>(i) * kBlock;
            if (idx < nv) {
                out[idx] = e.enc(v[i].x, scale) | (e.enc(v[i].y, scale) << 8) |
                           (e.enc(v[i].z, scale) << 16) | (e.enc(v[i].w, scale) << 24);
            }
        }
    }
    if (threadIdx.x == 0) scales[row] = scale;
}

// Per-token E4M3 of bf16 rows with cols % 8 == 0: rows_quant_reg_kernel's codes and scales
// with one 16-byte load of 8 values and one 8-byte store of 8 codes per lane and step.  TPR
// threads share a row: a workgroup of 256 threads holds 4 rows at TPR = 64 (no barrier), else
// one row over NT = TPR threads.  Each thread keeps VPT 16-byte pieces of its row in
// registers, so HBM sees each input byte once.  Threads past the row's end load its last 8
// values again (an index clamp, not a branch: a load under a divergent branch gets a wait of
// its own, and the loads would run one after another); a repeated element leaves the absmax
// unchanged, and those threads store nothing.
//
// For a row without NaN or infinity (the case this kernel is built for):
// - the absmax comes from the bit patterns: |v| of non-NaN bf16 values orders as the
//   magnitude bits, so a packed 16-bit max of (bits & 0x7fff) is the absmax's top half (a
//   result of 0x7f80 means an infinity, above it a NaN; both take the general path below);
// - amax finite gives 2.2e-15 <= scale <= 7.6e35 and y = 1 / scale normal, |v * y| <= 448.0001,
//   so div_by_scale's clamp never acts and is left out.  q0 = v * y corrected by two fmas,
//   q = q0 - (q0 * scale - v) * y, is the rounded quotient v / scale: div_by_scale's
//   residual with its sign flipped, which rounds to the same magnitudes and also keeps the
//   sign of a zero quotient (v = -0, or -tiny / scale underflowing: the last fma then adds
//   -0 to -0 or rounds a negative product, where q0 + (v - q0 * scale) * y gives +0);
// - |q| < 464, so q is never NaN and never reaches the conversion's NaN range: of the inputs
//   where v_cvt_pk_fp8_f32 differs from f32_to_e4m3fn only the log2-quirk mantissas
//   (0x7ffffe / 0x7fffff) remain, found by one unsigned max over 8 bit fields of 22 bits.
template <int VPT, int TPR, int NT>
__global__ __launch_bounds__(NT) void fp8_rows_bf16x8_kernel(const uint16_t *__restrict__ src, int64_t rows,
                                                             int64_t cols, uint8_t *__restrict__ codes,
                                                             float *__restrict__ scales) {
    static_assert(TPR % 64 == 0 && (TPR == 64 ? NT == 256 : NT == TPR), "4 one-wave rows or one row per workgroup");
    constexpr int kWavesPerRow = TPR / 64;
    __shared__ uint32_t red[kWavesPerRow];
    const int t = threadIdx.x % TPR;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (NT / TPR) + threadIdx.x / TPR;
    const bool live = row < rows;  // only a last, partial workgroup at TPR = 64 has rows past the end
    const int64_t nv = cols >> 3;
    const uint4 *p = reinterpret_cast<const uint4 *>(src + (live ? row : 0) * cols);
    uint4 u[VPT];
    static_for<VPT>([&](auto i) __attribute__((always_inline)) {
        u[i] = p[min(t + static_cast<int64_t>(i) * TPR, nv - 1)];
    });
    // row-wide max of a non-negative u32 (workgroup-uniform call: one row per workgroup when
    // the row spans several waves)
    auto row_umax = [&](uint32_t v) {
        v = wave_umax<64>(v);
        if constexpr (kWavesPerRow > 1) {
            __syncthreads();  // red[] may still be read by a previous call
            if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
            __syncthreads();
#pragma unroll
            for (int w = 0; w < kWavesPerRow; ++w) v = max(v, red[w]);
        }
        return v;
    };
    typedef unsigned short us2 __attribute__((ext_vector_type(2)));
    us2 mh = {0, 0};
    static_for<VPT>([&](auto i) __attribute__((always_inline)) {
        const uint4 w = u[i];
        mh = __builtin_elementwise_max(mh, __builtin_bit_cast(us2, w.x & 0x7fff7fffu));
        mh = __builtin_elementwise_max(mh, __builtin_bit_cast(us2, w.y & 0x7fff7fffu));
        mh = __builtin_elementwise_max(mh, __builtin_bit_cast(us2, w.z & 0x7fff7fffu));
        mh = __builtin_elementwise_max(mh, __builtin_bit_cast(us2, w.w & 0x7fff7fffu));
    });
    const uint32_t mx = mh.x, my = mh.y;
    const uint32_t mbits = row_umax(mx > my ? mx : my);
    auto lo4 = [](const uint4 &w) {
        return make_float4(__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                           __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u));
    };
    auto hi4 = [](const uint4 &w) {
        return make_float4(__uint_as_float(w.z << 16), __uint_as_float(w.z & 0xffff0000u),
                           __uint_as_float(w.w << 16), __uint_as_float(w.w & 0xffff0000u));
    };
    uint2 *out = reinterpret_cast<uint2 *>(codes + (live ? row : 0) * cols);
    const Fp8Enc e{};
    if (mbits < 0x7f80u) {
        const float scale = e.scale_of(__uint_as_float(mbits << 16));
        const float y = 1.0f / scale;
        static_for<VPT>([&](auto i) __attribute__((always_inline)) {
            const uint4 w = u[i];
            const uint32_t b[8] = {w.x << 16, w.x & 0xffff0000u, w.y << 16, w.y & 0xffff0000u,
                                   w.z << 16, w.z & 0xffff0000u, w.w << 16, w.w & 0xffff0000u};
            float q[8];
            uint32_t f = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = __uint_as_float(b[j]);
                const float q0 = v * y;
                q[j] = __builtin_fmaf(-__builtin_fmaf(q0, scale, -v), y, q0);
                f = max(f, __builtin_amdgcn_ubfe(__float_as_uint(q[j]), 1, 22));
            }
            uint32_t c0, c1;
            if (f == 0x3fffffu) {
                c0 = f32_to_e4m3fn(q[0]) | (f32_to_e4m3fn(q[1]) << 8) | (f32_to_e4m3fn(q[2]) << 16) |
                     (static_cast<uint32_t>(f32_to_e4m3fn(q[3])) << 24);
                c1 = f32_to_e4m3fn(q[4]) | (f32_to_e4m3fn(q[5]) << 8) | (f32_to_e4m3fn(q[6]) << 16) |
                     (static_cast<uint32_t>(f32_to_e4m3fn(q[7])) << 24);
            } else {
                c0 = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(
                    q[2], q[3], __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false), true));
                c1 = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(
                    q[6], q[7], __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false), true));
            }
            const int64_t idx = t + static_cast<int64_t>(i) * TPR;
            if (live && idx < nv) out[idx] = make_uint2(c0, c1);
        });
        if (live && t == 0) scales[row] = scale;
        return;
    }
    // A NaN or an infinity in the row (uniform over the workgroup when it spans several waves):
    // the absmax of the values (fmaxf drops NaN) and the per-value special handling.
    float am = 0.0f;
    static_for<VPT>([&](auto i) __attribute__((always_inline)) { am = amax4(amax4(am, lo4(u[i])), hi4(u[i])); });
    am = __uint_as_float(row_umax(__float_as_uint(am)));  // non-negative, non-NaN: orders as u32
    const float scale = e.scale_of(am);
    const float y = 1.0f / scale;
    if (!live) return;
    if (e.fast_ok(y)) {
        static_for<VPT>([&](auto i) __attribute__((always_inline)) {
            const int64_t idx = t + static_cast<int64_t>(i) * TPR;
            if (idx < nv) out[idx] = make_uint2(e.enc4_y(lo4(u[i]), scale, y), e.enc4_y(hi4(u[i]), scale, y));
        });
    } else {
        auto enc4 = [&](const float4 &v) {
            return e.enc(v.x, scale) | (e.enc(v.y, scale) << 8) | (e.enc(v.z, scale) << 16) | (e.enc(v.w, scale) << 24);
        };
        static_for<VPT>([&](auto i) __attribute__((always_inline)) {
            const int64_t idx = t + static_cast<int64_t>(i) * TPR;
            if (idx < nv) out[idx] = make_uint2(enc4(lo4(u[i])), enc4(hi4(u[i])));
        });
    }
    if (t == 0) scales[row] = scale;
}

// Any row length / alignment: two passes over the row (the second pass hits L2/MALL).
template <class Src, class Enc>
__global__ __launch_bounds__(kBlock) void rows_quant_generic_kernel(Src src, int64_t cols, Enc e,
                                                                     uint8_t *__restrict__ codes,
                                                                     float *__restrict__ scales) {
    __shared__ float red[kBlock / 64];
    const int64_t row = blockIdx.x;
    const int64_t base = row * cols;
    float am = 0.0f;
    for (int64_t i = threadIdx.x; i < cols; i += kBlock) am = fmaxf(am, fabsf(src.load1(base + i)));
    am = block_max(am, red);
    const float scale = e.scale_of(am);
    for (int64_t i = threadIdx.x; i < cols; i += kBlock)
        codes[base + i] = static_cast<uint8_t>(e.enc(src.load1(base + i), scale));
    if (threadIdx.x == 0) scales[row] = scale;
}

// The register kernel over a set of matrices (cols % 4 == 0, every row 16-byte aligned).
template <class Src, class Enc>
void launch_rows_quant_sets(const RowSets<typename Src::elem> &sets, int64_t rows, int64_t cols,
                            Enc e, hipStream_t st) {
    if (rows == 0) return;
    require(rows <= 0x7fffffff, "too many rows for one launch");
    const int64_t nv = cols / 4;
    require(nv >= 1 && nv <= 16 * kBlock, "row length outside the register kernel's range");
    dim3 grid(static_cast<unsigned>(rows)), block(kBlock);
    if (nv <= 1 * kBlock)
        rows_quant_reg_kernel<1, Src><<<grid, block, 0, st>>>(sets, cols, e);
    else if (nv <= 2 * kBlock)
        rows_quant_reg_kernel<2, Src><<<grid, block, 0, st>>>(sets, cols, e);
    else if (nv <= 4 * kBlock)
        rows_quant_reg_kernel<4, Src><<<grid, block, 0, st>>>(sets, cols, e);
    else if (nv <= 8 * kBlock)
        rows_quant_reg_kernel<8, Src><<<grid, block, 0, st>>>(sets, cols, e);
    else if (nv <= 12 * kBlock)
        rows_quant_reg_kernel<12, Src><<<grid, block, 0, st>>>(sets, cols, e);
    else
        rows_quant_reg_kernel<16, Src><<<grid, block, 0, st>>>(sets, cols, e);
    check_launch("rows_quant");
}

template <class Src, class Enc>
void launch_rows_quant(Src src, bool vec_ok, int64_t rows, int64_t cols, Enc e, uint8_t *codes,
                       float *scales, hipStream_t st) {
    if (rows == 0) return;
    require(rows <= 0x7fffffff, "too many rows for one launch");
    if (vec_ok && cols >= 4 && cols / 4 <= 16 * kBlock) {
        launch_rows_quant_sets<Src>(one_set(src.p, nullptr, codes, scales, nullptr, rows), rows, cols, e, st);
        return;
    }
    dim3 grid(static_cast<unsigned>(rows)), block(kBlock);
    rows_quant_generic_kernel<<<grid, block, 0, st>>>(src, cols, e, codes, scales);
    check_launch("rows_quant");
}

// ---- per-tensor (reference QuantizeWeightsPass) -----------------------------------------
// The absmax accumulates into scales[0] viewed as a u32 (non-negative floats order like
// their bit patterns); the quantize kernel derives the scale from it; a last one-thread
// kernel replaces the absmax by the scale.
__global__ void fill_u32_kernel(uint32_t *p, uint32_t v) { *p = v; }

__global__ __launch_bounds__(kBlock) void tensor_absmax_kernel(const float *__restrict__ src,
                                                               int64_t n, uint32_t *acc) {
    __shared__ float red[kBlock / 64];
    float am = 0.0f;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
        const int64_t nv = n >> 2;
        for (int64_t i = t; i < nv; i += stride)
            am = amax4(am, reinterpret_cast<const float4 *>(src)[i]);
        for (int64_t i = (nv << 2) + t; i < n; i += stride) am = fmaxf(am, fabsf(src[i]));
    } else {
        for (int64_t i = t; i < n; i += stride) am = fmaxf(am, fabsf(src[i]));
    }
    am = block_max(am, red);
    if (threadIdx.x == 0) atomicMax(acc, __float_as_uint(am));
}

__global__ __launch_bounds__(kBlock) void tensor_quant_kernel(const float *__restrict__ src,
                                                              int64_t n, SymEnc e,
                                                              const uint32_t *acc,
                                                              uint8_t *__restrict__ codes) {
    const float scale = e.scale_of(__uint_as_float(*acc));
    const float y = 1.0f / scale;  // SymEnc: enc_y is exact for every scale
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const bool vec = ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) &&
                     ((reinterpret_cast<uintptr_t>(codes) & 3u) == 0);
    int64_t done = 0;
    if (vec) {
        const int64_t nv = n >> 2;
        for (int64_t i = t; i < nv; i += stride) {
            float4 v = reinterpret_cast<const float4 *>(src)[i];
            reinterpret_cast<uint32_t *>(codes)[i] =
                e.enc_y(v.x, scale, y) | (e.enc_y(v.y, scale, y) << 8) |
                (e.enc_y(v.z, scale, y) << 16) | (e.enc_y(v.w, scale, y) << 24);
        }
        done = nv << 2;
    }
    for (int64_t i = done + t; i < n; i += stride)
        codes[i] = static_cast<uint8_t>(e.enc_y(src[i], scale, y));
}

__global__ void tensor_scale_finalize_kernel(float *scales, SymEnc e) {
    scales[0] = e.scale_of(scales[0]);
}

int grid_for(int64_t items, int per_block, int cap) {
    int64_t g = (items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return static_cast<int>(g);
}

// ---- INT4 asymmetric group-wise ------------------------------------------------------------
// A task is (row, zero-word) = up to 8 groups; each thread owns one code word (8 elements),
// so a task has GROUP threads and a group has GROUP/8 adjacent lanes.
__device__ __forceinline__ uint16_t int4_scale_bits(float mx, float mn) {
    const float range = mx - mn;
    uint16_t h = range >= 1e-12f ? f32_to_f16_rne(range / 15.0f) : static_cast<uint16_t>(0x3C00);
    if (h == 0) h = 0x0001;
    if (h == 0x7C00) h = 0x7BFF;
    return h;
}

// in_scale (optional, f32 [cols]): AWQ-style per-input-channel pre-scale, w' = f32(w * s[k])
// is what gets quantized (one rounding, as the oracle computes it).
template <int GROUP>
__global__ __launch_bounds__(kBlock) void int4g_quant_kernel(const float *__restrict__ src,
                                                             const float *__restrict__ in_scale,
                                                             int64_t rows, int64_t cols,
                                                             uint32_t *__restrict__ codes,
                                                             uint16_t *__restrict__ scales,
                                                             uint32_t *__restrict__ zeros) {
    constexpr int T = GROUP;          // threads per task
    constexpr int TPB = kBlock / T;   // tasks per block
    constexpr int TPG = GROUP / 8;    // threads per group
    __shared__ uint32_t zpart[kBlock / 64];
    const int64_t KW = cols >> 3, G = (cols + GROUP - 1) / GROUP, ZW = (G + 7) >> 3, GP = ZW * 8;
    const int64_t task = static_cast<int64_t>(blockIdx.x) * TPB + threadIdx.x / T;
    const int t = threadIdx.x % T;
    const int64_t row = task / ZW, zw = task - row * ZW;
    const bool task_ok = row < rows;
    const int64_t w = zw * T + t;
    const bool ok = task_ok && w < KW;
    float x[8];
    float mx = -INFINITY, mn = INFINITY;
    if (ok) {
        const float4 *p = reinterpret_cast<const float4 *>(src + row * cols + w * 8);
        float4 a = p[0], b = p[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        if (in_scale) {
            const float4 *q = reinterpret_cast<const float4 *>(in_scale + w * 8);
            const float4 c = q[0], d = q[1];
            x[0] *= c.x; x[1] *= c.y; x[2] *= c.z; x[3] *= c.w;
            x[4] *= d.x; x[5] *= d.y; x[6] *= d.z; x[7] *= d.w;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) { mx = fmaxf(mx, x[i]); mn = fminf(mn, x[i]); }
    }
    mx = wave_max<TPG>(mx);
    mn = wave_min<TPG>(mn);
    const uint16_t h = int4_scale_bits(mx, mn);
    const float s = f16_to_f32(h);
    float zf = rintf(-mn / s);
    if (zf != zf) zf = 0.0f;
    zf = fminf(fmaxf(zf, 0.0f), 15.0f);
    const int gi = t / TPG;  // group within the task
    uint32_t zn = 0;
    if (ok) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float r = rintf(x[i] / s);
            if (r != r) r = 0.0f;
            const float qf = fminf(fmaxf(r + zf, 0.0f), 15.0f);
            word |= static_cast<uint32_t>(qf) << (4 * i);
        }
        codes[row * KW + w] = word;
        if (t % TPG == 0) {
            scales[row * GP + zw * 8 + gi] = h;
            zn = static_cast<uint32_t>(zf) << (4 * gi);
        }
    }
    // pad scale slots of the last 8-group block (no valid thread) are written as 0
    if (task_ok && !ok && t % TPG == 0 && zw * 8 + gi >= G) scales[row * GP + zw * 8 + gi] = 0;
    if constexpr (T <= 64) {
        zn = wave_or<T>(zn);
        if (t == 0 && task_ok) zeros[row * ZW + zw] = zn;
    } else {
        zn = wave_or<64>(zn);
        if ((threadIdx.x & 63) == 0) zpart[threadIdx.x >> 6] = zn;
        __syncthreads();
        if (t == 0 && task_ok) {
            uint32_t z = 0;
            const int w0 = (threadIdx.x >> 6);
#pragma unroll
            for (int i = 0; i < T / 64; ++i) z |= zpart[w0 + i];
            zeros[row * ZW + zw] = z;
        }
    }
}

// ---- INT4 group-wise, 16 codes per thread (groups of 16 .. 256) ----------------------------
// Same results as int4g_quant_kernel, with three changes that cut the VALU work per code from
// about 50 instructions to about 10:
//   * x / s (an IEEE division, ~10 instructions) becomes div_by_scale's correction step with
//     y = RN(1 / s) computed once per group by the IEEE division, and lim 64: beyond
//     |x / s| = 64 every quotient gives the same clamped code.
//   * each thread holds 16 consecutive values (two code words), so the per-group work (min /
//     max, scale, zero point) is shared by twice the codes;
//   * min / max over a group's lanes use DPP row permutations instead of LDS shuffles, and for
//     group 128 one wave covers the 8 groups of a zero-point word.
template <int TPG>
__device__ __forceinline__ float group_reduce_max(float v) {
    if constexpr (TPG >= 2) v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    if constexpr (TPG >= 4) v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    if constexpr (TPG >= 8) v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
    if constexpr (TPG >= 16) v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
    static_assert(TPG <= 16, "a group spans at most one 16-lane DPP row");
    return v;
}
template <int TPG>
__device__ __forceinline__ float group_reduce_min(float v) {
    if constexpr (TPG >= 2) v = fminf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
    if constexpr (TPG >= 4) v = fminf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
    if constexpr (TPG >= 8) v = fminf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
    if constexpr (TPG >= 16) v = fminf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
    return v;
}

// Walsh-Hadamard rotation of the values of blocks of rot_b consecutive elements of a row, as
// rotate-hadamard computes it (formats.rs:303-327: butterfly stages h = 1, 2, .., rot_b/2 in
// order, then times norm): stages h < 16 inside a lane's 16 values, stages 16 <= h < rot_b
// (<= 1024) against lane ^ (h / 16), the lower lane keeping x + y and the upper x - y.  The
// lanes of a wave hold 1024 consecutive elements of one row, so every block lies in one wave.
__device__ __forceinline__ void hadamard16_lanes(float (&x)[16], int rot_b, float norm) {
    // stages as compile-time constants, so x stays in registers (no dynamic index)
    static_for<4>([&](auto S) {
        constexpr int h = 1 << decltype(S)::value;
        if (h < rot_b) {
#pragma unroll
            for (int i = 0; i < 16; i += 2 * h)
#pragma unroll
                for (int j = i; j < i + h; ++j) {
                    const float a = x[j], b = x[j + h];
                    x[j] = a + b;
                    x[j + h] = a - b;
                }
        }
    });
    lane_butterflies<16>(x, rot_b >> 4);  // stages h = 16 .. rot_b / 2 (wave-uniform)
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] *= norm;
}

// One cross-lane stage in the hsub16 layout: the partner's value (DPP control CTRL) times
// c = +1 on the lane whose sub-block has the stage's bit clear, -1 on the other, plus the
// lane's own value.
#ifndef CFH_HSTAGE_ASM
#define CFH_HSTAGE_ASM 1
#endif
// One v_fmac_f32 per value with the partner read through DPP (x = partner * c + x, the same
// fused multiply-add as fmaf): the compiler's DPP combine does not fold a DPP move into an
// fmac, whose accumulator is tied to its result, and would spend two instructions.  s_nop 1
// gives the two wait states a DPP read needs after a VALU write of its source; inside the
// block each value's source was written 16 instructions before.  CTL: the DPP control.
#define CFH_HS(i, CTL) "v_fmac_f32_dpp %" #i ", %" #i ", %16 " CTL " row_mask:0xf bank_mask:0xf\n"
#define CFH_HSTAGE_BLOCK(CTL)                                                                          \
    asm volatile("s_nop 1\n" CFH_HS(0, CTL) CFH_HS(1, CTL) CFH_HS(2, CTL) CFH_HS(3, CTL) CFH_HS(4, CTL)      \
                 CFH_HS(5, CTL) CFH_HS(6, CTL) CFH_HS(7, CTL) CFH_HS(8, CTL) CFH_HS(9, CTL) CFH_HS(10, CTL)   \
                 CFH_HS(11, CTL) CFH_HS(12, CTL) CFH_HS(13, CTL) CFH_HS(14, CTL) CFH_HS(15, CTL)            \
                 : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]),    \
                   "+v"(x[7]), "+v"(x[8]), "+v"(x[9]), "+v"(x[10]), "+v"(x[11]), "+v"(x[12]), "+v"(x[13]), \
                   "+v"(x[14]), "+v"(x[15])                                                             \
                 : "v"(c))
template <int CTRL>
__device__ __forceinline__ void hstage16(float (&x)[16], float c) {
    static_assert(CTRL == 0xB1 || CTRL == 0x4E || CTRL == 0x141 || CTRL == 0x128, "DPP control");
#if CFH_HSTAGE_ASM
    if constexpr (CTRL == 0xB1) CFH_HSTAGE_BLOCK("quad_perm:[1,0,3,2]");
    else if constexpr (CTRL == 0x4E) CFH_HSTAGE_BLOCK("quad_perm:[2,3,0,1]");
    else if constexpr (CTRL == 0x141) CFH_HSTAGE_BLOCK("row_half_mirror");
    else CFH_HSTAGE_BLOCK("row_ror:8");
#else
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float p = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x[i]), CTRL, 0xF, 0xF, false));
        x[i] = __builtin_fmaf(p, c, x[i]);
    }
#endif
}

// hadamard16_lanes for blocks of 32 .. 256 values in the hsub16 layout (thread t holds
// sub-block hsub16(t)).  A cross-lane stage is one fma per value: on the lane that keeps the
// sum it is the reference's x + y, on its partner it is y - x = -(x - y), and that value
// carries the opposite sign from then on (the next stages add and subtract it with the same
// rule, so the signs compose).  Every value ends as (-1)^(number of stages its lane took the
// difference on) times the reference's, and the final multiply by that sign times norm
// restores it.  Products by +-1 are exact, so each value is rounded once per stage as in the
// reference; only the sign of an exact zero or of a NaN can differ, and no INT4 code depends
// on either.
__device__ __forceinline__ void hadamard16_lanes_fast(float (&x)[16], int rot_b, float norm, int t) {
#pragma unroll
    for (int h = 1; h < 16; h *= 2) {
#pragma unroll
        for (int i = 0; i < 16; i += 2 * h)
#pragma unroll
            for (int j = i; j < i + h; ++j) {
                const float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
    }
    const int sb = hsub16(t) & 15 & ((rot_b >> 4) - 1);  // the sub-block bits the stages use
    hstage16<0xB1>(x, (sb & 1) ? -1.0f : 1.0f);                      // h = 16: lane ^ 1
    if (rot_b >= 64) hstage16<0x4E>(x, (sb & 2) ? -1.0f : 1.0f);     // h = 32: lane ^ 2
    if (rot_b >= 128) hstage16<0x141>(x, (sb & 4) ? -1.0f : 1.0f);   // h = 64: lane ^ 7
    if (rot_b >= 256) hstage16<0x128>(x, (sb & 8) ? -1.0f : 1.0f);   // h = 128: lane ^ 8
    const float f = (__builtin_popcount(static_cast<unsigned>(sb)) & 1) ? -norm : norm;
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] *= f;
}

// One row's group scales, codes and zero words from each thread's 16 values x (pre-scaled and
// rotated already): min/max over the group's lanes, f16 scale, codes x / s + z packed 8 per word.
template <int GROUP>
__device__ __forceinline__ void int4g16_row(float (&x)[16], int64_t row, int par, uint32_t *__restrict__ rcodes,
                                            uint16_t *__restrict__ rscales, uint32_t *__restrict__ zeros, uint32_t G,
                                            uint32_t ZW, uint32_t zw, int t, bool task_ok, uint32_t w0, bool ok0,
                                            bool ok1, uint32_t (&zpart)[2][kBlock / 64]) {
    constexpr int TPG = GROUP / 16;  // threads per group
    constexpr int T = 8 * TPG;       // threads per task
    float mx = -INFINITY, mn = INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (h == 0 ? ok0 : ok1) {
#pragma unroll
            for (int i = 0; i < 8; ++i) { mx = fmaxf(mx, x[8 * h + i]); mn = fminf(mn, x[8 * h + i]); }
        }
    }
    mx = group_reduce_max<TPG>(mx);
    mn = group_reduce_min<TPG>(mn);
    const uint16_t hs = int4_scale_bits(mx, mn);
    const float s = f16_to_f32(hs);
    float zf = rintf(-mn / s);
    if (zf != zf) zf = 0.0f;
    zf = fminf(fmaxf(zf, 0.0f), 15.0f);
    const float y = 1.0f / s;
    const int gi = t / TPG;  // group within the task
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (h == 0 ? ok0 : ok1) {
            uint32_t word = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float r = rintf(div_by_scale(x[8 * h + i], s, y, 64.0f));
                if (r != r) r = 0.0f;
                const float qf = fminf(fmaxf(r + zf, 0.0f), 15.0f);
                word |= static_cast<uint32_t>(qf) << (4 * i);
            }
            rcodes[w0 + h] = word;
        }
    }
    uint32_t zn = 0;
    if (t % TPG == 0) {
        if (ok0) {
            rscales[zw * 8 + gi] = hs;
            zn = static_cast<uint32_t>(zf) << (4 * gi);
        } else if (task_ok && zw * 8 + gi >= G) {
            rscales[zw * 8 + gi] = 0;  // pad scale slots of the last 8-group block
        }
    }
    if constexpr (T <= 64) {
        zn = wave_or<T>(zn);
        if (t == 0 && task_ok) zeros[row * ZW + zw] = zn;
    } else {
        // alternate buffers: a row's readers finish before the barrier of the next row,
        // which comes before the row after it overwrites their buffer
        uint32_t *zp = zpart[par];
        zn = wave_or<64>(zn);
        if ((threadIdx.x & 63) == 0) zp[threadIdx.x >> 6] = zn;
        __syncthreads();
        if (t == 0 && task_ok) {
            uint32_t z = 0;
            const int w0i = (threadIdx.x >> 6);
#pragma unroll
            for (int i = 0; i < T / 64; ++i) z |= zp[w0i + i];
            zeros[row * ZW + zw] = z;
        }
    }
}

// R rows per grid row (R > 1 when every matrix of the launch has a multiple of R rows): the
// AWQ pre-scale of the thread's 16 columns is loaded once and serves all R rows.
template <int GROUP, int R>
__global__ __launch_bounds__(kBlock) void int4g_quant16_kernel(RowSets<float> sets, int64_t cols, int rot_b,
                                                               float rot_norm) {
    constexpr int TPG = GROUP / 16;   // threads per group
    constexpr int T = 8 * TPG;        // threads per task (8 groups: one zero-point word)
    constexpr int TPB = kBlock / T;   // tasks per block
    __shared__ uint32_t zpart[2][kBlock / 64];
    // R rows of one matrix per grid row: the rows' bases are uniform and every offset below
    // is 32-bit
    int64_t row0;
    const int set = sets.find(static_cast<int64_t>(blockIdx.y) * R, row0);
    const float *__restrict__ src = sets.src[set];
    const float *__restrict__ in_scale = sets.in_scale[set];
    uint32_t *__restrict__ codes = static_cast<uint32_t *>(sets.codes[set]);
    uint16_t *__restrict__ scales = static_cast<uint16_t *>(sets.scales[set]);
    uint32_t *__restrict__ zeros = sets.zeros[set];
    const uint32_t KW = static_cast<uint32_t>(cols >> 3);
    const uint32_t G = static_cast<uint32_t>((cols + GROUP - 1) / GROUP), ZW = (G + 7) >> 3, GP = ZW * 8;
    const uint32_t zw = blockIdx.x * TPB + threadIdx.x / T;  // zero-point word (task) in the row
    // the task's sub-block this thread holds: its own index, or hsub16 of it for the one-fma
    // Hadamard stages (which keeps every group on the same lanes: hsub16 only swaps sub-blocks
    // within aligned runs of 8, and within runs of 2 and 4 it maps runs onto runs)
    const bool fast_rot = rot_b >= 32 && rot_b <= 256;  // uniform
    const int t = fast_rot ? hsub16(static_cast<int>(threadIdx.x % T)) : static_cast<int>(threadIdx.x % T);
    const bool task_ok = zw < ZW;
    const uint32_t w0 = zw * (2 * T) + 2 * t;  // this thread's first code word
    const bool ok0 = task_ok && w0 < KW, ok1 = task_ok && w0 + 1 < KW;
    // the thread's 16 AWQ pre-scales (1 outside the row): loaded once, after the rows' own
    // loads, so that those are all issued before anything waits
    float sc[16];
    auto load_scales = [&]() {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool okh = h == 0 ? ok0 : ok1;
            const float4 *q = reinterpret_cast<const float4 *>(in_scale + (okh ? w0 + h : 0u) * 8);
            const float4 c = q[0], d = q[1];
            float *ss = sc + 8 * h;
            ss[0] = okh ? c.x : 1.0f; ss[1] = okh ? c.y : 1.0f; ss[2] = okh ? c.z : 1.0f; ss[3] = okh ? c.w : 1.0f;
            ss[4] = okh ? d.x : 1.0f; ss[5] = okh ? d.y : 1.0f; ss[6] = okh ? d.z : 1.0f; ss[7] = okh ? d.w : 1.0f;
        }
    };
    // every row's values are loaded before the first row is processed, so the R rows' loads
    // are in flight together (the loop below stores between rows, and loads are not moved
    // across those stores)
    float xr[R][16];
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        const float *rsrc = src + (row0 + rr) * cols;
        // a part past the row's end reads the row's first word and is zeroed: unconditional
        // loads (a load under a divergent branch gets a wait of its own before the next one
        // is issued); every launch has cols >= 8, so word 0 exists
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool okh = h == 0 ? ok0 : ok1;
            const float4 *p = reinterpret_cast<const float4 *>(rsrc + (okh ? w0 + h : 0u) * 8);
            const float4 a = p[0], b = p[1];
            float *xx = xr[rr] + 8 * h;
            xx[0] = okh ? a.x : 0.0f; xx[1] = okh ? a.y : 0.0f; xx[2] = okh ? a.z : 0.0f; xx[3] = okh ? a.w : 0.0f;
            xx[4] = okh ? b.x : 0.0f; xx[5] = okh ? b.y : 0.0f; xx[6] = okh ? b.z : 0.0f; xx[7] = okh ? b.w : 0.0f;
        }
    }
    if (in_scale) load_scales();  // uniform; after the rows' loads, which it would otherwise wait for
#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
        const int64_t row = row0 + rr;
        uint32_t *rcodes = codes + row * KW;
        uint16_t *rscales = scales + row * GP;
        float (&x)[16] = xr[rr];
        if (in_scale) {  // uniform
#pragma unroll
            for (int i = 0; i < 16; ++i) x[i] *= sc[i];  // 0 * 1 outside the row
        }
        if (fast_rot) hadamard16_lanes_fast(x, rot_b, rot_norm, static_cast<int>(threadIdx.x));  // uniform
        else if (rot_b > 1) hadamard16_lanes(x, rot_b, rot_norm);  // uniform: every lane takes part
        int4g16_row<GROUP>(x, row, rr & 1, rcodes, rscales, zeros, G, ZW, zw, t, task_ok, w0, ok0, ok1, zpart);
    }
}

// ---- NF4 block-wise ------------------------------------------------------------------------
__constant__ float kNf4Table[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

// code = #{i : x > 0.5f*(T[i]+T[i+1])}; NaN -> 7.  The midpoints are exact f32 constants.
__device__ __forceinline__ uint32_t nf4_code(float x) {
    if (x != x) return 7u;
    constexpr float m0 = 0.5f * (-1.0f + -0.6961928009986877f);
    constexpr float m1 = 0.5f * (-0.6961928009986877f + -0.5250730514526367f);
    constexpr float m2 = 0.5f * (-0.5250730514526367f + -0.39491748809814453f);
    constexpr float m3 = 0.5f * (-0.39491748809814453f + -0.28444138169288635f);
    constexpr float m4 = 0.5f * (-0.28444138169288635f + -0.18477343022823334f);
    constexpr float m5 = 0.5f * (-0.18477343022823334f + -0.09105003625154495f);
    constexpr float m6 = 0.5f * (-0.09105003625154495f + 0.0f);
    constexpr float m7 = 0.5f * (0.0f + 0.07958029955625534f);
    constexpr float m8 = 0.5f * (0.07958029955625534f + 0.16093020141124725f);
    constexpr float m9 = 0.5f * (0.16093020141124725f + 0.24611230194568634f);
    constexpr float m10 = 0.5f * (0.24611230194568634f + 0.33791524171829224f);
    constexpr float m11 = 0.5f * (0.33791524171829224f + 0.44070982933044434f);
    constexpr float m12 = 0.5f * (0.44070982933044434f + 0.5626170039176941f);
    constexpr float m13 = 0.5f * (0.5626170039176941f + 0.7229568362236023f);
    constexpr float m14 = 0.5f * (0.7229568362236023f + 1.0f);
    uint32_t c = (x > m0) + (x > m1) + (x > m2) + (x > m3) + (x > m4) + (x > m5) + (x > m6) +
                 (x > m7) + (x > m8) + (x > m9) + (x > m10) + (x > m11) + (x > m12) + (x > m13) +
                 (x > m14);
    return c;
}

template <int BLOCK>
__global__ __launch_bounds__(kBlock) void nf4_quant_kernel(const float *__restrict__ src,
                                                           int64_t rows, int64_t cols,
                                                           uint32_t *__restrict__ codes,
                                                           float *__restrict__ absmax) {
    constexpr int TPG = BLOCK / 8;  // threads per quantization block
    const int64_t KW = cols >> 3, B = (cols + BLOCK - 1) / BLOCK, KWp = B * TPG;
    const int64_t gt = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t row = gt / KWp, w = gt - row * KWp;
    const bool ok = row < rows && w < KW;
    float x[8];
    float am = 0.0f;
    if (ok) {
        const float4 *p = reinterpret_cast<const float4 *>(src + row * cols + w * 8);
        float4 a = p[0], b = p[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
#pragma unroll
        for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(x[i]));
    }
    am = wave_max<TPG>(am);
    const float st = am < 1e-12f ? 1.0f : am;
    if (ok) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) word |= nf4_code(x[i] / st) << (4 * i);
        codes[row * KW + w] = word;
        if (w % TPG == 0) absmax[row * B + w / TPG] = st;
    }
}

// ---- dequantize (TensorStore::resolve_f32_attr for the packed backings) -------------------
__global__ void dequant_int8_kernel(const int8_t *__restrict__ q, const float *__restrict__ scales,
                                    int64_t rows, int64_t cols, int per_row,
                                    float *__restrict__ out) {
    const int64_t n = rows * cols;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float s = per_row ? scales[i / cols] : scales[0];
        out[i] = static_cast<float>(static_cast<int32_t>(q[i])) * s;
    }
}

__global__ void dequant_int4g_kernel(const uint32_t *__restrict__ codes,
                                     const uint16_t *__restrict__ scales,
                                     const uint32_t *__restrict__ zeros, int64_t rows, int64_t cols,
                                     int64_t group, float *__restrict__ out) {
    const int64_t KW = cols >> 3, G = (cols + group - 1) / group, ZW = (G + 7) >> 3, GP = ZW * 8;
    const int64_t nw = rows * KW;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nw; i += stride) {
        const int64_t r = i / KW, w = i - r * KW;
        const uint32_t word = codes[i];
        for (int j = 0; j < 8; ++j) {
            const int64_t k = w * 8 + j, g = k / group;
            const int32_t z = static_cast<int32_t>((zeros[r * ZW + (g >> 3)] >> (4 * (g & 7))) & 15u);
            const int32_t q = static_cast<int32_t>((word >> (4 * j)) & 15u);
            out[r * cols + k] = static_cast<float>(q - z) * f16_to_f32(scales[r * GP + g]);
        }
    }
}

__global__ void dequant_nf4_kernel(const uint32_t *__restrict__ codes,
                                   const float *__restrict__ absmax, int64_t rows, int64_t cols,
                                   int64_t block, float *__restrict__ out) {
    const int64_t KW = cols >> 3, B = (cols + block - 1) / block;
    const int64_t nw = rows * KW;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nw; i += stride) {
        const int64_t r = i / KW, w = i - r * KW;
        const uint32_t word = codes[i];
        for (int j = 0; j < 8; ++j) {
            const int64_t k = w * 8 + j;
            out[r * cols + k] = kNf4Table[(word >> (4 * j)) & 15u] * absmax[r * B + k / block];
        }
    }
}

__global__ void dequant_fp8_kernel(const uint8_t *__restrict__ q, const float *__restrict__ scales,
                                   int64_t rows, int64_t cols, float *__restrict__ out) {
    const int64_t n = rows * cols;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = e4m3fn_to_f32(q[i]) * scales[i / cols];
}

constexpr int kGridCap = 256 * 64;

bool pow2_in(int64_t v, int64_t lo, int64_t hi) {
    return v >= lo && v <= hi && (v & (v - 1)) == 0;
}

void check_shape(int64_t rows, int64_t cols) {
    require(rows >= 0 && cols >= 0, "rows and cols must be non-negative");
    require(cols == 0 || rows <= INT64_MAX / cols, "rows * cols overflows");
}

}  // namespace
}  // namespace cfh

using namespace cfh;

extern "C" {

int32_t castforge_hip_quantize_int8(const float *src, int64_t rows, int64_t cols, int32_t bits,
                                    int32_t granularity, int32_t round_mode, int8_t *codes,
                                    float *scales, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        check_shape(rows, cols);
        require(granularity == CFH_GRAN_TENSOR || granularity == CFH_GRAN_CHANNEL,
                "granularity must be CFH_GRAN_TENSOR or CFH_GRAN_CHANNEL");
        require(round_mode == CFH_ROUND_HALF_AWAY || round_mode == CFH_ROUND_HALF_EVEN,
                "round_mode must be CFH_ROUND_HALF_AWAY or CFH_ROUND_HALF_EVEN");
        // per channel, zero rows have no scales to write
        require(scales != nullptr || (granularity == CFH_GRAN_CHANNEL && rows == 0), "scales must not be NULL");
        const int64_t n = rows * cols;
        require(n == 0 || (src && codes), "src and codes must not be NULL");
        // formats.rs:654-660: bits == 4 -> [-8, 7], anything else -> [-128, 127]
        SymEnc e{bits == 4 ? -8.0f : -128.0f, bits == 4 ? 7.0f : 127.0f, round_mode};
        hipStream_t st = static_cast<hipStream_t>(stream);
        if (granularity == CFH_GRAN_CHANNEL) {
            const bool vec = (cols % 4 == 0) && aligned(src, 16) && aligned(codes, 4);
            with_round_mode(e, [&](auto em) {
                launch_rows_quant(F32x4Src{src}, vec, rows, cols, em, reinterpret_cast<uint8_t *>(codes), scales, st);
            });
            return;
        }
        uint32_t *acc = reinterpret_cast<uint32_t *>(scales);
        fill_u32_kernel<<<1, 1, 0, st>>>(acc, 0u);
        check_launch("fill_u32");
        if (n > 0) {
            tensor_absmax_kernel<<<grid_for(n / 4 + 1, kBlock, kGridCap), kBlock, 0, st>>>(src, n, acc);
            check_launch("tensor_absmax");
            tensor_quant_kernel<<<grid_for(n / 4 + 1, kBlock, kGridCap), kBlock, 0, st>>>(
                src, n, e, acc, reinterpret_cast<uint8_t *>(codes));
            check_launch("tensor_quant");
        }
        tensor_scale_finalize_kernel<<<1, 1, 0, st>>>(scales, e);
        check_launch("tensor_scale_finalize");
    });
}

int32_t castforge_hip_absmax_f32(const float *src, int64_t n, float *out, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(n >= 0, "n must be non-negative");
        require(out != nullptr && (n == 0 || src != nullptr), "buffers must not be NULL");
        hipStream_t st = static_cast<hipStream_t>(stream);
        uint32_t *acc = reinterpret_cast<uint32_t *>(out);
        fill_u32_kernel<<<1, 1, 0, st>>>(acc, 0u);
        check_launch("fill_u32");
        if (n > 0) {
            tensor_absmax_kernel<<<grid_for(n / 4 + 1, kBlock, kGridCap), kBlock, 0, st>>>(src, n, acc);
            check_launch("tensor_absmax");
        }
    });
}

int32_t castforge_hip_dequantize_int8(const int8_t *codes, const float *scales, int64_t rows,
                                      int64_t cols, int32_t granularity, float *out, void *stream,
                                      char **out_error) {
    return guarded(out_error, [&] {
        check_shape(rows, cols);
        require(granularity == CFH_GRAN_TENSOR || granularity == CFH_GRAN_CHANNEL,
                "granularity must be CFH_GRAN_TENSOR or CFH_GRAN_CHANNEL");
        const int64_t n = rows * cols;
        if (n == 0) return;
        require(codes && scales && out, "codes, scales and out must not be NULL");
        dequant_int8_kernel<<<grid_for(n, kBlock, kGridCap), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
            codes, scales, rows, cols, granularity == CFH_GRAN_CHANNEL, out);
        check_launch("dequant_int8");
    });
}

}  // extern "C"

namespace cfh {
namespace {
// int4g_quant16_kernel over a set of matrices (rows <= 65535 in total, group 16..256).
void launch_int4g16(const RowSets<float> &sets, int64_t rows, int64_t cols, int64_t group, hipStream_t st,
                    int rot_b = 0, float rot_norm = 1.0f) {
    // 16 codes per thread: a task (8 groups) takes group / 2 threads; one grid row per row
    const int64_t G = (cols + group - 1) / group, ZW = (G + 7) / 8;
    const int64_t tpb = kBlock / (group / 2);
    // with an AWQ pre-scale, CFH_INT4Q16_AWQ_ROWS rows per grid row when every matrix allows
    bool awq = false, even = true;
    for (int i = 0; i < sets.count; ++i) {
        awq = awq || sets.in_scale[i] != nullptr;
        even = even && (sets.row_end[i] - (i > 0 ? sets.row_end[i - 1] : 0)) % CFH_INT4Q16_AWQ_ROWS == 0;
    }
    const int R = awq && even ? CFH_INT4Q16_AWQ_ROWS : 1;
    dim3 g(static_cast<unsigned>((ZW + tpb - 1) / tpb), static_cast<unsigned>(rows / R)), b(kBlock);
    auto go = [&](auto grp, auto r) {
        int4g_quant16_kernel<decltype(grp)::value, decltype(r)::value><<<g, b, 0, st>>>(sets, cols, rot_b, rot_norm);
    };
    auto by_group = [&](auto r) {
        switch (group) {
        case 16: go(std::integral_constant<int, 16>{}, r); break;
        case 32: go(std::integral_constant<int, 32>{}, r); break;
        case 64: go(std::integral_constant<int, 64>{}, r); break;
        case 128: go(std::integral_constant<int, 128>{}, r); break;
        default: go(std::integral_constant<int, 256>{}, r); break;
        }
    };
    if (R == 1) by_group(std::integral_constant<int, 1>{});
    else by_group(std::integral_constant<int, CFH_INT4Q16_AWQ_ROWS>{});
    check_launch("int4g_quant16");
}

void quantize_int4g_impl(const float *src, const float *in_scale, int64_t rows, int64_t cols, int64_t group,
                         uint32_t *codes, uint16_t *scales_f16, uint32_t *zeros, void *stream) {
    check_shape(rows, cols);
    require(pow2_in(group, 8, 256), "group must be a power of two in [8, 256]");
    require(cols % 8 == 0, "cols must be a multiple of 8 (8 codes per 32-bit word)");
    if (rows == 0 || cols == 0) return;
    require(src && codes && scales_f16 && zeros, "buffers must not be NULL");
    require(aligned(src, 16), "src must be 16-byte aligned");
    require(!in_scale || aligned(in_scale, 16), "in_scale must be 16-byte aligned");
    require(aligned(codes, 4) && aligned(scales_f16, 2) && aligned(zeros, 4),
            "codes/zeros must be 4-byte and scales 2-byte aligned");
    const int64_t G = (cols + group - 1) / group, ZW = (G + 7) / 8;
    const int64_t tasks = rows * ZW;
    hipStream_t st = static_cast<hipStream_t>(stream);
    dim3 b(kBlock);
    if (group >= 16 && CFH_INT4Q16 && rows <= 65535 && cols < (int64_t{1} << 31)) {
        launch_int4g16(one_set(src, in_scale, codes, scales_f16, zeros, rows), rows, cols, group, st);
        return;
    }
    const int64_t tpb = kBlock / group;
    const int64_t blocks = (tasks + tpb - 1) / tpb;
    require(blocks <= 0x7fffffff, "tensor too large for one launch");
    dim3 g(static_cast<unsigned>(blocks));
    switch (group) {
    case 8: int4g_quant_kernel<8><<<g, b, 0, st>>>(src, in_scale, rows, cols, codes, scales_f16, zeros); break;
    case 16: int4g_quant_kernel<16><<<g, b, 0, st>>>(src, in_scale, rows, cols, codes, scales_f16, zeros); break;
    case 32: int4g_quant_kernel<32><<<g, b, 0, st>>>(src, in_scale, rows, cols, codes, scales_f16, zeros); break;
    case 64: int4g_quant_kernel<64><<<g, b, 0, st>>>(src, in_scale, rows, cols, codes, scales_f16, zeros); break;
    case 128: int4g_quant_kernel<128><<<g, b, 0, st>>>(src, in_scale, rows, cols, codes, scales_f16, zeros); break;
    default: int4g_quant_kernel<256><<<g, b, 0, st>>>(src, in_scale, rows, cols, codes, scales_f16, zeros); break;
    }
    check_launch("int4g_quant");
}

// INT8 symmetric per-channel of one matrix (the castforge_hip_quantize_int8 channel path).
void quantize_int8_rows(const float *src, int64_t rows, int64_t cols, SymEnc e, int8_t *codes,
                        float *scales, hipStream_t st) {
    const bool vec = (cols % 4 == 0) && aligned(src, 16) && aligned(codes, 4);
    with_round_mode(e, [&](auto em) {
        launch_rows_quant(F32x4Src{src}, vec, rows, cols, em, reinterpret_cast<uint8_t *>(codes), scales, st);
    });
}

// Batched quantize: the problems are grouped by column count (in order of first appearance);
// each group is quantized by as few launches as possible (at most kQSets matrices, and for
// INT4 at most 65535 rows, per launch).  A matrix the batched kernels cannot take (alignment,
// row length, group size) is quantized on its own by the single-matrix path.
// in_scales (INT4 only, may be NULL): per problem, the AWQ per-column pre-scale (device f32
// [cols], 16-byte aligned) fused into the pass as in castforge_hip_quantize_int4g_awq.
void quantize_batched(const cfh_quant_problem_t *ps, const float *const *in_scales, int32_t count,
                      bool int4, int64_t group, SymEnc e, hipStream_t st) {
    require(count >= 0 && count <= CFH_MAX_BATCH, "count must be in [0, CFH_MAX_BATCH]");
    require(count == 0 || ps != nullptr, "problems must not be NULL");
    if (int4) require(pow2_in(group, 8, 256), "group must be a power of two in [8, 256]");
    for (int i = 0; i < count; ++i) {
        const cfh_quant_problem_t &q = ps[i];
        check_shape(q.rows, q.cols);
        require(q.rows == 0 || q.cols == 0 || (q.src && q.codes && q.scales), "problem buffers must not be NULL");
        if (int4) {
            require(q.cols % 8 == 0, "cols must be a multiple of 8 (8 codes per 32-bit word)");
            require(q.rows == 0 || q.cols == 0 || q.zeros, "zeros must not be NULL");
            if (in_scales && q.rows > 0 && q.cols > 0)
                require(in_scales[i] != nullptr && aligned(in_scales[i], 16),
                        "in_scale must be a non-NULL 16-byte aligned device pointer");
        } else {
            require(q.rows == 0 || q.scales, "scales must not be NULL");
        }
    }
    bool done[CFH_MAX_BATCH] = {};
    for (int i = 0; i < count; ++i) {
        if (done[i]) continue;
        const int64_t cols = ps[i].cols;
        RowSets<float> sets{};
        int64_t rows = 0;
        auto flush = [&]() {
            if (sets.count > 0) {
                if (int4) launch_int4g16(sets, rows, cols, group, st);
                else with_round_mode(e, [&](auto em) { launch_rows_quant_sets<F32x4Src>(sets, rows, cols, em, st); });
            }
            sets = RowSets<float>{};
            rows = 0;
        };
        for (int j = i; j < count; ++j) {
            const cfh_quant_problem_t &q = ps[j];
            if (done[j] || q.cols != cols) continue;
            done[j] = true;
            if (int4 && q.rows > 0 && cols > 0) {
                const bool ok = group >= 16 && CFH_INT4Q16 && q.rows <= 65535 && cols < (int64_t{1} << 31) &&
                                aligned(q.src, 16) && aligned(q.codes, 4) && aligned(q.scales, 2) && aligned(q.zeros, 4);
                if (!ok) {
                    quantize_int4g_impl(q.src, in_scales ? in_scales[j] : nullptr, q.rows, cols, group,
                                        static_cast<uint32_t *>(q.codes), static_cast<uint16_t *>(q.scales),
                                        q.zeros, st);
                    continue;
                }
                if (rows + q.rows > 65535) flush();
            } else if (!int4 && q.rows > 0) {
                const bool ok = cols > 0 && cols % 4 == 0 && cols / 4 <= 16 * kBlock && aligned(q.src, 16) &&
                                aligned(q.codes, 4) && rows + q.rows <= 0x7fffffff;
                if (!ok) {
                    quantize_int8_rows(q.src, q.rows, cols, e, static_cast<int8_t *>(q.codes),
                                       static_cast<float *>(q.scales), st);
                    continue;
                }
            } else {
                continue;  // nothing to quantize
            }
            if (sets.count == kQSets) flush();
            sets.src[sets.count] = q.src;
            sets.in_scale[sets.count] = int4 && in_scales ? in_scales[j] : nullptr;
            sets.codes[sets.count] = q.codes;
            sets.scales[sets.count] = q.scales;
            sets.zeros[sets.count] = q.zeros;
            rows += q.rows;
            sets.row_end[sets.count] = rows;
            ++sets.count;
        }
        flush();
    }
}
}  // namespace

float hadamard_norm(int64_t b);  // rotate.hip: 1 / sqrt(b) as the reference computes it

}  // namespace cfh

extern "C" {

int32_t castforge_hip_quantize_int4g_hadamard(const float *src, int64_t rows, int64_t cols, int64_t group,
                                              int64_t block, uint32_t *codes, uint16_t *scales_f16,
                                              uint32_t *zeros, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        check_shape(rows, cols);
        require(pow2_in(group, 16, 256), "group must be a power of two in [16, 256]");
        require(pow2_in(block, 2, 1024), "block must be a power of two in [2, 1024]");
        require(cols % 8 == 0 && cols % block == 0, "cols must be a multiple of 8 and of block");
        require(cols < (int64_t{1} << 31), "cols too large");
        if (rows == 0 || cols == 0) return;
        require(src && codes && scales_f16 && zeros, "buffers must not be NULL");
        require(aligned(src, 16), "src must be 16-byte aligned");
        require(aligned(codes, 4) && aligned(scales_f16, 2) && aligned(zeros, 4),
                "codes/zeros must be 4-byte and scales 2-byte aligned");
        const int64_t G = (cols + group - 1) / group, ZW = (G + 7) / 8, GP = ZW * 8;
        const float norm = hadamard_norm(block);
        hipStream_t st = static_cast<hipStream_t>(stream);
        for (int64_t r0 = 0; r0 < rows; r0 += 65535) {  // one grid row per matrix row
            const int64_t nr = std::min<int64_t>(rows - r0, 65535);
            launch_int4g16(one_set(src + r0 * cols, nullptr, codes + r0 * (cols / 8), scales_f16 + r0 * GP,
                                   zeros + r0 * ZW, nr),
                           nr, cols, group, st, static_cast<int>(block), norm);
        }
    });
}

int32_t castforge_hip_quantize_int4g(const float *src, int64_t rows, int64_t cols, int64_t group,
                                     uint32_t *codes, uint16_t *scales_f16, uint32_t *zeros,
                                     void *stream, char **out_error) {
    return guarded(out_error, [&] {
        quantize_int4g_impl(src, nullptr, rows, cols, group, codes, scales_f16, zeros, stream);
    });
}

int32_t castforge_hip_quantize_int4g_awq(const float *src, const float *in_scale, int64_t rows, int64_t cols,
                                         int64_t group, uint32_t *codes, uint16_t *scales_f16,
                                         uint32_t *zeros, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(rows == 0 || cols == 0 || in_scale != nullptr, "in_scale must not be NULL");
        quantize_int4g_impl(src, in_scale, rows, cols, group, codes, scales_f16, zeros, stream);
    });
}

int32_t castforge_hip_dequantize_int4g(const uint32_t *codes, const uint16_t *scales_f16,
                                       const uint32_t *zeros, int64_t rows, int64_t cols,
                                       int64_t group, float *out, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        check_shape(rows, cols);
        require(group >= 8 && group % 8 == 0, "group must be a positive multiple of 8");
        require(cols % 8 == 0, "cols must be a multiple of 8");
        if (rows == 0 || cols == 0) return;
        require(codes && scales_f16 && zeros && out, "buffers must not be NULL");
        dequant_int4g_kernel<<<grid_for(rows * (cols / 8), kBlock, kGridCap), kBlock, 0,
                               static_cast<hipStream_t>(stream)>>>(codes, scales_f16, zeros, rows,
                                                                   cols, group, out);
        check_launch("dequant_int4g");
    });
}

int32_t castforge_hip_quantize_nf4(const float *src, int64_t rows, int64_t cols, int64_t block,
                                   uint32_t *codes, float *absmax, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        check_shape(rows, cols);
        require(pow2_in(block, 8, 512), "block must be a power of two in [8, 512]");
        require(cols % 8 == 0, "cols must be a multiple of 8 (8 codes per 32-bit word)");
        if (rows == 0 || cols == 0) return;
        require(src && codes && absmax, "buffers must not be NULL");
        require(aligned(src, 16) && aligned(codes, 4) && aligned(absmax, 4),
                "src must be 16-byte aligned, codes/absmax 4-byte aligned");
        const int64_t B = (cols + block - 1) / block, KWp = B * (block / 8);
        const int64_t threads = rows * KWp, blocks = (threads + kBlock - 1) / kBlock;
        require(blocks <= 0x7fffffff, "tensor too large for one launch");
        hipStream_t st = static_cast<hipStream_t>(stream);
        dim3 g(static_cast<unsigned>(blocks)), b(kBlock);
        switch (block) {
        case 8: nf4_quant_kernel<8><<<g, b, 0, st>>>(src, rows, cols, codes, absmax); break;
        case 16: nf4_quant_kernel<16><<<g, b, 0, st>>>(src, rows, cols, codes, absmax); break;
        case 32: nf4_quant_kernel<32><<<g, b, 0, st>>>(src, rows, cols, codes, absmax); break;
        case 64: nf4_quant_kernel<64><<<g, b, 0, st>>>(src, rows, cols, codes, absmax); break;
        case 128: nf4_quant_kernel<128><<<g, b, 0, st>>>(src, rows, cols, codes, absmax); break;
        case 256: nf4_quant_kernel<256><<<g, b, 0, st>>>(src, rows, cols, codes, absmax); break;
        default: nf4_quant_kernel<512><<<g, b, 0, st>>>(src, rows, cols, codes, absmax); break;
        }
        check_launch("nf4_quant");
    });
}

int32_t castforge_hip_dequantize_nf4(const uint32_t *codes, const float *absmax, int64_t rows,
                                     int64_t cols, int64_t block, float *out, void *stream,
                                     char **out_error) {
    return guarded(out_error, [&] {
        check_shape(rows, cols);
        require(block >= 8 && block % 8 == 0, "block must be a positive multiple of 8");
        require(cols % 8 == 0, "cols must be a multiple of 8");
        if (rows == 0 || cols == 0) return;
        require(codes && absmax && out, "buffers must not be NULL");
        dequant_nf4_kernel<<<grid_for(rows * (cols / 8), kBlock, kGridCap), kBlock, 0,
                             static_cast<hipStream_t>(stream)>>>(codes, absmax, rows, cols, block, out);
        check_launch("dequant_nf4");
    });
}

// Threads per row and 16-byte pieces per thread for fp8_rows_bf16x8_kernel, by row length
// (nv8 = cols / 8 pieces, at most 8 per thread).
#ifndef CFH_FP8_TPR
#define CFH_FP8_TPR 0
#endif
void launch_fp8_rows_bf16x8(const uint16_t *src, int64_t rows, int64_t cols, uint8_t *codes, float *scales,
                            hipStream_t st) {
    const int64_t nv8 = cols / 8;
    auto go = [&](auto vpt, auto tpr) {
        constexpr int V = decltype(vpt)::value, T = decltype(tpr)::value, N = T == 64 ? 256 : T;
        constexpr int rpw = N / T;
        require((rows + rpw - 1) / rpw <= 0x7fffffff, "too many rows for one launch");
        const dim3 grid(static_cast<unsigned>((rows + rpw - 1) / rpw)), block(N);
        fp8_rows_bf16x8_kernel<V, T, N><<<grid, block, 0, st>>>(src, rows, cols, codes, scales);
        check_launch("fp8_rows_bf16x8");
    };
    int tpr = CFH_FP8_TPR ? CFH_FP8_TPR : (nv8 <= 2048 ? 256 : 1024);
    if (nv8 > 16 * tpr) tpr = 1024;
    auto by_vpt = [&](auto tprc) {
        constexpr int T = decltype(tprc)::value;
        if (nv8 <= 1 * T) go(std::integral_constant<int, 1>{}, tprc);
        else if (nv8 <= 2 * T) go(std::integral_constant<int, 2>{}, tprc);
        else if (nv8 <= 3 * T) go(std::integral_constant<int, 3>{}, tprc);
        else if (nv8 <= 4 * T) go(std::integral_constant<int, 4>{}, tprc);
        else if (nv8 <= 6 * T) go(std::integral_constant<int, 6>{}, tprc);
        else if (nv8 <= 8 * T) go(std::integral_constant<int, 8>{}, tprc);
        else if (nv8 <= 11 * T) go(std::integral_constant<int, 11>{}, tprc);
        else {
            require(nv8 <= 16 * T, "row too long for fp8_rows_bf16x8_kernel");
            go(std::integral_constant<int, 16>{}, tprc);
        }
    };
    switch (tpr) {
        case 64: by_vpt(std::integral_constant<int, 64>{}); break;
        case 128: by_vpt(std::integral_constant<int, 128>{}); break;
        case 512: by_vpt(std::integral_constant<int, 512>{}); break;
        case 1024: by_vpt(std::integral_constant<int, 1024>{}); break;
        default: by_vpt(std::integral_constant<int, 256>{}); break;
    }
}

int32_t castforge_hip_quantize_fp8(const void *src, int32_t src_dtype, int64_t rows, int64_t cols,
                                   uint8_t *codes, float *scales, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        check_shape(rows, cols);
        require(src_dtype == CFH_DTYPE_F32 || src_dtype == CFH_DTYPE_BF16,
                "src_dtype must be CFH_DTYPE_F32 or CFH_DTYPE_BF16");
        if (rows == 0) return;
        require(scales != nullptr, "scales must not be NULL");
        require(cols == 0 || (src && codes), "src and codes must not be NULL");
        hipStream_t st = static_cast<hipStream_t>(stream);
        if (src_dtype == CFH_DTYPE_F32) {
            const bool vec = (cols % 4 == 0) && aligned(src, 16) && aligned(codes, 4);
            launch_rows_quant(F32x4Src{static_cast<const float *>(src)}, vec, rows, cols, Fp8Enc{},
                              codes, scales, st);
        } else {
            const int64_t nv8 = cols / 8;
            if (cols > 0 && cols % 8 == 0 && aligned(src, 16) && aligned(codes, 8) && nv8 <= 8 * 1024) {
                launch_fp8_rows_bf16x8(static_cast<const uint16_t *>(src), rows, cols, codes, scales, st);
                return;
            }
            const bool vec = (cols % 4 == 0) && aligned(src, 8) && aligned(codes, 4);
            launch_rows_quant(Bf16x4Src{static_cast<const uint16_t *>(src)}, vec, rows, cols,
                              Fp8Enc{}, codes, scales, st);
        }
    });
}

int32_t castforge_hip_dequantize_fp8(const uint8_t *codes, const float *scales, int64_t rows,
                                     int64_t cols, float *out, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        check_shape(rows, cols);
        const int64_t n = rows * cols;
        if (n == 0) return;
        require(codes && scales && out, "buffers must not be NULL");
        dequant_fp8_kernel<<<grid_for(n, kBlock, kGridCap), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
            codes, scales, rows, cols, out);
        check_launch("dequant_fp8");
    });
}

}  // extern "C"

extern "C" {

int32_t castforge_hip_quantize_int4g_batched(const cfh_quant_problem_t *problems, int32_t count,
                                             int64_t group, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        quantize_batched(problems, nullptr, count, true, group, SymEnc{}, static_cast<hipStream_t>(stream));
    });
}
int32_t castforge_hip_quantize_int4g_awq_batched(const cfh_quant_problem_t *problems,
                                                 const float *const *in_scales, int32_t count,
                                                 int64_t group, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(count == 0 || in_scales != nullptr, "in_scales must not be NULL");
        quantize_batched(problems, in_scales, count, true, group, SymEnc{}, static_cast<hipStream_t>(stream));
    });
}

int32_t castforge_hip_quantize_int8_batched(const cfh_quant_problem_t *problems, int32_t count,
                                            int32_t bits, int32_t round_mode, void *stream,
                                            char **out_error) {
    return guarded(out_error, [&] {
        require(round_mode == CFH_ROUND_HALF_AWAY || round_mode == CFH_ROUND_HALF_EVEN,
                "round_mode must be CFH_ROUND_HALF_AWAY or CFH_ROUND_HALF_EVEN");
        // formats.rs:654-660: bits == 4 -> [-8, 7], anything else -> [-128, 127]
        SymEnc e{bits == 4 ? -8.0f : -128.0f, bits == 4 ? 7.0f : 127.0f, round_mode};
        quantize_batched(problems, nullptr, count, false, 0, e, static_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
