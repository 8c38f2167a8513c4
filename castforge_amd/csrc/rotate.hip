// Outlier-suppression write-back passes on the GPU, gfx950 (built -ffp-contract=off).
//
//  * rotate-hadamard (passes/quantize/formats.rs:260-343): every block of b consecutive
//    elements along the rotated axis goes through the radix-2 butterfly (x + y, x - y) with
//    stages h = 1, 2, 4, ..., b/2 in that order, then each value is multiplied by
//    1 / sqrt(b).  A stage's pairs are independent, so any split of the stages over threads
//    that keeps the stage order gives the reference's values bit for bit.  The split used
//    here: a first phase of up to 64 stages' worth of values per thread in registers (axis 0,
//    strided columns) or 8 values per lane with cross-lane stages up to 512 (axis 1,
//    contiguous rows); later phases take G <= 64 values at stride h_lo, one pass over HBM
//    each (b <= 64: one pass; b <= 4096: two).
//  * smooth-quantize (passes/quantize/schemes.rs:190-298): per element
//    q = clamp(round_half_away((v * s) / e), qmin, qmax), v' = (q * e) / s with the per-tensor
//    smoothing scale s and quantizer step e; the two scalars are computed on the host with
//    the C library's powf, as the reference computes them (f32::powf).
#include <cmath>

#include <algorithm>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxG = 64;      // values per thread in a strided phase
constexpr int kWaveSpan = 512; // contiguous values per wave in the first phase along rows

// Stages h = 1 .. G/2 over G values held in registers (stride 1 in the array).
template <int G>
__device__ __forceinline__ void butterfly(float (&v)[G]) {
#pragma unroll
    for (int h = 1; h < G; h *= 2)
#pragma unroll
        for (int i = 0; i < G; i += 2 * h)
#pragma unroll
            for (int j = i; j < i + h; ++j) {
                const float x = v[j], y = v[j + h];
                v[j] = x + y;
                v[j + h] = x - y;
            }
}

// One phase: stages h_lo, 2 h_lo, .., (G/2) h_lo.  The tensor is O independent lines of L
// elements along the rotated axis (element (o, p) at o * o_stride + p * ax_stride); a thread
// owns the G elements base + m * h_lo of one line, base = blk * h_lo * G + low, low < h_lo.
// o_fast: consecutive threads take consecutive lines (axis 0: adjacent columns are adjacent
// addresses), else consecutive `low` (axis 1).  norm != 0 scales the results (last phase).
template <int G>
__global__ __launch_bounds__(kBlock) void fwht_strided_kernel(const float *src, float *dst, int64_t O,
                                                              int64_t o_stride, int64_t L, int64_t ax_stride,
                                                              int64_t h_lo, int o_fast, float norm) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t groups = L / G;
    if (t >= O * groups) return;
    int64_t o, grp;
    if (o_fast) {
        o = t % O;
        grp = t / O;
    } else {
        grp = t % groups;
        o = t / groups;
    }
    const int64_t base = (grp / h_lo) * h_lo * G + grp % h_lo;
    const float *s = src + o * o_stride + base * ax_stride;
    float *d = dst + o * o_stride + base * ax_stride;
    const int64_t step = h_lo * ax_stride;
    float v[G];
#pragma unroll
    for (int m = 0; m < G; ++m) v[m] = s[m * step];
    butterfly<G>(v);
    if (norm != 0.0f) {
#pragma unroll
        for (int m = 0; m < G; ++m) v[m] *= norm;
    }
#pragma unroll
    for (int m = 0; m < G; ++m) d[m * step] = v[m];
}

// First phase along contiguous rows: the flattened tensor in segments of 512 values, lane l
// of a wave owning values 8l .. 8l+7 of its segment.  Stages h < 8 run in registers, stages
// 8 <= h < ext (ext <= 512) against lane l ^ (h / 8) (lane_butterflies).  Blocks never
// straddle rows (b divides the row length).
template <bool VEC>
__global__ __launch_bounds__(kBlock) void fwht_rows_wave_kernel(const float *src, float *dst, int64_t n, int ext,
                                                                float norm) {
    const int64_t e = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * 8;
    float v[8];
    if (VEC && e + 8 <= n) {
        const float4 a = *reinterpret_cast<const float4 *>(src + e), b = *reinterpret_cast<const float4 *>(src + e + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = e + i < n ? src[e + i] : 0.0f;
    }
#pragma unroll
    for (int h = 1; h < 8; h *= 2) {
        if (h >= ext) break;
#pragma unroll
        for (int i = 0; i < 8; i += 2 * h)
#pragma unroll
            for (int j = i; j < i + h; ++j) {
                const float x = v[j], y = v[j + h];
                v[j] = x + y;
                v[j + h] = x - y;
            }
    }
    lane_butterflies<8>(v, ext >> 3);  // stages h = 8 .. ext / 2 (wave-uniform)
    if (norm != 0.0f) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] *= norm;
    }
    if (VEC && e + 8 <= n) {
        *reinterpret_cast<float4 *>(dst + e) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(dst + e + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (e + i < n) dst[e + i] = v[i];
    }
}

// Rows rotation for b = 16 .. 128 in one phase, 8 values per lane: lane l of each 16-lane DPP
// row holds the 8-value sub-block hsub16(l) of its 128 values, so the cross-lane stages
// h = 8, 16, 32, 64 read lane ^ 1, ^ 2, ^ 7, ^ 8, one DPP move each.
//  * A wave whose inputs are all finite, none -0 and all below 2^117 in magnitude (no
//    intermediate can overflow) runs each cross-lane stage as one fma: the partner's value
//    times +1 on the lane keeping the sum, -1 on the other, plus its own, so the second lane
//    holds -(x - y) from then on; every value ends as (-1)^popcount(its lane's stage bits)
//    times the reference's, and the final fma by that sign times norm plus +0 restores it,
//    -0 included: from such inputs the reference never produces -0 (a sum or difference is -0
//    only with a -0 operand), and +0 turns any -0 of ours into +0.
//  * Any other wave runs x + y and x - y per stage in the same layout: the reference's
//    operations on its operands, NaN and zero signs included.
template <int CTRL>
__device__ __forceinline__ float dpp_read(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ void stage_fast(float (&v)[8], float c) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(dpp_read<CTRL>(v[i]), c, v[i]);
}
template <int CTRL>
__device__ __forceinline__ void stage_exact(float (&v)[8], bool lower) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float p = dpp_read<CTRL>(v[i]);
        v[i] = lower ? v[i] + p : p - v[i];
    }
}
template <int B>
__global__ __launch_bounds__(kBlock) void fwht_rows_fast_kernel(const float *__restrict__ src, float *__restrict__ dst,
                                                                int64_t n, float norm) {
    static_assert(B >= 16 && B <= 128, "one to four cross-lane stages");
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int sb = hsub16(static_cast<int>(threadIdx.x & 15)) & (B / 8 - 1);  // the stage bits
    const int64_t e = ((t & ~int64_t{15}) + hsub16(static_cast<int>(t & 15))) * 8;
    const bool in = e + 8 <= n;  // n is a multiple of B: a block is wholly in or out
    float v[8];
    if (in) {
        const float4 a = *reinterpret_cast<const float4 *>(src + e), b = *reinterpret_cast<const float4 *>(src + e + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
    bool odd = false;  // -0, +-inf, NaN (class bits 0, 1, 2, 5, 9) or |v| >= 2^117
#pragma unroll
    for (int i = 0; i < 8; ++i) odd |= __builtin_amdgcn_classf(v[i], 0x227) || __builtin_fabsf(v[i]) >= 0x1p117f;
#pragma unroll
    for (int h = 1; h < 8; h *= 2)
#pragma unroll
        for (int i = 0; i < 8; i += 2 * h)
#pragma unroll
            for (int j = i; j < i + h; ++j) {
                const float x = v[j], y = v[j + h];
                v[j] = x + y;
                v[j + h] = x - y;
            }
    if (__builtin_amdgcn_ballot_w64(odd) == 0) {  // wave-uniform
        stage_fast<0xB1>(v, (sb & 1) ? -1.0f : 1.0f);                     // h = 8: lane ^ 1
        if constexpr (B >= 32) stage_fast<0x4E>(v, (sb & 2) ? -1.0f : 1.0f);   // h = 16: lane ^ 2
        if constexpr (B >= 64) stage_fast<0x141>(v, (sb & 4) ? -1.0f : 1.0f);  // h = 32: lane ^ 7
        if constexpr (B >= 128) stage_fast<0x128>(v, (sb & 8) ? -1.0f : 1.0f); // h = 64: lane ^ 8
        const float f = (__builtin_popcount(static_cast<unsigned>(sb)) & 1) ? -norm : norm;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(v[i], f, 0.0f);
    } else {
        stage_exact<0xB1>(v, (sb & 1) == 0);
        if constexpr (B >= 32) stage_exact<0x4E>(v, (sb & 2) == 0);
        if constexpr (B >= 64) stage_exact<0x141>(v, (sb & 4) == 0);
        if constexpr (B >= 128) stage_exact<0x128>(v, (sb & 8) == 0);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] *= norm;
    }
    if (in) {
        *reinterpret_cast<float4 *>(dst + e) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(dst + e + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
}

template <int G>
void launch_strided(const float *src, float *dst, int64_t O, int64_t o_stride, int64_t L, int64_t ax_stride,
                    int64_t h_lo, int o_fast, float norm, hipStream_t st) {
    const int64_t threads = O * (L / G);
    const int64_t grid = (threads + kBlock - 1) / kBlock;
    require(grid <= 0x7fffffff, "tensor too large for one launch");
    fwht_strided_kernel<G><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(src, dst, O, o_stride, L, ax_stride,
                                                                          h_lo, o_fast, norm);
    check_launch("fwht_strided");
}

void strided_phase(int g, const float *src, float *dst, int64_t O, int64_t o_stride, int64_t L, int64_t ax_stride,
                   int64_t h_lo, int o_fast, float norm, hipStream_t st) {
    switch (g) {
    case 2: launch_strided<2>(src, dst, O, o_stride, L, ax_stride, h_lo, o_fast, norm, st); break;
    case 4: launch_strided<4>(src, dst, O, o_stride, L, ax_stride, h_lo, o_fast, norm, st); break;
    case 8: launch_strided<8>(src, dst, O, o_stride, L, ax_stride, h_lo, o_fast, norm, st); break;
    case 16: launch_strided<16>(src, dst, O, o_stride, L, ax_stride, h_lo, o_fast, norm, st); break;
    case 32: launch_strided<32>(src, dst, O, o_stride, L, ax_stride, h_lo, o_fast, norm, st); break;
    default: launch_strided<64>(src, dst, O, o_stride, L, ax_stride, h_lo, o_fast, norm, st); break;
    }
}

bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

// Rust's f32::clamp / max on the host (NaN handling of the scale arithmetic)
float rust_max(float a, float b) { return std::isnan(a) ? b : (std::isnan(b) ? a : (a > b ? a : b)); }

__global__ __launch_bounds__(kBlock) void smoothquant_kernel(const float *w, int64_t n, float s, float e, float qmin,
                                                             float qmax, float *out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    const float r = roundf((w[i] * s) / e);
    const float q = r != r ? r : (r < qmin ? qmin : (r > qmax ? qmax : r));
    out[i] = (q * e) / s;
}

}  // namespace

// 1 / sqrt(b) in f32 as the reference computes it: 1.0_f32 / (b as f32).sqrt().
float hadamard_norm(int64_t b) {
    const float sb = std::sqrt(static_cast<float>(b));
    return 1.0f / sb;
}

// In-place or out-of-place rotation of [d0, d1] f32 along `axis` in blocks of b.
void rotate_hadamard_impl(const float *src, float *dst, int64_t d0, int64_t d1, int64_t b, int axis, hipStream_t st) {
    const int64_t L = axis == 0 ? d0 : d1;
    const float norm = hadamard_norm(b);
    const float *in = src;
    int64_t h_lo = 1;
    if (axis == 1) {
        const int64_t n = d0 * d1;
        const int ext = static_cast<int>(b < kWaveSpan ? b : kWaveSpan);
        const int64_t grid = ((n + 7) / 8 + kBlock - 1) / kBlock;
        require(grid <= 0x7fffffff, "tensor too large for one launch");
        const float nm = ext == b ? norm : 0.0f;
        const bool vec = aligned(in, 16) && aligned(dst, 16);
        if (vec && b >= 16 && b <= 128) {
            if (b == 16) fwht_rows_fast_kernel<16><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(in, dst, n, norm);
            else if (b == 32) fwht_rows_fast_kernel<32><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(in, dst, n, norm);
            else if (b == 64) fwht_rows_fast_kernel<64><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(in, dst, n, norm);
            else fwht_rows_fast_kernel<128><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(in, dst, n, norm);
        } else if (vec)
            fwht_rows_wave_kernel<true><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(in, dst, n, ext, nm);
        else
            fwht_rows_wave_kernel<false><<<static_cast<unsigned>(grid), kBlock, 0, st>>>(in, dst, n, ext, nm);
        check_launch("fwht_rows_wave");
        in = dst;
        h_lo = ext;
    }
    const int64_t O = axis == 0 ? d1 : d0;
    const int64_t o_stride = axis == 0 ? 1 : d1, ax_stride = axis == 0 ? d1 : 1;
    while (h_lo < b) {
        const int64_t g = std::min<int64_t>(b / h_lo, kMaxG);
        const bool last = h_lo * g == b;
        strided_phase(static_cast<int>(g), in, dst, O, o_stride, L, ax_stride, h_lo, axis == 0,
                      last ? norm : 0.0f, st);
        in = dst;
        h_lo *= g;
    }
}

}  // namespace cfh

using namespace cfh;

extern "C" {

int32_t castforge_hip_rotate_hadamard(const float *src, int64_t d0, int64_t d1, int64_t block, int32_t axis,
                                      float *dst, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(axis == 0 || axis == 1, "axis must be 0 (rows of [d0, d1] blocks, the reference) or 1");
        require(d0 >= 0 && d1 >= 0, "d0 and d1 must be non-negative");
        require(pow2(block) && block >= 2, "block must be a power of two >= 2");
        const int64_t L = axis == 0 ? d0 : d1;
        require(L % block == 0, "the rotated axis length must be a multiple of block");
        if (d0 == 0 || d1 == 0) return;
        require(src && dst, "src and dst must not be NULL");
        rotate_hadamard_impl(src, dst, d0, d1, block, axis, static_cast<hipStream_t>(stream));
    });
}

int32_t castforge_hip_smoothquant_scales(float act_max, float w_max, float alpha, int32_t bits, float *out_scales,
                                         char **out_error) {
    return guarded(out_error, [&] {
        require(out_scales != nullptr, "out_scales must not be NULL");
        // schemes.rs:231-233 (alpha is clamped by the caller, schemes.rs:196)
        const float qmax = bits == 4 ? 7.0f : 127.0f;  // formats.rs:654-660
        const float num = std::pow(rust_max(act_max, 1e-4f), alpha);
        const float den = std::pow(w_max, 1.0f - alpha);
        const float s = rust_max(num / den, 1e-4f);
        const float e = rust_max(w_max * s / qmax, 1e-6f);
        out_scales[0] = s;
        out_scales[1] = e;
    });
}

int32_t castforge_hip_smoothquant(const float *w, int64_t n, float smooth_scale, float eff_qscale, int32_t bits,
                                  float *out, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(n >= 0, "n must be non-negative");
        if (n == 0) return;
        require(w && out, "w and out must not be NULL");
        const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
        const int64_t grid = (n + kBlock - 1) / kBlock;
        require(grid <= 0x7fffffff, "tensor too large for one launch");
        smoothquant_kernel<<<static_cast<unsigned>(grid), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
            w, n, smooth_scale, eff_qscale, qmin, qmax, out);
        check_launch("smoothquant");
    });
}

}  // extern "C"
