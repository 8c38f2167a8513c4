// The reference's write-back quantizers on gfx950: group-wise / AWQ-salient
// (QuantizeGroupwisePass, passes/quantize/schemes.rs:456-630) and the FP8 / MXFP8 uniform-grid
// pass (QuantizeFp8Pass, schemes.rs:633-754).  Both return dequantized f32 values of the same
// shape, as the reference writes back into the TensorStore (schemes.rs:565-570, 714-720).
//
// Bit-exact f32 arithmetic: correctly rounded division, no contraction (this file is built with
// -ffp-contract=off), Rust's f32::round (half away from zero) or IEEE half-even, Rust's
// f32::clamp (NaN propagates) and f32::max (NaN ignored) semantics.
//
// The AWQ salient threshold (schemes.rs:522-530: |w| sorted descending with total_cmp, element
// salient_count - 1) is an exact k-th-largest selection: for non-negative floats the 31-bit
// pattern orders exactly as total_cmp does (NaN above +inf), so four byte-wise radix passes
// (histogram, then a one-wave bin search) find the threshold's bit pattern without sorting.
#include <algorithm>
#include <mutex>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

constexpr int kBlock = 256;

struct SelectState {
    uint32_t prefix;     // bits of the threshold fixed so far
    uint32_t mask;       // which bits are fixed
    uint32_t k;          // rank still to find among keys matching prefix (1-based)
    uint32_t thresh;     // final threshold bits
};

// workspace: hist[256] then SelectState
struct SelectWs {
    uint32_t hist[256];
    SelectState st;
};
static_assert(sizeof(SelectWs) <= CFH_GROUPWISE_WORKSPACE_BYTES, "workspace size");

__device__ __forceinline__ uint32_t abs_key(float v) { return __float_as_uint(v) & 0x7fffffffu; }

// Rust f32::clamp: NaN stays NaN.
__device__ __forceinline__ float rust_clamp(float x, float lo, float hi) {
    return x != x ? x : fminf(fmaxf(x, lo), hi);
}

__device__ __forceinline__ float round_sel(float x, int mode) {
    return mode == CFH_ROUND_HALF_EVEN ? rintf(x) : roundf(x);
}

__global__ void select_init_kernel(SelectWs *ws, uint32_t k) {
    const int t = threadIdx.x;
    ws->hist[t] = 0;
    if (t == 0) ws->st = SelectState{0u, 0u, k, 0u};
}

// Histogram of byte `shift / 8` of |v| over the elements whose higher bytes match the prefix.
__global__ __launch_bounds__(kBlock) void select_count_kernel(const float *__restrict__ v, int64_t n,
                                                             SelectWs *ws, int shift) {
    __shared__ uint32_t h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const uint32_t prefix = ws->st.prefix, mask = ws->st.mask;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const uint32_t key = abs_key(v[i]);
        if ((key & mask) == prefix) atomicAdd(&h[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (h[threadIdx.x]) atomicAdd(&ws->hist[threadIdx.x], h[threadIdx.x]);
}

// One wave: walk the bins from the top, fix this byte of the k-th largest key, clear the
// histogram for the next pass.
__global__ void select_pick_kernel(SelectWs *ws, int shift) {
    const int lane = threadIdx.x;  // 64 lanes, 4 bins each (lane 0 holds the top bins)
    uint32_t c[4];
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        c[j] = ws->hist[255 - (lane * 4 + j)];
        sum += c[j];
    }
    // exclusive prefix of `sum` over lanes (descending key order)
    uint32_t incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
    }
    const uint32_t excl = incl - sum;
    const uint32_t k = ws->st.k;
    // the lane whose range [excl, incl) contains rank k - 1
    const bool mine = excl < k && k <= incl;
    if (mine) {
        uint32_t before = excl;
        int bin = 255 - lane * 4;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (before + c[j] >= k) {
                bin = 255 - (lane * 4 + j);
                break;
            }
            before += c[j];
        }
        SelectState s = ws->st;
        s.prefix |= static_cast<uint32_t>(bin) << shift;
        s.mask |= 255u << shift;
        s.k = k - before;
        if (shift == 0) s.thresh = s.prefix;
        ws->st = s;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) ws->hist[lane * 4 + j] = 0;
}

// One wave per group of `gs` consecutive elements (schemes.rs:532-549).
__global__ __launch_bounds__(kBlock) void groupwise_kernel(const float *__restrict__ v, int64_t n, int64_t gs,
                                                          float qmin, float qmax, int awq, int mode,
                                                          const SelectWs *ws, float *__restrict__ deq,
                                                          float *__restrict__ scales) {
    const int lane = threadIdx.x & 63;
    const int64_t g = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
    const int64_t c0 = g * gs;
    if (c0 >= n) return;
    const int64_t c1 = c0 + gs < n ? c0 + gs : n;
    float gmax = 0.0f;
    for (int64_t i = c0 + lane; i < c1; i += 64) gmax = fmaxf(gmax, fabsf(v[i]));
    gmax = wave_max<64>(gmax);
    const float scale = gmax < 1e-12f ? 1.0f : gmax / qmax;
    if (scales && lane == 0) scales[g] = scale;
    const float thr = awq ? __uint_as_float(ws->st.thresh) : 0.0f;
    for (int64_t i = c0 + lane; i < c1; i += 64) {
        const float x = v[i];
        const float eff = (awq && fabsf(x) >= thr) ? scale * 0.5f : scale;
        const float q = rust_clamp(round_sel(x / eff, mode), qmin, qmax);
        deq[i] = q * eff;
    }
}

// Exponent c with 2^c == powf(2, ceilf(log2f(raw))) as the reference computes the MX scale
// (schemes.rs:706).  ceil(log2(raw)) is e for raw = 2^e, else e + 1, except where the f32
// rounding of log2f lands exactly on the integer e: raw = 2^e (1 + m 2^-23) with a small m,
// below the half-spacing of f32 values next to e.  This closed form agrees with glibc's
// log2f on every positive normal f32 (checked exhaustively on the CPU by the oracle tests).
__device__ __forceinline__ int mx_scale_exp(float raw) {
    const uint32_t b = __float_as_uint(raw);
    const int e = static_cast<int>((b >> 23) & 0xffu) - 127;
    const uint32_t m = b & 0x7fffffu;
    if (m == 0) return e;
    if (e == 0) return 1;
    const int a = e > 0 ? e : -e;
    const int fl = 31 - __builtin_clz(static_cast<unsigned>(a));
    const double h = (e < 0 && (a & (a - 1)) == 0) ? ldexp(1.0, fl - 25) : ldexp(1.0, fl - 24);
    const double thr = (exp2(h) - 1.0) * 8388608.0;
    return static_cast<double>(m) < thr ? e : e + 1;
}

// One wave per block of `bs` consecutive elements (schemes.rs:697-713).
__global__ __launch_bounds__(kBlock) void fp8_grid_kernel(const float *__restrict__ v, int64_t n, int64_t bs,
                                                         float fp8_max, float grid_steps, int mxfp8,
                                                         float *__restrict__ deq) {
    const int lane = threadIdx.x & 63;
    const int64_t blk = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
    const int64_t c0 = blk * bs;
    if (c0 >= n) return;
    const int64_t c1 = c0 + bs < n ? c0 + bs : n;
    float amax = 0.0f;
    for (int64_t i = c0 + lane; i < c1; i += 64) amax = fmaxf(amax, fabsf(v[i]));
    amax = wave_max<64>(amax);
    const float raw = amax < 1e-12f ? 1.0f : amax / fp8_max;
    // the reference's raw is a normal f32 here (>= 1e-12 / 57344) or +inf
    const float scale = mxfp8 ? ldexpf(1.0f, mx_scale_exp(raw)) : raw;
    const float step = fmaxf(fp8_max / grid_steps, 1e-6f);
    for (int64_t i = c0 + lane; i < c1; i += 64) {
        const float scaled = rust_clamp(v[i] / scale, -fp8_max, fp8_max);
        const float q = roundf(scaled / step) * step;
        deq[i] = q * scale;
    }
}

// Scratch of castforge_hip_quantize_groupwise_noalloc: one threshold-search state per device,
// held until the process ends.  Host code never passes `scratch` itself to a kernel (in host
// code the name is a stand-in, not a device address): device_scratch() resolves this device's
// copy once with hipGetSymbolAddress and every use goes through that pointer.
static __device__ __align__(256) uint8_t scratch[CFH_GROUPWISE_WORKSPACE_BYTES];
static_assert(sizeof(SelectWs) <= sizeof(scratch), "selection state fits the scratch array");

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void *scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch`, resolved on the first call made on the device (the
// device current at that call).
void *device_scratch() {
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < kMaxDevices, "device ordinal beyond the scratch table (64 devices)");
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        void *p = nullptr;
        check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        require(p != nullptr, "hipGetSymbolAddress(scratch) returned NULL");
        scratch_ptr[dev] = p;
    }
    return scratch_ptr[dev];
}

// Both groupwise entry points: `workspace` is the caller's buffer or this device's scratch.
int32_t groupwise(const float *src, int64_t n, int32_t bits, int64_t group_size, int32_t awq_salient,
                  float salient_ratio, int32_t round_mode, float *deq, float *scales, void *workspace,
                  bool use_scratch, int64_t *salient_count_out, void *stream, char **out_error) {
    if (salient_count_out) *salient_count_out = 0;
    return guarded(out_error, [&] {
        require(n >= 0, "n must be non-negative");
        require(round_mode == CFH_ROUND_HALF_AWAY || round_mode == CFH_ROUND_HALF_EVEN,
                "round_mode must be CFH_ROUND_HALF_AWAY or CFH_ROUND_HALF_EVEN");
        require(n < (int64_t{1} << 32), "tensors of 2^32 or more elements are not supported");
        // schemes.rs:486-487: group_size.max(2), salient_ratio.clamp(0.001, 0.5)
        const int64_t gs = group_size < 2 ? 2 : group_size;
        float ratio = salient_ratio != salient_ratio ? salient_ratio
                                                     : fminf(fmaxf(salient_ratio, 0.001f), 0.5f);
        // schemes.rs:524-527: ceil(f32(n) * ratio) as usize, then max(1).min(n)
        const float cnt_f = ceilf(static_cast<float>(n) * ratio);
        int64_t cnt = (cnt_f != cnt_f || cnt_f <= 0.0f) ? 0
                      : cnt_f >= 9.2e18f ? INT64_MAX : static_cast<int64_t>(cnt_f);
        if (cnt < 1) cnt = 1;
        if (cnt > n) cnt = n;
        if (salient_count_out) *salient_count_out = n > 0 ? cnt : 1;
        if (n == 0) return;
        require(src && deq, "src and deq must not be NULL");
        if (use_scratch && awq_salient) workspace = device_scratch();
        require(!awq_salient || workspace, "workspace must not be NULL when awq_salient is set");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const float qmin = bits == 4 ? -8.0f : -128.0f, qmax = bits == 4 ? 7.0f : 127.0f;
        SelectWs *ws = static_cast<SelectWs *>(workspace);
        if (awq_salient) {
            select_init_kernel<<<1, 256, 0, st>>>(ws, static_cast<uint32_t>(cnt));
            check_launch("select_init");
            const int64_t blocks = std::min<int64_t>((n + kBlock - 1) / kBlock, 4096);
            for (int shift = 24; shift >= 0; shift -= 8) {
                select_count_kernel<<<static_cast<unsigned>(blocks), kBlock, 0, st>>>(src, n, ws, shift);
                check_launch("select_count");
                select_pick_kernel<<<1, 64, 0, st>>>(ws, shift);
                check_launch("select_pick");
            }
        }
        const int64_t groups = (n + gs - 1) / gs;
        const int64_t grid = (groups + kBlock / 64 - 1) / (kBlock / 64);
        require(grid <= 0x7fffffff, "too many groups");
        groupwise_kernel<<<static_cast<unsigned>(grid), kBlock, 0, st>>>(src, n, gs, qmin, qmax, awq_salient ? 1 : 0,
                                                                      round_mode, ws, deq, scales);
        check_launch("groupwise");
    });
}

}  // namespace
}  // namespace cfh

using namespace cfh;

extern "C" {

int32_t castforge_hip_quantize_groupwise(const float *src, int64_t n, int32_t bits, int64_t group_size,
                                         int32_t awq_salient, float salient_ratio, int32_t round_mode,
                                         float *deq, float *scales, void *workspace,
                                         int64_t *salient_count_out, void *stream, char **out_error) {
    return groupwise(src, n, bits, group_size, awq_salient, salient_ratio, round_mode, deq, scales, workspace,
                     false, salient_count_out, stream, out_error);
}

int32_t castforge_hip_quantize_groupwise_noalloc(const float *src, int64_t n, int32_t bits,
                                                 int64_t group_size, int32_t awq_salient,
                                                 float salient_ratio, int32_t round_mode, float *deq,
                                                 float *scales, int64_t *salient_count_out, void *stream,
                                                 char **out_error) {
    return groupwise(src, n, bits, group_size, awq_salient, salient_ratio, round_mode, deq, scales, nullptr,
                     true, salient_count_out, stream, out_error);
}

int32_t castforge_hip_quantize_fp8_grid(const float *src, int64_t n, int32_t e5m2, int32_t mxfp8,
                                        int64_t block_size, float *deq, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(n >= 0, "n must be non-negative");
        if (n == 0) return;
        require(src && deq, "src and deq must not be NULL");
        const int64_t bs = block_size < 4 ? 4 : block_size;  // schemes.rs:676
        const float fp8_max = e5m2 ? 57344.0f : 448.0f, steps = e5m2 ? 15.0f : 31.0f;
        const int64_t blocks = (n + bs - 1) / bs;
        const int64_t grid = (blocks + kBlock / 64 - 1) / (kBlock / 64);
        require(grid <= 0x7fffffff, "too many blocks");
        fp8_grid_kernel<<<static_cast<unsigned>(grid), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
            src, n, bs, fp8_max, steps, mxfp8 ? 1 : 0, deq);
        check_launch("fp8_grid");
    });
}

}  // extern "C"
