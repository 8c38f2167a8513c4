// FP8 E4M3 W8A8 GEMM for gfx950: Y[m, n] = bf16((sum_k A[m, k] * W[n, k]) * sa[m] * sw[n]).
//
// A: fp8 [M, K] activations with per-token scales sa[M]; W: fp8 [N, K] weights with per-row
// scales sw[N]; both K-contiguous (the packed_rhs layout, passes/weights/fold.rs:549-554).
// This is the prefill GEMM the FP8 variant of `castforge.fused_qmatmul` lowers to
// (codegen/eval.rs:1145-1179 semantics: dequantize then eval_matmul_2d, eval.rs:1465-1507).
//
// Design (compute-bound, AI ~2.4k flop/B):
//   * workgroup tile 256 x 128, BK = 128, 4 waves in a 2 x 2 grid, 128 x 64 per wave;
//   * v_mfma_f32_16x16x128_f8f6f4 (OCP E4M3 operands), 32 accumulator tiles per wave;
//   * global -> registers -> LDS double buffer (one barrier per K step), rows padded to 144 B;
//   * XCD-aware tile order: consecutive tiles run on the same XCD (shared L2), grouped by 8
//     M-tiles so an XCD reuses the same W columns.
#include <atomic>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

typedef int int32x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BM = 256, BN = 128, BK = 128;
constexpr int kThreads = 256;
constexpr int kStride = BK + 16;                          // LDS bytes per tile row
constexpr int kStageBytes = (BM + BN) * kStride;          // 55296
constexpr int kLdsBytes = 2 * kStageBytes;                // 110592
constexpr int kALoads = BM * BK / 16 / kThreads;          // 8 x 16 B per thread
constexpr int kBLoads = BN * BK / 16 / kThreads;          // 4 x 16 B per thread
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

__device__ __forceinline__ int32x8 lds_frag(const uint8_t *base) {
    const uint4 a = *reinterpret_cast<const uint4 *>(base);
    const uint4 b = *reinterpret_cast<const uint4 *>(base + 16);
    int32x8 r = {static_cast<int>(a.x), static_cast<int>(a.y), static_cast<int>(a.z), static_cast<int>(a.w),
                 static_cast<int>(b.x), static_cast<int>(b.y), static_cast<int>(b.z), static_cast<int>(b.w)};
    return r;
}

__global__ __launch_bounds__(kThreads) void fp8_gemm_kernel(
    const uint8_t *__restrict__ A, const float *__restrict__ sa, const uint8_t *__restrict__ W,
    const float *__restrict__ sw, void *__restrict__ Y, int y_bf16, int M, int N, int K,
    int tiles_m, int tiles_n) {
    extern __shared__ __align__(16) uint8_t lds[];

    // ---- XCD-aware tile mapping ----
    const int ntiles = tiles_m * tiles_n;
    int pid = blockIdx.x;
    {
        // workgroups are dealt round-robin to the 8 XCDs; renumber so each XCD owns a
        // contiguous range of tiles (the last partial round keeps its identity order).
        const int per_xcd = ntiles / kXcds;
        const int full = per_xcd * kXcds;
        if (pid < full) pid = (pid % kXcds) * per_xcd + pid / kXcds;
    }
    const int group_span = kGroupM * tiles_n;
    const int grp = pid / group_span;
    const int first_m = grp * kGroupM;
    const int gsize = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int tm = first_m + (pid % group_span) % gsize;
    const int tn = (pid % group_span) / gsize;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * 64;
    const int lr = lane & 15, lk = (lane >> 4) * 32;

    floatx4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    uint4 ra[kALoads], rb[kBLoads];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < kALoads; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 16;
            const int gm = m0 + row;
            ra[i] = gm < M ? *reinterpret_cast<const uint4 *>(A + static_cast<int64_t>(gm) * K + k0 + col)
                           : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kBLoads; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 16;
            const int gn = n0 + row;
            rb[i] = gn < N ? *reinterpret_cast<const uint4 *>(W + static_cast<int64_t>(gn) * K + k0 + col)
                           : make_uint4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
        uint8_t *sa_ = lds + buf * kStageBytes;
        uint8_t *sb_ = sa_ + BM * kStride;
#pragma unroll
        for (int i = 0; i < kALoads; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 16;
            *reinterpret_cast<uint4 *>(sa_ + row * kStride + col) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < kBLoads; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 16;
            *reinterpret_cast<uint4 *>(sb_ + row * kStride + col) = rb[i];
        }
    };

    const int KT = K / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * BK);
        const uint8_t *sa_ = lds + buf * kStageBytes;
        const uint8_t *sb_ = sa_ + BM * kStride;
        int32x8 bf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bf[j] = lds_frag(sb_ + (wn + j * 16 + lr) * kStride + lk);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int32x8 af = lds_frag(sa_ + (wm + i * 16 + lr) * kStride + lk);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af, bf[j], acc[i][j], 0, 0, 0, 0, 0, 0);
        }
        if (kt + 1 < KT) lstore(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: per-token x per-channel scales, bf16 store ----
    const int lq = (lane >> 4) * 4;
    float swv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn + j * 16 + lr;
        swv[j] = n < N ? sw[n] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm + i * 16 + lq + r;
            if (m >= M) continue;
            const float s = sa[m];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n = n0 + wn + j * 16 + lr;
                if (n >= N) continue;
                const float v = acc[i][j][r] * s * swv[j];
                if (y_bf16)
                    static_cast<uint16_t *>(Y)[static_cast<int64_t>(m) * N + n] = f32_to_bf16_rne(v);
                else
                    static_cast<float *>(Y)[static_cast<int64_t>(m) * N + n] = v;
            }
        }
    }
}

// Any shape (K % 4 == 0): one thread per output, exact e4m3 decode, f32 accumulation.
__global__ void fp8_gemm_generic_kernel(const uint8_t *__restrict__ A, const float *__restrict__ sa,
                                        const uint8_t *__restrict__ W, const float *__restrict__ sw,
                                        void *__restrict__ Y, int y_bf16, int64_t M, int64_t N,
                                        int64_t K) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= M * N) return;
    const int64_t m = idx / N, n = idx - m * N;
    float acc = 0.f;
    for (int64_t k = 0; k < K; ++k) acc += e4m3fn_to_f32(A[m * K + k]) * e4m3fn_to_f32(W[n * K + k]);
    const float v = acc * sa[m] * sw[n];
    if (y_bf16) static_cast<uint16_t *>(Y)[idx] = f32_to_bf16_rne(v);
    else static_cast<float *>(Y)[idx] = v;
}

// devices (bit = device ordinal < 64) on which the kernel's dynamic-LDS limit has been raised
std::atomic<uint64_t> lds_attr_devices{0};

}  // namespace
}  // namespace cfh

using namespace cfh;

extern "C" int32_t castforge_hip_gemm_fp8(const uint8_t *qa, const float *sa, int64_t m,
                                          const uint8_t *qw, const float *sw, int64_t n, int64_t k,
                                          void *y, int32_t y_dtype, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(m >= 0 && n >= 0 && k >= 0, "m, n, k must be non-negative");
        if (m == 0 || n == 0) return;
        require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
        require(qa && sa && qw && sw && y, "buffers must not be NULL");
        const int yb = y_dtype == CFH_DTYPE_BF16;
        require(m <= 0x7fffffff && n <= 0x7fffffff && k <= 0x7fffffff, "dimensions must fit in int32");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const bool fast = k > 0 && k % BK == 0 && aligned(qa, 16) && aligned(qw, 16);
        if (fast) {
            int dev = 0;
            check_hip(hipGetDevice(&dev), "hipGetDevice");
            const uint64_t bit = dev < 64 ? (uint64_t{1} << dev) : 0;
            if (bit == 0 || !(lds_attr_devices.load(std::memory_order_acquire) & bit)) {
                check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(fp8_gemm_kernel),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes),
                          "hipFuncSetAttribute(fp8_gemm_kernel)");
                lds_attr_devices.fetch_or(bit, std::memory_order_acq_rel);
            }
            const int tiles_m = static_cast<int>((m + BM - 1) / BM), tiles_n = static_cast<int>((n + BN - 1) / BN);
            fp8_gemm_kernel<<<dim3(tiles_m * tiles_n), dim3(kThreads), kLdsBytes, st>>>(
                qa, sa, qw, sw, y, yb, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k),
                tiles_m, tiles_n);
            check_launch("fp8_gemm");
        } else {
            const int64_t tot = m * n;
            require((tot + 255) / 256 <= 0x7fffffff, "shape too large for the generic FP8 kernel");
            fp8_gemm_generic_kernel<<<dim3(static_cast<unsigned>((tot + 255) / 256)), dim3(256), 0, st>>>(
                qa, sa, qw, sw, y, yb, m, n, k);
            check_launch("fp8_gemm_generic");
        }
    });
}
