// Elementwise steps around the dequant-fused matmul, on gfx950:
//   * the `castforge.fused_qmatmul` epilogue (codegen/eval.rs:1151-1176): bias add, then
//     relu / tanh / silu / gelu / scale, applied in place to the f32 GEMM output;
//   * f32 <-> bf16 conversion of activations (the bf16 operands `lower-mixed-precision`
//     introduces, passes/quantize/formats.rs:563-591);
//   * the [K, N] -> [N, K] transpose of `pack-weights` (passes/weights/fold.rs:549-554), also
//     used for i8 codes of an unpacked right-hand side;
//   * eval_matmul_2d (codegen/eval.rs:1465-1507) for f32 operands: one thread per output, k in
//     ascending order with a separate multiply and add, so the result is bit-identical to the
//     reference interpreter's (the evaluator's unfused dot_general; not the fused hot path).
// Built with -ffp-contract=off so the epilogue's f32 operations keep the evaluator's order;
// tanhf / expf are the device library's (within a few ulp of the host libm the reference uses).
#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

constexpr int kBlock = 256;

// eval.rs:1733-1735, same operation order.
__device__ __forceinline__ float gelu_tanh(float x) {
    const float inner = x + 0.044715f * x * x * x;
    return 0.5f * x * (1.0f + tanhf(0.7978846f * inner));
}

__global__ __launch_bounds__(kBlock) void epilogue_kernel(float *__restrict__ y, int64_t count,
                                                         const float *__restrict__ bias, int64_t blen,
                                                         const float *__restrict__ z, int64_t zlen, int kind) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count; i += stride) {
        const float val = y[i] + bias[i % blen];
        const float zi = zlen > 0 ? z[i % zlen] : 0.0f;
        float r;
        switch (kind) {
            case CFH_EPI_RELU: r = fmaxf(val, zi); break;  // f32::max ignores NaN
            case CFH_EPI_TANH: r = tanhf(val); break;
            case CFH_EPI_SILU: r = val / (1.0f + expf(-val)); break;
            case CFH_EPI_GELU: r = gelu_tanh(val); break;
            case CFH_EPI_SCALE: r = val * zi; break;
            default: r = val; break;
        }
        y[i] = r;
    }
}

__global__ __launch_bounds__(kBlock) void f32_to_bf16_kernel(const float *__restrict__ src, int64_t n,
                                                            uint16_t *__restrict__ dst) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        dst[i] = f32_to_bf16_rne(src[i]);
}

__global__ __launch_bounds__(kBlock) void bf16_to_f32_kernel(const uint16_t *__restrict__ src, int64_t n,
                                                            float *__restrict__ dst) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        dst[i] = bf16_to_f32(src[i]);
}

// 64 x 64 tiles through LDS (one padding element per row: no bank conflicts on the
// transposed reads); T is the element type (1, 2 or 4 bytes).
template <typename T>
__global__ __launch_bounds__(kBlock) void transpose_kernel(const T *__restrict__ src, int64_t rows,
                                                          int64_t cols, T *__restrict__ dst) {
    __shared__ T t[64][65];
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += kBlock / 64) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < rows && c < cols) t[i][tx] = src[r * cols + c];
    }
    __syncthreads();
    for (int i = ty; i < 64; i += kBlock / 64) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (r < rows && c < cols) dst[c * rows + r] = t[tx][i];
    }
}

__global__ __launch_bounds__(kBlock) void matmul_f32_kernel(const float *__restrict__ a, int64_t m, int64_t k,
                                                           const float *__restrict__ b, int64_t n, int packed,
                                                           float *__restrict__ out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; idx < m * n; idx += stride) {
        const int64_t row = idx / n, col = idx - row * n;
        float acc = 0.0f;
        for (int64_t kk = 0; kk < k; ++kk) {
            const float bv = packed ? b[col * k + kk] : b[kk * n + col];
            acc += a[row * k + kk] * bv;
        }
        out[idx] = acc;
    }
}

unsigned grid_for(int64_t n) {
    const int64_t b = (n + kBlock - 1) / kBlock;
    return static_cast<unsigned>(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

// castforge.static_quantize (codegen/eval.rs:1369-1382): (x / sc).round().clamp(-qmax, qmax) * sc
// in f32; Rust's round is half away from zero (roundf) and its clamp lets NaN through.
__global__ __launch_bounds__(kBlock) void static_quantize_kernel(const float *__restrict__ x, int64_t n, float sc,
                                                                 float qmax, float *__restrict__ y) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const float r = roundf(x[i] / sc);
        const float c = r != r ? r : fminf(fmaxf(r, -qmax), qmax);
        y[i] = c * sc;
    }
}

}  // namespace
}  // namespace cfh

using namespace cfh;

extern "C" {

int32_t castforge_hip_qmatmul_epilogue(float *y, int64_t count, const float *bias, int64_t bias_len,
                                       const float *z, int64_t z_len, int32_t kind, void *stream,
                                       char **out_error) {
    return guarded(out_error, [&] {
        require(count >= 0 && bias_len >= 0 && z_len >= 0, "sizes must be non-negative");
        require(kind >= CFH_EPI_BIAS && kind <= CFH_EPI_SCALE, "unknown epilogue kind");
        if (count == 0) return;
        require(y && bias && bias_len > 0, "y and a non-empty bias are required");
        require(z_len == 0 || z, "z must not be NULL when z_len > 0");
        epilogue_kernel<<<grid_for(count), kBlock, 0, static_cast<hipStream_t>(stream)>>>(y, count, bias, bias_len,
                                                                                        z, z_len, kind);
        check_launch("epilogue");
    });
}

int32_t castforge_hip_static_quantize(const float *x, int64_t n, float scale, int32_t bits, float *y,
                                      void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(n >= 0, "n must be non-negative");
        require(scale > 0.0f && scale <= 3.4028235e38f, "scale must be positive and finite");
        if (n == 0) return;
        require(x && y, "x and y must not be NULL");
        static_quantize_kernel<<<grid_for(n), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
            x, n, scale, bits == 4 ? 7.0f : 127.0f, y);
        check_launch("static_quantize");
    });
}

int32_t castforge_hip_convert_f32_to_bf16(const float *src, int64_t n, uint16_t *dst, void *stream,
                                          char **out_error) {
    return guarded(out_error, [&] {
        require(n >= 0, "n must be non-negative");
        if (n == 0) return;
        require(src && dst, "src and dst must not be NULL");
        f32_to_bf16_kernel<<<grid_for(n), kBlock, 0, static_cast<hipStream_t>(stream)>>>(src, n, dst);
        check_launch("f32_to_bf16");
    });
}

int32_t castforge_hip_convert_bf16_to_f32(const uint16_t *src, int64_t n, float *dst, void *stream,
                                          char **out_error) {
    return guarded(out_error, [&] {
        require(n >= 0, "n must be non-negative");
        if (n == 0) return;
        require(src && dst, "src and dst must not be NULL");
        bf16_to_f32_kernel<<<grid_for(n), kBlock, 0, static_cast<hipStream_t>(stream)>>>(src, n, dst);
        check_launch("bf16_to_f32");
    });
}

int32_t castforge_hip_transpose(const void *src, int64_t rows, int64_t cols, int32_t elem_bytes, void *dst,
                                void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(rows >= 0 && cols >= 0, "rows and cols must be non-negative");
        require(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4, "elem_bytes must be 1, 2 or 4");
        if (rows == 0 || cols == 0) return;
        require(src && dst && src != dst, "src and dst must be distinct non-NULL buffers");
        const int64_t gx = (cols + 63) / 64, gy = (rows + 63) / 64;
        require(gx <= 0x7fffffff && gy <= 65535, "matrix too large for one launch");
        const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy));
        hipStream_t st = static_cast<hipStream_t>(stream);
        if (elem_bytes == 4)
            transpose_kernel<uint32_t><<<grid, kBlock, 0, st>>>(static_cast<const uint32_t *>(src), rows, cols,
                                                              static_cast<uint32_t *>(dst));
        else if (elem_bytes == 2)
            transpose_kernel<uint16_t><<<grid, kBlock, 0, st>>>(static_cast<const uint16_t *>(src), rows, cols,
                                                              static_cast<uint16_t *>(dst));
        else
            transpose_kernel<uint8_t><<<grid, kBlock, 0, st>>>(static_cast<const uint8_t *>(src), rows, cols,
                                                             static_cast<uint8_t *>(dst));
        check_launch("transpose");
    });
}

int32_t castforge_hip_matmul_f32(const float *a, int64_t m, int64_t k, const float *b, int64_t n,
                                 int32_t packed_rhs, float *out, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(m >= 0 && k >= 0 && n >= 0, "m, k, n must be non-negative");
        if (m == 0 || n == 0) return;
        require(out != nullptr && (k == 0 || (a && b)), "buffers must not be NULL");
        matmul_f32_kernel<<<grid_for(m * n), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
            a, m, k, b, n, packed_rhs ? 1 : 0, out);
        check_launch("matmul_f32");
    });
}

}  // extern "C"
