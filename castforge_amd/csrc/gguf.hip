// GGUF tensor payloads on the GPU, gfx950.
//
// Replaces the CPU element loops of the reference's GGUF reader and writer:
//   * decode_ggml_tensor (ir/formats/gguf.rs:486-550): F32 / F16 / BF16 arrays and the
//     32-element blocks Q4_0 (f16 d + 16 bytes, element 2j = low nibble of byte j, 2j+1 = high
//     nibble, value (nibble - 8) * d) and Q8_0 (f16 d + 32 int8, value q * d), blocks running
//     over the flattened tensor;
//   * the payload half of export_gguf_bytes (gguf.rs:280-322): Q8_0 blocks of a QuantizedI8
//     tensor (its one scale truncated to f16 in every block, gguf.rs:283-296) and the
//     truncating F16 / BF16 converters (ir/tensor_store.rs:84-111).
//
// It also converts the two block formats to and from the layout the dequant-fused GEMV reads
// ("GGUF planes"): a code plane and an f16 scale plane per matrix [N, K] whose blocks run
// along K, each row cut into chunks (Q4_0: 128 elements = 4 blocks = 64 bytes; Q8_0: 64
// elements = 2 blocks = 64 bytes) and each chunk stored as four 16-byte parts, part p holding
// elements 8p .. 8p+7 of every block of the chunk (Q4_0: 4 bytes per block, nibble order as
// in the block; Q8_0: 8 bytes per block).  One 16-byte load per lane then feeds one MFMA per
// block with the four lanes of a row covering exactly that block, so each block's f32 dot
// product is scaled by its own d.  Scales: f16 bits [N, GP], GP = 8 * ceil(K/32 / 8), pad 0.
//
// Everything here is byte movement plus an exact product ((nibble - 8) and q are small
// integers, d an f16: the f32 product is exact), so results equal the reference bit for bit;
// only NaN payloads may differ.
#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

constexpr int kBlock = 256;

// tensor_store.rs:59-82 without relying on the hardware's f16 denormal mode: exact for every
// input, NaN payload kept unquieted.
__device__ __forceinline__ float f16_exact(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1fu) return __uint_as_float(sign | 0x7f800000u | (m << 13));
    if (e == 0u) return __uint_as_float(sign | __float_as_uint(static_cast<float>(m) * 0x1p-24f));
    return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

// tensor_store.rs:84-102: f16 by mantissa truncation, overflow to Inf, underflow to signed 0,
// NaN to 0x7E00 with the sign.
__host__ __device__ inline uint16_t f16_trunc(float v) {
    uint32_t bits;
    memcpy(&bits, &v, 4);
    const uint16_t sign = static_cast<uint16_t>((bits >> 16) & 0x8000u);
    const int32_t exp = static_cast<int32_t>((bits >> 23) & 0xffu);
    const uint32_t mant = bits & 0x7fffffu;
    if (exp == 255) return sign | 0x7c00u | (mant != 0 ? 0x0200u : 0u);
    const int32_t ne = exp - 127 + 15;
    if (ne >= 31) return sign | 0x7c00u;
    if (ne <= 0) return sign;
    return sign | static_cast<uint16_t>(ne << 10) | static_cast<uint16_t>(mant >> 13);
}

__device__ __forceinline__ uint32_t ld16(const uint8_t *p) {
    return *reinterpret_cast<const uint16_t *>(p);  // p is 2-byte aligned
}
__device__ __forceinline__ uint32_t ld32_a2(const uint8_t *p) {  // 4 bytes at a 2-aligned address
    return ld16(p) | (ld16(p + 2) << 16);
}
__device__ __forceinline__ void st32_a2(uint8_t *p, uint32_t v) {
    reinterpret_cast<uint16_t *>(p)[0] = static_cast<uint16_t>(v);
    reinterpret_cast<uint16_t *>(p)[1] = static_cast<uint16_t>(v >> 16);
}

// Eight consecutive outputs starting at e (8-aligned); the tail of the tensor is written
// element by element.
template <bool VEC>
__device__ __forceinline__ void store8(float *out, int64_t e, int64_t n, const float (&v)[8]) {
    if (VEC && e + 8 <= n) {
        float4 *o = reinterpret_cast<float4 *>(out + e);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (e + i < n) out[e + i] = v[i];
    }
}

// One thread per 8 consecutive elements (a quarter of a 32-element block).
template <int TYPE, bool VEC>
__global__ __launch_bounds__(kBlock) void gguf_decode_kernel(const uint8_t *raw, int64_t n, float *out) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t e = t * 8;
    if (e >= n) return;
    float v[8];
    if constexpr (TYPE == CFH_GGML_Q4_0) {
        const uint8_t *blk = raw + (t >> 2) * 18;
        const float d = f16_exact(ld16(blk));
        const uint32_t w = ld32_a2(blk + 2 + 4 * (t & 3));
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = static_cast<float>(static_cast<int32_t>((w >> (4 * i)) & 15u) - 8) * d;
    } else if constexpr (TYPE == CFH_GGML_Q8_0) {
        const uint8_t *blk = raw + (t >> 2) * 34;
        const float d = f16_exact(ld16(blk));
        const uint32_t w0 = ld32_a2(blk + 2 + 8 * (t & 3)), w1 = ld32_a2(blk + 6 + 8 * (t & 3));
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = static_cast<float>(static_cast<int8_t>(((i < 4 ? w0 : w1) >> (8 * (i & 3))) & 0xffu)) * d;
    } else if constexpr (TYPE == CFH_GGML_F32) {
        const uint32_t *s = reinterpret_cast<const uint32_t *>(raw) + e;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = e + i < n ? __uint_as_float(s[i]) : 0.0f;
    } else {
        const uint16_t *s = reinterpret_cast<const uint16_t *>(raw) + e;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t h = e + i < n ? s[i] : 0u;
            v[i] = TYPE == CFH_GGML_F16 ? f16_exact(h) : __uint_as_float(h << 16);
        }
    }
    store8<VEC>(out, e, n, v);
}

// Q8_0 blocks of a QuantizedI8 tensor, one thread per block; codes past n are 0.
__global__ __launch_bounds__(kBlock) void gguf_encode_q8_0_kernel(const int8_t *codes, int64_t n,
                                                                  int64_t blocks, uint32_t d_bits,
                                                                  uint8_t *raw) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (b >= blocks) return;
    uint8_t *blk = raw + b * 34;
    reinterpret_cast<uint16_t *>(blk)[0] = static_cast<uint16_t>(d_bits);
    const int64_t e0 = b * 32;
#pragma unroll
    for (int j = 0; j < 32; j += 2) {
        const uint32_t lo = e0 + j < n ? static_cast<uint8_t>(codes[e0 + j]) : 0u;
        const uint32_t hi = e0 + j + 1 < n ? static_cast<uint8_t>(codes[e0 + j + 1]) : 0u;
        reinterpret_cast<uint16_t *>(blk + 2)[j >> 1] = static_cast<uint16_t>(lo | (hi << 8));
    }
}

// F16 / BF16 payloads of f32 values with the reference's truncating converters.
template <int TYPE>
__global__ __launch_bounds__(kBlock) void gguf_encode_half_kernel(const float *src, int64_t n, uint16_t *raw) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    raw[i] = TYPE == CFH_GGML_F16 ? f16_trunc(src[i]) : static_cast<uint16_t>(__float_as_uint(src[i]) >> 16);
}

// Blocks -> planes.  One thread per (row, chunk, part): Q4_0 gathers 4 bytes of each of the
// chunk's 4 blocks, Q8_0 8 bytes of each of its 2 blocks, and stores one 16-byte part; part 0
// also stores the chunk's scales, and the last chunk's part 1 the row's scale padding.
template <int TYPE>
__global__ __launch_bounds__(kBlock) void gguf_repack_kernel(const uint8_t *raw, int64_t rows, int64_t k,
                                                             uint8_t *codes, uint16_t *scales) {
    constexpr int BPC = TYPE == CFH_GGML_Q4_0 ? 4 : 2;   // blocks per chunk
    constexpr int BB = TYPE == CFH_GGML_Q4_0 ? 18 : 34;  // bytes per block
    constexpr int PB = 16 / BPC;                         // bytes per block and part
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t chunks = k / (32 * BPC);
    if (t >= rows * chunks * 4) return;
    const int p = static_cast<int>(t & 3);
    const int64_t c = (t >> 2) % chunks, r = (t >> 2) / chunks;
    const int64_t G = k / 32, GP = (G + 7) / 8 * 8;
    const uint8_t *b0 = raw + (r * G + c * BPC) * BB;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < BPC; ++j) {
        const uint8_t *src = b0 + j * BB + 2 + PB * p;
        if constexpr (BPC == 4) {
            w[j] = ld32_a2(src);
        } else {
            w[2 * j] = ld32_a2(src);
            w[2 * j + 1] = ld32_a2(src + 4);
        }
    }
    const int64_t row_bytes = TYPE == CFH_GGML_Q4_0 ? k / 2 : k;
    *reinterpret_cast<uint4 *>(codes + r * row_bytes + c * 64 + 16 * p) = make_uint4(w[0], w[1], w[2], w[3]);
    uint16_t *srow = scales + r * GP;
    if (p == 0) {
#pragma unroll
        for (int j = 0; j < BPC; ++j) srow[c * BPC + j] = static_cast<uint16_t>(ld16(b0 + j * BB));
    } else if (p == 1 && c == chunks - 1) {
        for (int64_t g = G; g < GP; ++g) srow[g] = 0;
    }
}

// Planes -> blocks (the inverse of gguf_repack_kernel).
template <int TYPE>
__global__ __launch_bounds__(kBlock) void gguf_unpack_kernel(const uint8_t *codes, const uint16_t *scales,
                                                             int64_t rows, int64_t k, uint8_t *raw) {
    constexpr int BPC = TYPE == CFH_GGML_Q4_0 ? 4 : 2;
    constexpr int BB = TYPE == CFH_GGML_Q4_0 ? 18 : 34;
    constexpr int PB = 16 / BPC;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t chunks = k / (32 * BPC);
    if (t >= rows * chunks * 4) return;
    const int p = static_cast<int>(t & 3);
    const int64_t c = (t >> 2) % chunks, r = (t >> 2) / chunks;
    const int64_t G = k / 32, GP = (G + 7) / 8 * 8;
    const int64_t row_bytes = TYPE == CFH_GGML_Q4_0 ? k / 2 : k;
    const uint4 v = *reinterpret_cast<const uint4 *>(codes + r * row_bytes + c * 64 + 16 * p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint8_t *b0 = raw + (r * G + c * BPC) * BB;
#pragma unroll
    for (int j = 0; j < BPC; ++j) {
        uint8_t *dst = b0 + j * BB + 2 + PB * p;
        if constexpr (BPC == 4) {
            st32_a2(dst, w[j]);
        } else {
            st32_a2(dst, w[2 * j]);
            st32_a2(dst + 4, w[2 * j + 1]);
        }
        if (p == 0) reinterpret_cast<uint16_t *>(b0 + j * BB)[0] = scales[r * GP + c * BPC + j];
    }
}

// Planes -> f32 [rows, k]: one thread per (row, chunk, part), 8 elements per block.
template <int TYPE>
__global__ __launch_bounds__(kBlock) void gguf_planes_dequant_kernel(const uint8_t *codes, const uint16_t *scales,
                                                                     int64_t rows, int64_t k, float *out) {
    constexpr int BPC = TYPE == CFH_GGML_Q4_0 ? 4 : 2;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t chunks = k / (32 * BPC);
    if (t >= rows * chunks * 4) return;
    const int p = static_cast<int>(t & 3);
    const int64_t c = (t >> 2) % chunks, r = (t >> 2) / chunks;
    const int64_t G = k / 32, GP = (G + 7) / 8 * 8;
    const int64_t row_bytes = TYPE == CFH_GGML_Q4_0 ? k / 2 : k;
    const uint4 v = *reinterpret_cast<const uint4 *>(codes + r * row_bytes + c * 64 + 16 * p);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < BPC; ++j) {
        const float d = f16_exact(scales[r * GP + c * BPC + j]);
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if constexpr (BPC == 4)
                o[i] = static_cast<float>(static_cast<int32_t>((w[j] >> (4 * i)) & 15u) - 8) * d;
            else
                o[i] = static_cast<float>(static_cast<int8_t>((w[2 * j + (i >> 2)] >> (8 * (i & 3))) & 0xffu)) * d;
        }
        float4 *dst = reinterpret_cast<float4 *>(out + r * k + c * 32 * BPC + 32 * j + 8 * p);
        dst[0] = make_float4(o[0], o[1], o[2], o[3]);
        dst[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
}

// Q4_0 planes -> the INT4g layout (natural code order, group 32, zero point 8): one thread per
// (row, chunk, part); part p's word j is word p of the chunk's block j, which INT4g keeps at
// word 4j + p of the chunk.  The scale plane is shared as it is ([rows, GP] f16 in both).
__global__ __launch_bounds__(kBlock) void gguf_q4_to_int4g_kernel(const uint8_t *codes, int64_t rows, int64_t k,
                                                                  uint32_t *out, uint32_t *zeros) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t chunks = k / 128;
    if (t >= rows * chunks * 4) return;
    const int p = static_cast<int>(t & 3);
    const int64_t c = (t >> 2) % chunks, r = (t >> 2) / chunks;
    const uint4 v = *reinterpret_cast<const uint4 *>(codes + r * (k / 2) + c * 64 + 16 * p);
    uint32_t *o = out + r * (k / 8) + c * 16 + p;
    o[0] = v.x;
    o[4] = v.y;
    o[8] = v.z;
    o[12] = v.w;
    if (t % (chunks * 4) == 0) {
        const int64_t zw = (k / 32 + 7) / 8;
        for (int64_t i = 0; i < zw; ++i) zeros[r * zw + i] = 0x88888888u;
    }
}

unsigned grid_for(int64_t threads) {
    const int64_t g = (threads + kBlock - 1) / kBlock;
    require(g <= 0x7fffffff, "tensor too large for one launch");
    return static_cast<unsigned>(g);
}

bool is_block_type(int32_t t) { return t == CFH_GGML_Q4_0 || t == CFH_GGML_Q8_0; }

// Payload bytes of num_elems elements of a GGUF type (gguf.rs:491-550).
int64_t payload_bytes(int32_t t, int64_t n) {
    if (t == CFH_GGML_Q4_0) return (n + 31) / 32 * 18;
    if (t == CFH_GGML_Q8_0) return (n + 31) / 32 * 34;
    if (t == CFH_GGML_F32) return n * 4;
    return n * 2;
}

void check_planes(int32_t t, int64_t rows, int64_t k, const void *codes, const void *scales) {
    require(is_block_type(t), "ggml_type must be CFH_GGML_Q4_0 or CFH_GGML_Q8_0");
    require(rows >= 0 && k >= 0, "rows and k must be non-negative");
    const int64_t ck = t == CFH_GGML_Q4_0 ? 128 : 64;
    require(k % ck == 0, t == CFH_GGML_Q4_0 ? "Q4_0 planes need k % 128 == 0" : "Q8_0 planes need k % 64 == 0");
    if (rows > 0 && k > 0) {
        require(codes && scales, "codes and scales must not be NULL");
        require(aligned(codes, 16) && aligned(scales, 16), "codes and scales must be 16-byte aligned");
    }
}

}  // namespace

// f16 bits of a scale by the reference's truncating converter (shared with the exporter).
uint16_t gguf_f16_trunc_host(float v) { return f16_trunc(v); }

}  // namespace cfh

using namespace cfh;

extern "C" {

int32_t castforge_hip_gguf_payload_bytes(int32_t ggml_type, int64_t num_elems, int64_t *out_bytes,
                                         char **out_error) {
    return guarded(out_error, [&] {
        require(out_bytes != nullptr, "out_bytes must not be NULL");
        *out_bytes = 0;
        require(ggml_type == CFH_GGML_F32 || ggml_type == CFH_GGML_F16 || ggml_type == CFH_GGML_BF16 ||
                    is_block_type(ggml_type),
                "Unsupported GGML tensor type id: " + std::to_string(ggml_type));
        require(num_elems >= 0, "num_elems must be non-negative");
        *out_bytes = payload_bytes(ggml_type, num_elems);
    });
}

int32_t castforge_hip_gguf_decode(int32_t ggml_type, const void *raw, int64_t num_elems, float *out,
                                  void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(num_elems >= 0, "num_elems must be non-negative");
        require(ggml_type == CFH_GGML_F32 || ggml_type == CFH_GGML_F16 || ggml_type == CFH_GGML_BF16 ||
                    is_block_type(ggml_type),
                "Unsupported GGML tensor type id: " + std::to_string(ggml_type));
        if (num_elems == 0) return;
        require(raw && out, "raw and out must not be NULL");
        require(aligned(raw, ggml_type == CFH_GGML_F32 ? 4 : 2),
                "raw must be 4-byte (F32) or 2-byte (other types) aligned");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const unsigned g = grid_for((num_elems + 7) / 8);
        const uint8_t *r = static_cast<const uint8_t *>(raw);
        const bool vec = aligned(out, 16);
#define CFH_DECODE(T)                                                                        \
    do {                                                                                     \
        if (vec) gguf_decode_kernel<T, true><<<g, kBlock, 0, st>>>(r, num_elems, out);        \
        else gguf_decode_kernel<T, false><<<g, kBlock, 0, st>>>(r, num_elems, out);           \
    } while (0)
        switch (ggml_type) {
        case CFH_GGML_Q4_0: CFH_DECODE(CFH_GGML_Q4_0); break;
        case CFH_GGML_Q8_0: CFH_DECODE(CFH_GGML_Q8_0); break;
        case CFH_GGML_F32: CFH_DECODE(CFH_GGML_F32); break;
        case CFH_GGML_F16: CFH_DECODE(CFH_GGML_F16); break;
        default: CFH_DECODE(CFH_GGML_BF16); break;
        }
#undef CFH_DECODE
        check_launch("gguf_decode");
    });
}

int32_t castforge_hip_gguf_encode(int32_t ggml_type, const void *src, int64_t num_elems, float scale,
                                  void *raw_out, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(num_elems >= 0, "num_elems must be non-negative");
        require(ggml_type == CFH_GGML_F32 || ggml_type == CFH_GGML_F16 || ggml_type == CFH_GGML_BF16 ||
                    ggml_type == CFH_GGML_Q8_0,
                "ggml_type must be CFH_GGML_F32, F16, BF16 or Q8_0");
        hipStream_t st = static_cast<hipStream_t>(stream);
        if (ggml_type == CFH_GGML_Q8_0) {
            // gguf.rs:285: max(n, 1) elements, so an empty tensor still writes one zero block
            const int64_t blocks = ((num_elems > 1 ? num_elems : 1) + 31) / 32;
            require(raw_out != nullptr, "raw_out must not be NULL");
            require(aligned(raw_out, 2), "raw_out must be 2-byte aligned");
            require(num_elems == 0 || src != nullptr, "src must not be NULL");
            gguf_encode_q8_0_kernel<<<grid_for(blocks), kBlock, 0, st>>>(
                static_cast<const int8_t *>(src), num_elems, blocks, f16_trunc(scale), static_cast<uint8_t *>(raw_out));
            check_launch("gguf_encode_q8_0");
            return;
        }
        if (num_elems == 0) return;
        require(src && raw_out, "src and raw_out must not be NULL");
        if (ggml_type == CFH_GGML_F32) {
            check_hip(hipMemcpyAsync(raw_out, src, static_cast<size_t>(num_elems) * 4, hipMemcpyDeviceToDevice, st),
                      "gguf_encode (F32 copy)");
            return;
        }
        require(aligned(raw_out, 2) && aligned(src, 4), "raw_out must be 2-byte and src 4-byte aligned");
        const unsigned g = grid_for(num_elems);
        if (ggml_type == CFH_GGML_F16)
            gguf_encode_half_kernel<CFH_GGML_F16><<<g, kBlock, 0, st>>>(static_cast<const float *>(src), num_elems,
                                                                        static_cast<uint16_t *>(raw_out));
        else
            gguf_encode_half_kernel<CFH_GGML_BF16><<<g, kBlock, 0, st>>>(static_cast<const float *>(src), num_elems,
                                                                         static_cast<uint16_t *>(raw_out));
        check_launch("gguf_encode_half");
    });
}

int32_t castforge_hip_gguf_repack(int32_t ggml_type, const void *raw, int64_t rows, int64_t k, void *codes,
                                  uint16_t *scales_f16, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        check_planes(ggml_type, rows, k, codes, scales_f16);
        if (rows == 0 || k == 0) return;
        require(raw != nullptr && aligned(raw, 2), "raw must not be NULL and must be 2-byte aligned");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const int64_t threads = rows * (k / (ggml_type == CFH_GGML_Q4_0 ? 128 : 64)) * 4;
        const unsigned g = grid_for(threads);
        const uint8_t *r = static_cast<const uint8_t *>(raw);
        if (ggml_type == CFH_GGML_Q4_0)
            gguf_repack_kernel<CFH_GGML_Q4_0><<<g, kBlock, 0, st>>>(r, rows, k, static_cast<uint8_t *>(codes), scales_f16);
        else
            gguf_repack_kernel<CFH_GGML_Q8_0><<<g, kBlock, 0, st>>>(r, rows, k, static_cast<uint8_t *>(codes), scales_f16);
        check_launch("gguf_repack");
    });
}

int32_t castforge_hip_gguf_unpack(int32_t ggml_type, const void *codes, const uint16_t *scales_f16, int64_t rows,
                                  int64_t k, void *raw_out, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        check_planes(ggml_type, rows, k, codes, scales_f16);
        if (rows == 0 || k == 0) return;
        require(raw_out != nullptr && aligned(raw_out, 2), "raw_out must not be NULL and must be 2-byte aligned");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const int64_t threads = rows * (k / (ggml_type == CFH_GGML_Q4_0 ? 128 : 64)) * 4;
        const unsigned g = grid_for(threads);
        const uint8_t *c = static_cast<const uint8_t *>(codes);
        if (ggml_type == CFH_GGML_Q4_0)
            gguf_unpack_kernel<CFH_GGML_Q4_0><<<g, kBlock, 0, st>>>(c, scales_f16, rows, k, static_cast<uint8_t *>(raw_out));
        else
            gguf_unpack_kernel<CFH_GGML_Q8_0><<<g, kBlock, 0, st>>>(c, scales_f16, rows, k, static_cast<uint8_t *>(raw_out));
        check_launch("gguf_unpack");
    });
}

int32_t castforge_hip_gguf_q4_0_to_int4g(const void *codes, int64_t rows, int64_t k, uint32_t *int4_codes,
                                         uint32_t *zeros, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(rows >= 0 && k >= 0 && k % 128 == 0, "Q4_0 planes need k % 128 == 0");
        if (rows == 0 || k == 0) return;
        require(codes && int4_codes && zeros, "buffers must not be NULL");
        require(aligned(codes, 16) && aligned(int4_codes, 4) && aligned(zeros, 4),
                "codes must be 16-byte, int4_codes and zeros 4-byte aligned");
        gguf_q4_to_int4g_kernel<<<grid_for(rows * (k / 128) * 4), kBlock, 0, static_cast<hipStream_t>(stream)>>>(
            static_cast<const uint8_t *>(codes), rows, k, int4_codes, zeros);
        check_launch("gguf_q4_to_int4g");
    });
}

int32_t castforge_hip_dequantize_gguf(int32_t ggml_type, const void *codes, const uint16_t *scales_f16,
                                      int64_t rows, int64_t k, float *out, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        check_planes(ggml_type, rows, k, codes, scales_f16);
        if (rows == 0 || k == 0) return;
        require(out != nullptr && aligned(out, 16), "out must not be NULL and must be 16-byte aligned");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const int64_t threads = rows * (k / (ggml_type == CFH_GGML_Q4_0 ? 128 : 64)) * 4;
        const unsigned g = grid_for(threads);
        const uint8_t *c = static_cast<const uint8_t *>(codes);
        if (ggml_type == CFH_GGML_Q4_0)
            gguf_planes_dequant_kernel<CFH_GGML_Q4_0><<<g, kBlock, 0, st>>>(c, scales_f16, rows, k, out);
        else
            gguf_planes_dequant_kernel<CFH_GGML_Q8_0><<<g, kBlock, 0, st>>>(c, scales_f16, rows, k, out);
        check_launch("gguf_planes_dequant");
    });
}

}  // extern "C"
