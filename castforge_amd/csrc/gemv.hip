// Dequant-fused GEMV / skinny GEMM (M <= 16) for packed INT4 / INT8 / NF4 weights, gfx950.
//
// Replaces the evaluation of `castforge.fused_qmatmul` (eval.rs:1145-1179 with
// eval_matmul_2d, eval.rs:1465-1507) and the one-thread-per-row HIP text the reference emits
// for it (gpu_c.rs:208-292): out[m, n] = sum_k x[m, k] * dequant(W)[n, k], W stored [N, K]
// row-major (packed_rhs layout, fold.rs:549-554).
//
// Decode is HBM-bound on the packed weight stream.  Design:
//   * a workgroup (4 waves) owns 16 weight rows; the 4 waves split K;
//   * each lane streams 16 B of one row per load (lane%16 = row, lane/16 = 16-byte part), so a
//     wave-wide load covers 64 B of each of 16 rows: one 128-element INT4 group per row;
//   * codes become exact f16 values (q - z) with the magic-exponent trick (or an LDS table
//     for NF4) and feed v_mfma_f32_16x16x32_f16 as the B operand; the activation rows are
//     the A operand, converted once per workgroup from bf16 to f16 in LDS, in the permuted
//     order the nibble extraction produces, so M = 1..16 costs the same MFMA count;
//   * INT4 group scales (one per row per 128-k chunk) multiply the fp32 chunk result;
//     NF4 block scales (64 k) are folded into the f16 operand; INT8 scales are per row.
#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kLdsBytesMax = 32768;  // activation stage per workgroup
constexpr int kMaxProblems = 8;

enum Fmt { FMT_INT4 = 0, FMT_INT8 = 1, FMT_NF4 = 2 };

struct Problem {
    const uint16_t *x;      // bf16 [M, K]
    const void *codes;      // INT4/NF4: u32 [N, K/8]; INT8: i8 [N, K]
    const void *scales;     // INT4: f16 [N, G]; INT8: f32 [N] or [1]; NF4: f32 [N, K/block]
    const uint32_t *zeros;  // INT4: u32 [N, ceil(G/8)]
    void *y;                // [M, N] f32 or bf16
    int64_t n, k;
    int32_t group;          // INT4 group / NF4 block
    int32_t scale_per_row;  // INT8: 1 per-channel, 0 per-tensor
    int32_t tile_begin;     // first workgroup index of this problem
    int32_t kc;             // K elements staged per LDS pass
};

struct Batch {
    Problem p[kMaxProblems];
    int32_t count;
    int32_t m;
    int32_t y_bf16;
};

// Chunk = the K span one wave-wide 16-byte-per-lane load covers for each of the 16 rows.
template <int FMT> struct FmtTraits;
template <> struct FmtTraits<FMT_INT4> { static constexpr int kChunk = 128; };
template <> struct FmtTraits<FMT_NF4> { static constexpr int kChunk = 128; };
template <> struct FmtTraits<FMT_INT8> { static constexpr int kChunk = 64; };

// Position, within each 8-element k-run, of the element the extraction places in f16 slot i.
// INT4: (n0,n4),(n1,n5),(n2,n6),(n3,n7); INT8 (two words): (b0,b2),(b1,b3) of each word.
__device__ __forceinline__ int perm_src(int fmt, int i) {
    if (fmt == FMT_INT4) return (i >> 1) + ((i & 1) << 2);
    if (fmt == FMT_INT8) return ((i >> 2) << 2) + ((i >> 1) & 1) + ((i & 1) << 1);
    return i;
}

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// INT4 word -> 4 f16 pairs of exact (q - z).  zc1024 = -(1024+z) splat, zc64 = -(64+z) splat.
__device__ __forceinline__ void int4_word_to_h(uint32_t w, half2_t zc1024, half2_t zc64,
                                               uint32_t out[4]) {
    const half2_t sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    const uint32_t w8 = w >> 8;
    half2_t lo0 = as_h2((w & 0x000F000Fu) | 0x64006400u) + zc1024;
    half2_t hi0 = as_h2((w & 0x00F000F0u) | 0x64006400u) * sixteenth + zc64;
    half2_t lo1 = as_h2((w8 & 0x000F000Fu) | 0x64006400u) + zc1024;
    half2_t hi1 = as_h2((w8 & 0x00F000F0u) | 0x64006400u) * sixteenth + zc64;
    out[0] = as_u(lo0);
    out[1] = as_u(hi0);
    out[2] = as_u(lo1);
    out[3] = as_u(hi1);
}

// INT8 word (4 signed codes) -> 2 f16 pairs of exact q.
__device__ __forceinline__ void int8_word_to_h(uint32_t w, uint32_t out[2]) {
    const half2_t c1152 = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    const uint32_t u = w ^ 0x80808080u;
    out[0] = as_u(as_h2((u & 0x00FF00FFu) | 0x64006400u) + c1152);
    out[1] = as_u(as_h2(((u >> 8) & 0x00FF00FFu) | 0x64006400u) + c1152);
}

__device__ __forceinline__ half8_t pack8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    uint4 v = make_uint4(a, b, c, d);
    return __builtin_bit_cast(half8_t, v);
}

__constant__ float kNf4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

template <int FMT>
__global__ __launch_bounds__(kThreads) void skinny_qgemm_kernel(Batch b) {
    using Tr = FmtTraits<FMT>;
    extern __shared__ __align__(16) _Float16 xs[];  // [M][KC], permuted per 8-run
    __shared__ floatx4 red[kWaves - 1][64];
    __shared__ uint32_t nf4_lut[FMT == FMT_NF4 ? 256 : 1];

    // locate the problem of this workgroup
    int pi = 0;
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
        if (i < b.count && static_cast<int>(blockIdx.x) >= b.p[i].tile_begin) pi = i;
    const Problem &P = b.p[pi];
    const int M = b.m;
    const int64_t N = P.n, K = P.k;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x - P.tile_begin) * 16;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, part = lane >> 4;
    const int64_t nrow = n0 + lr;
    const bool row_ok = nrow < N;

    if constexpr (FMT == FMT_NF4) {
        for (int i = tid; i < 256; i += kThreads) {
            half2_t v = {static_cast<_Float16>(kNf4[i & 15]), static_cast<_Float16>(kNf4[i >> 4])};
            nf4_lut[i] = as_u(v);
        }
    }

    const int64_t row_bytes = (FMT == FMT_INT8) ? K : K / 2;
    const uint8_t *wrow = static_cast<const uint8_t *>(P.codes) + (row_ok ? nrow : 0) * row_bytes;
    const int64_t G = (FMT == FMT_INT4) ? (K + P.group - 1) / P.group : 0;
    const int64_t ZW = (G + 7) / 8;

    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const int KC = P.kc;

    for (int64_t k0 = 0; k0 < K; k0 += KC) {
        const int kc = static_cast<int>((K - k0) < KC ? (K - k0) : KC);
        // ---- stage x[:, k0:k0+kc] as permuted f16 ----
        __syncthreads();
        const int runs = kc >> 3;
        for (int it = tid; it < M * runs; it += kThreads) {
            const int m = it / runs, r = it - m * runs;
            const uint4 raw = *reinterpret_cast<const uint4 *>(P.x + static_cast<int64_t>(m) * K + k0 + r * 8);
            const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
            uint32_t o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int s0 = perm_src(FMT, 2 * i), s1 = perm_src(FMT, 2 * i + 1);
                const uint16_t b0 = static_cast<uint16_t>(wv[s0 >> 1] >> (16 * (s0 & 1)));
                const uint16_t b1 = static_cast<uint16_t>(wv[s1 >> 1] >> (16 * (s1 & 1)));
                half2_t h = {static_cast<_Float16>(bf16_to_f32(b0)), static_cast<_Float16>(bf16_to_f32(b1))};
                o[i] = as_u(h);
            }
            *reinterpret_cast<uint4 *>(xs + m * KC + r * 8) = make_uint4(o[0], o[1], o[2], o[3]);
        }
        __syncthreads();

        // ---- stream this stage's chunks; wave w takes chunks w, w+4, ... ----
        const int nchunks = kc / Tr::kChunk;
        constexpr int NB = 4;  // chunks in flight per wave
        for (int cb = wave; cb < nchunks; cb += kWaves * NB) {
            uint4 wq[NB];
            float sc[NB];
            uint32_t zw[NB];
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int c = cb + j * kWaves;
                wq[j] = make_uint4(0, 0, 0, 0);
                sc[j] = 0.f;
                zw[j] = 0;
                if (c < nchunks && row_ok) {
                    const int64_t kk = k0 + static_cast<int64_t>(c) * Tr::kChunk;
                    const int64_t boff = (FMT == FMT_INT8 ? kk : kk / 2) + part * 16;
                    wq[j] = *reinterpret_cast<const uint4 *>(wrow + boff);
                    if constexpr (FMT == FMT_INT4) {
                        const int64_t g = kk / P.group;
                        sc[j] = f16_to_f32(static_cast<const uint16_t *>(P.scales)[nrow * G + g]);
                        zw[j] = (P.zeros[nrow * ZW + (g >> 3)] >> (4 * (g & 7))) & 15u;
                    } else if constexpr (FMT == FMT_NF4) {
                        const int64_t nb = (K + P.group - 1) / P.group;
                        sc[j] = static_cast<const float *>(P.scales)[nrow * nb + (kk + part * 32) / P.group];
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int c = cb + j * kWaves;
                if (c >= nchunks) break;
                const uint32_t ww[4] = {wq[j].x, wq[j].y, wq[j].z, wq[j].w};
                const int xoff = c * Tr::kChunk + part * (Tr::kChunk / 4);
                floatx4 part_acc = {0.f, 0.f, 0.f, 0.f};
                if constexpr (FMT == FMT_INT4) {
                    const _Float16 z1024 = static_cast<_Float16>(-1024.0f - static_cast<float>(zw[j]));
                    const _Float16 z64 = static_cast<_Float16>(-64.0f - static_cast<float>(zw[j]));
                    const half2_t zc1024 = {z1024, z1024}, zc64 = {z64, z64};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        uint32_t hb[4];
                        int4_word_to_h(ww[t], zc1024, zc64, hb);
                        half8_t bop = pack8(hb[0], hb[1], hb[2], hb[3]);
                        half8_t aop = {};
                        if (lr < M) aop = *reinterpret_cast<const half8_t *>(xs + lr * KC + xoff + t * 8);
                        part_acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, part_acc, 0, 0, 0);
                    }
                    acc += part_acc * sc[j];
                } else if constexpr (FMT == FMT_INT8) {
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        uint32_t h0[2], h1[2];
                        int8_word_to_h(ww[2 * t], h0);
                        int8_word_to_h(ww[2 * t + 1], h1);
                        half8_t bop = pack8(h0[0], h0[1], h1[0], h1[1]);
                        half8_t aop = {};
                        if (lr < M) aop = *reinterpret_cast<const half8_t *>(xs + lr * KC + xoff + t * 8);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, acc, 0, 0, 0);
                    }
                } else {
                    const _Float16 s16 = static_cast<_Float16>(sc[j]);
                    const half2_t s2 = {s16, s16};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const uint32_t w = ww[t];
                        uint32_t hb[4];
#pragma unroll
                        for (int q = 0; q < 4; ++q) hb[q] = as_u(as_h2(nf4_lut[(w >> (8 * q)) & 255u]) * s2);
                        half8_t bop = pack8(hb[0], hb[1], hb[2], hb[3]);
                        half8_t aop = {};
                        if (lr < M) aop = *reinterpret_cast<const half8_t *>(xs + lr * KC + xoff + t * 8);
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, acc, 0, 0, 0);
                    }
                }
            }
        }
    }

    // ---- reduce the 4 waves' partial tiles and store ----
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int w = 0; w < kWaves - 1; ++w) acc += red[w][lane];
        if constexpr (FMT == FMT_INT8) {
            if (row_ok) {
                const float *s = static_cast<const float *>(P.scales);
                acc *= P.scale_per_row ? s[nrow] : s[0];
            }
        }
        if (row_ok) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = part * 4 + r;
                if (m < M) {
                    if (b.y_bf16)
                        static_cast<uint16_t *>(P.y)[static_cast<int64_t>(m) * N + nrow] = f32_to_bf16_rne(acc[r]);
                    else
                        static_cast<float *>(P.y)[static_cast<int64_t>(m) * N + nrow] = acc[r];
                }
            }
        }
    }
}

// ---- generic fallback: any M, any group/block, K % 8 == 0 (f32 VALU, one wave per row) ----
template <int FMT>
__global__ __launch_bounds__(64) void generic_qgemm_kernel(Problem P, int M, int y_bf16) {
    const int64_t n = blockIdx.x;
    const int m0 = blockIdx.y * 8;
    const int lane = threadIdx.x;
    const int64_t K = P.k, N = P.n;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const int64_t G = (FMT == FMT_INT4) ? (K + P.group - 1) / P.group : 0, ZW = (G + 7) / 8;
    const int64_t NB = (FMT == FMT_NF4) ? (K + P.group - 1) / P.group : 0;
    for (int64_t k = lane; k < K; k += 64) {
        float w;
        if constexpr (FMT == FMT_INT8) {
            w = static_cast<float>(static_cast<const int8_t *>(P.codes)[n * K + k]);
        } else {
            const uint32_t word = static_cast<const uint32_t *>(P.codes)[n * (K / 8) + k / 8];
            const uint32_t q = (word >> (4 * (k & 7))) & 15u;
            if constexpr (FMT == FMT_INT4) {
                const int64_t g = k / P.group;
                const int32_t z = static_cast<int32_t>((P.zeros[n * ZW + (g >> 3)] >> (4 * (g & 7))) & 15u);
                w = static_cast<float>(static_cast<int32_t>(q) - z) *
                    f16_to_f32(static_cast<const uint16_t *>(P.scales)[n * G + g]);
            } else {
                w = kNf4[q] * static_cast<const float *>(P.scales)[n * NB + k / P.group];
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (m0 + i < M) acc[i] += bf16_to_f32(P.x[static_cast<int64_t>(m0 + i) * K + k]) * w;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = wave_sum<64>(acc[i]);
    if (lane == 0) {
        float s = 1.0f;
        if constexpr (FMT == FMT_INT8) {
            const float *sp = static_cast<const float *>(P.scales);
            s = P.scale_per_row ? sp[n] : sp[0];
        }
        for (int i = 0; i < 8; ++i) {
            if (m0 + i >= M) break;
            const float v = acc[i] * s;
            if (y_bf16)
                static_cast<uint16_t *>(P.y)[static_cast<int64_t>(m0 + i) * N + n] = f32_to_bf16_rne(v);
            else
                static_cast<float *>(P.y)[static_cast<int64_t>(m0 + i) * N + n] = v;
        }
    }
}

template <int FMT>
bool skinny_ok(const Problem &p, int64_t m) {
    using Tr = FmtTraits<FMT>;
    if (m < 1 || m > 16) return false;
    if (p.k % Tr::kChunk != 0) return false;
    if (!aligned(p.x, 16) || !aligned(p.codes, 16)) return false;
    if (FMT == FMT_INT4 && (p.group % 128 != 0)) return false;
    if (FMT == FMT_NF4 && (p.group % 32 != 0)) return false;
    return true;
}

template <int FMT>
int32_t kc_for(int64_t k, int64_t m) {
    using Tr = FmtTraits<FMT>;
    int64_t kc = (kLdsBytesMax / 2) / m;
    kc = (kc / Tr::kChunk) * Tr::kChunk;
    if (kc < Tr::kChunk) kc = Tr::kChunk;
    return static_cast<int32_t>(kc < k ? kc : k);
}

// Launch a batch of problems that share M; all must pass skinny_ok.
template <int FMT>
void launch_skinny(Problem *ps, int count, int64_t m, int y_bf16, hipStream_t st) {
    Batch b{};
    int64_t tiles = 0, max_lds = 0;
    for (int i = 0; i < count; ++i) {
        b.p[i] = ps[i];
        b.p[i].tile_begin = static_cast<int32_t>(tiles);
        b.p[i].kc = kc_for<FMT>(ps[i].k, m);
        tiles += (ps[i].n + 15) / 16;
        const int64_t lds = m * b.p[i].kc * 2;
        if (lds > max_lds) max_lds = lds;
    }
    require(tiles <= 0x7fffffff, "too many rows for one launch");
    b.count = count;
    b.m = static_cast<int32_t>(m);
    b.y_bf16 = y_bf16;
    if (tiles == 0) return;
    skinny_qgemm_kernel<FMT><<<dim3(static_cast<unsigned>(tiles)), dim3(kThreads),
                               static_cast<size_t>(max_lds), st>>>(b);
    check_launch("skinny_qgemm");
}

template <int FMT>
void launch_generic(const Problem &p, int64_t m, int y_bf16, hipStream_t st) {
    if (p.n == 0 || m == 0) return;
    require(p.n <= 0x7fffffff && (m + 7) / 8 <= 65535, "shape too large for the generic kernel");
    generic_qgemm_kernel<FMT><<<dim3(static_cast<unsigned>(p.n), static_cast<unsigned>((m + 7) / 8)),
                                dim3(64), 0, st>>>(p, static_cast<int>(m), y_bf16);
    check_launch("generic_qgemm");
}

void common_checks(const void *x, int64_t m, int64_t n, int64_t k, const void *codes, void *y,
                   int32_t y_dtype) {
    require(m >= 0 && n >= 0 && k >= 0, "m, n, k must be non-negative");
    require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
    require(k % 8 == 0, "k must be a multiple of 8");
    if (m > 0 && n > 0) require(y != nullptr, "y must not be NULL");
    if (m > 0 && n > 0 && k > 0) require(x && codes, "x and codes must not be NULL");
}

}  // namespace

// Exposed to the prefill GEMM translation unit: route M <= 16 through the skinny kernel.
bool gemv_try_skinny(int fmt, const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                     const void *codes, const void *scales, const uint32_t *zeros, int per_row,
                     void *y, int y_bf16, hipStream_t st);

bool gemv_try_skinny(int fmt, const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                     const void *codes, const void *scales, const uint32_t *zeros, int per_row,
                     void *y, int y_bf16, hipStream_t st) {
    Problem p{x, codes, scales, zeros, y, n, k, static_cast<int32_t>(group), per_row, 0, 0};
    if (fmt == FMT_INT4 && skinny_ok<FMT_INT4>(p, m)) { launch_skinny<FMT_INT4>(&p, 1, m, y_bf16, st); return true; }
    if (fmt == FMT_INT8 && skinny_ok<FMT_INT8>(p, m)) { launch_skinny<FMT_INT8>(&p, 1, m, y_bf16, st); return true; }
    if (fmt == FMT_NF4 && skinny_ok<FMT_NF4>(p, m)) { launch_skinny<FMT_NF4>(&p, 1, m, y_bf16, st); return true; }
    return false;
}

void gemv_generic(int fmt, const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                  const void *codes, const void *scales, const uint32_t *zeros, int per_row, void *y,
                  int y_bf16, hipStream_t st) {
    Problem p{x, codes, scales, zeros, y, n, k, static_cast<int32_t>(group), per_row, 0, 0};
    if (fmt == FMT_INT4) launch_generic<FMT_INT4>(p, m, y_bf16, st);
    else if (fmt == FMT_INT8) launch_generic<FMT_INT8>(p, m, y_bf16, st);
    else launch_generic<FMT_NF4>(p, m, y_bf16, st);
}

}  // namespace cfh

using namespace cfh;

extern "C" {

int32_t castforge_hip_gemv_w4a16(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                                 const uint32_t *codes, const uint16_t *scales_f16,
                                 const uint32_t *zeros, void *y, int32_t y_dtype, void *stream,
                                 char **out_error) {
    return guarded(out_error, [&] {
        common_checks(x, m, n, k, codes, y, y_dtype);
        require(group >= 8 && group % 8 == 0, "group must be a positive multiple of 8");
        if (m == 0 || n == 0) return;
        require(k == 0 || (scales_f16 && zeros), "scales and zeros must not be NULL");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const int yb = y_dtype == CFH_DTYPE_BF16;
        if (!gemv_try_skinny(FMT_INT4, x, m, n, k, group, codes, scales_f16, zeros, 1, y, yb, st))
            gemv_generic(FMT_INT4, x, m, n, k, group, codes, scales_f16, zeros, 1, y, yb, st);
    });
}

int32_t castforge_hip_gemv_w8a16(const uint16_t *x, int64_t m, int64_t n, int64_t k,
                                 const int8_t *codes, const float *scales, int32_t granularity,
                                 void *y, int32_t y_dtype, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        common_checks(x, m, n, k, codes, y, y_dtype);
        require(granularity == CFH_GRAN_TENSOR || granularity == CFH_GRAN_CHANNEL,
                "granularity must be CFH_GRAN_TENSOR or CFH_GRAN_CHANNEL");
        if (m == 0 || n == 0) return;
        require(scales != nullptr, "scales must not be NULL");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const int yb = y_dtype == CFH_DTYPE_BF16, pr = granularity == CFH_GRAN_CHANNEL;
        if (!gemv_try_skinny(FMT_INT8, x, m, n, k, 0, codes, scales, nullptr, pr, y, yb, st))
            gemv_generic(FMT_INT8, x, m, n, k, 0, codes, scales, nullptr, pr, y, yb, st);
    });
}

int32_t castforge_hip_gemv_nf4(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t block,
                               const uint32_t *codes, const float *absmax, void *y, int32_t y_dtype,
                               void *stream, char **out_error) {
    return guarded(out_error, [&] {
        common_checks(x, m, n, k, codes, y, y_dtype);
        require(block >= 8 && block % 8 == 0, "block must be a positive multiple of 8");
        if (m == 0 || n == 0) return;
        require(k == 0 || absmax, "absmax must not be NULL");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const int yb = y_dtype == CFH_DTYPE_BF16;
        if (!gemv_try_skinny(FMT_NF4, x, m, n, k, block, codes, absmax, nullptr, 1, y, yb, st))
            gemv_generic(FMT_NF4, x, m, n, k, block, codes, absmax, nullptr, 1, y, yb, st);
    });
}

int32_t castforge_hip_gemv_w4a16_batched(const cfh_w4a16_problem_t *problems, int32_t count,
                                         int64_t m, int32_t y_dtype, void *stream,
                                         char **out_error) {
    return guarded(out_error, [&] {
        require(count >= 0 && count <= CFH_MAX_BATCH, "count must be in [0, CFH_MAX_BATCH]");
        require(count == 0 || problems != nullptr, "problems must not be NULL");
        require(m >= 1 && m <= 16, "batched GEMV requires 1 <= m <= 16");
        require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
        Problem ps[kMaxProblems];
        int used = 0;
        for (int i = 0; i < count; ++i) {
            const cfh_w4a16_problem_t &q = problems[i];
            common_checks(q.x, m, q.n, q.k, q.codes, q.y, y_dtype);
            if (q.n == 0) continue;
            require(q.k > 0 && q.scales_f16 && q.zeros, "problem buffers must not be NULL");
            Problem p{q.x, q.codes, q.scales_f16, q.zeros, q.y, q.n, q.k,
                      static_cast<int32_t>(q.group), 1, 0, 0};
            require(skinny_ok<FMT_INT4>(p, m),
                    "batched GEMV needs k % 128 == 0, group % 128 == 0 and 16-byte aligned x/codes");
            ps[used++] = p;
        }
        if (used) launch_skinny<FMT_INT4>(ps, used, m, y_dtype == CFH_DTYPE_BF16,
                                          static_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
