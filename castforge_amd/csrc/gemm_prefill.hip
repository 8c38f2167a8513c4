// Prefill (M > 64) dequant-fused GEMM for packed INT4 / INT8 / NF4 / GGUF weights on gfx950 MFMA.
//
// Y[m, n] = sum_k x[m, k] * dequant(W)[n, k]: x bf16 [M, K]; W packed [N, K] (the packed_rhs
// layout, passes/weights/fold.rs:549-554).  This is the evaluation of `castforge.fused_qmatmul`
// (codegen/eval.rs:1145-1179 -> eval_matmul_2d, eval.rs:1465-1507) at prefill sizes, where the
// reference interpreter runs an M*N*K scalar f32 loop on one core.
//
// Exactness.  The product must stay within 1e-2 relative / 1e-3 absolute of the f32 evaluator
// for any finite input, including near-zero outputs and activations beyond f16's range, so
// v_mfma_f32_32x32x16_bf16 is fed exact operands only: x as the bf16 it is, and every weight as
// one or more bf16 terms that sum exactly to the f32 weight the evaluator uses.
//   INT4  (q - z) * s and Q4_0 (q - 8) * d (15 significant bits): two terms, hi = bf16(w),
//         lo = w - hi;
//   INT8  one term, the integer q; the per-row (or tensor) scale multiplies the accumulator;
//   Q8_0  q * d (19 bits) and NF4 f32(T[q] * absmax) (24 bits): three terms.
//   A non-finite scale gives a non-finite weight (the remainder terms are 0) and so, as in the
//   evaluator, non-finite outputs on its row.
//   INT4 whose groups are whole 128-wide K blocks, INT8 and GGUF Q4_0 / Q8_0 planes have a
//   second kernel, prefill_i4_kernel below: one MFMA per product on the exact integer (q - z,
//   q - 8 or q) decoded in registers, a fresh f32 partial per group (GGUF: per 32-wide block;
//   INT8: one sum), and the group's scale applied to the partial by one fma into the total.
//   (A one-term INT4 form that instead multiplied the running accumulator by s_prev / s_cur
//   at every group start was measured and dropped: the rounding of the running sum put
//   near-zero outputs of cancellation-heavy rows further from the exact value than the
//   evaluator's own f32 sum.)
//   Range of that kernel: its partials hold sum x * q with |q| <= 127 (INT4: 15, Q4_0: 8)
//   before any scale, so they reach |x| * 127 * K.  It is exact-range for |x| <= 2^100 and
//   K <= 2^20 (2^127 < f32 max); past that a partial can overflow to +-inf where the
//   evaluator's x * (q * s) stays finite.  The two-term kernel (CASTFORGE_PREFILL_I4=0)
//   keeps the scale inside the weight and has no such bound.
//
// Design:
//   * workgroup tile BN (n) x BM (m) with 4 waves; W is the MFMA row operand, so each lane
//     ends with 4 consecutive n of one m;
//   * per K slice of 32 the workgroup loads codes / metadata and x into registers, decodes the
//     weights once per workgroup (shared by all BM rows of x) into bf16 planes in LDS and
//     copies x as is: 64-byte rows, 16-byte chunks XOR-swizzled by row so fragment reads hit
//     distinct banks; both operands in natural k order;
//   * two LDS stages: while slice t's MFMAs run, slice t+1 is decoded from registers into the
//     other stage and slice t+R's global loads are issued;
//   * XCD-aware tile order (each XCD owns a contiguous range of tiles grouped by m).
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// FMT_Q4G / FMT_Q8G: GGUF Q4_0 / Q8_0 planes (codes, one f16 d per 32; the same numbers as the
// GEMV's FMT_Q4_0 / FMT_Q8_0)
enum Fmt { FMT_INT4 = 0, FMT_INT8 = 1, FMT_NF4 = 2, FMT_Q4G = 3, FMT_Q8G = 4,
           // INT4 with groups of 32 / 64: instances of the one-MFMA kernel only
           FMT_I4G32 = 5, FMT_I4G64 = 6 };

// bf16 weight planes per format
template <int FMT> constexpr int planes() {
    return FMT == FMT_INT8 ? 1 : FMT == FMT_Q4G || FMT == FMT_INT4 ? 2 : 3;
}

constexpr int kThreads = 256;
constexpr int BK = 32;     // K elements per slice: one 64-byte bf16 row per tile row
constexpr int kXcds = 8;
constexpr int kGroupM = 4;

__constant__ float kNf4Pf[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

struct PfArgs {
    const uint16_t *x;      // bf16 [M, K]
    const void *codes;      // INT4 / NF4: u32 [N, K/8]; INT8: i8 [N, K]
    const void *scales;     // INT4: f16 [N, GP]; INT8: f32 [N] or [1]; NF4: f32 [N, NB]
    const uint32_t *zeros;  // INT4: u32 [N, ZW]
    void *y;                // [M, N] f32 or bf16
    int M, N, K;
    int group;              // INT4 group / NF4 block (multiple of 32)
    int per_row;            // INT8: 1 per-channel scales, 0 per-tensor
    int y_bf16;
    int y_vec;              // N % 4 == 0 and y 16-byte aligned: 4 outputs per store
    int tiles_m, tiles_n;
};

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

// f32 of the low / high bf16 of a packed pair
__device__ __forceinline__ float bf_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }

// Upper halves of two f32 holding bf16-exact values -> one bf16 pair (a low, b high).
__device__ __forceinline__ uint32_t pack_hi16(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

// Physical 16-byte chunk of logical chunk c in a 64-byte tile row r.
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 2) & 3); }

// INT8 word (signed codes of k .. k + 3) -> 2 bf16 pairs of exact q in k order.
__device__ __forceinline__ uint2 int8_word_bf16(uint32_t w) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = static_cast<float>(static_cast<int32_t>(w << (24 - 8 * j)) >> 24);
    return make_uint2(pack_hi16(v[0], v[1]), pack_hi16(v[2], v[3]));
}

// f32 pair -> T bf16 pairs whose sum is the pair exactly (for values of up to 8 T significant
// bits; T = 2 or 3).  Each term is the RNE bf16 of what the previous ones leave, and that
// remainder is exact in f32.  A non-finite value gives a non-finite first term (and NaN
// remainders), so its products stay non-finite.
template <int T>
__device__ __forceinline__ void split_bf16(float w0, float w1, uint32_t (&t)[3]) {
#pragma unroll
    for (int i = 0; i < T; ++i) {
        t[i] = f32x2_to_bf16x2_rne(w0, w1);
        w0 -= bf_lo(t[i]);
        w1 -= bf_hi(t[i]);
    }
}

template <int BM, int BN, int WN>
struct Cfg {
    static constexpr int WM = 4 / WN;            // waves along m
    static constexpr int TN = BN / WN;           // wave tile (n)
    static constexpr int TM = BM / WM;           // wave tile (m)
    static constexpr int I = TN / 32, J = TM / 32;
    static constexpr int kRowBytes = BK * 2;     // 64
};

// LDS bytes of one stage: P weight planes, then the x tile.
template <int FMT, int BM, int BN>
constexpr int stage_bytes() { return planes<FMT>() * BN * 64 + BM * 64; }

// W rows handled per thread per slice: BN / 256 (BN = 256 -> 1 row, BN = 128 -> lanes pair up)
// Large tiles keep one wave per SIMD (their accumulators fill the register file); tiles of
// 128 x 128 and below leave room for a second workgroup per CU.
template <int FMT, int BM, int BN, int WN, int R>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(BM * BN > 128 * 128 ? 1 : 2, BM * BN > 128 * 128 ? 1 : 2)))
void prefill_qgemm_kernel(PfArgs a) {
    using C = Cfg<BM, BN, WN>;
    constexpr int P = planes<FMT>();
    constexpr int kWPlane = BN * C::kRowBytes;
    constexpr int kStage = stage_bytes<FMT, BM, BN>();
    // x slice: BM rows x 4 chunks of 16 bytes; W slice: BN rows x (16 B INT4/NF4/Q4_0 | 32 B INT8/Q8_0)
    constexpr int kXPieces = BM * 4 / kThreads;  // 16-byte x pieces per thread
    constexpr int kWRowsPerThread = BN >= kThreads ? BN / kThreads : 1;
    constexpr int kWThreadsPerRow = BN >= kThreads ? 1 : kThreads / BN;  // split a row's bytes
    constexpr int kWBytesRow = FMT == FMT_INT8 || FMT == FMT_Q8G ? 32 : 16;
    constexpr int kWBytesThread = kWBytesRow / kWThreadsPerRow;  // 16, 8 or 4 (per row)
    static_assert(kXPieces >= 1 && kWRowsPerThread == 1, "tile / thread mapping");
    static_assert(kWBytesThread >= 4, "W bytes per thread");
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint2 lut[FMT == FMT_NF4 ? 256 : 1];  // NF4: byte -> (T[lo], T[hi]) as f32 bits

    const int M = a.M, N = a.N, K = a.K;
    // ---- XCD-aware tile order ----
    const int ntiles = a.tiles_m * a.tiles_n;
    int pid = blockIdx.x;
    {
        const int per_xcd = ntiles / kXcds, full = per_xcd * kXcds;
        if (pid < full) pid = (pid % kXcds) * per_xcd + pid / kXcds;
    }
    const int group_span = kGroupM * a.tiles_n;
    const int grp = pid / group_span;
    const int first_m = grp * kGroupM;
    const int gsize = (a.tiles_m - first_m) < kGroupM ? (a.tiles_m - first_m) : kGroupM;
    const int tm = first_m + (pid % group_span) % gsize;
    const int tn = (pid % group_span) / gsize;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    if constexpr (FMT == FMT_NF4) {
        for (int i = tid; i < 256; i += kThreads)
            lut[i] = make_uint2(__float_as_uint(kNf4Pf[i & 15]), __float_as_uint(kNf4Pf[i >> 4]));
    }

    // ---- global sources (descriptors over the tile's rows: rows past M / N read zero) ----
    const int m_valid = min(BM, M - m0), n_valid = min(BN, N - n0);
    const rsrc_t rx = make_rsrc(a.x + static_cast<int64_t>(m0) * K, static_cast<uint32_t>(m_valid) * K * 2);
    const int64_t w_row_bytes = FMT == FMT_INT8 || FMT == FMT_Q8G ? K : K / 2;
    const rsrc_t rw = make_rsrc(static_cast<const uint8_t *>(a.codes) + n0 * w_row_bytes,
                                static_cast<uint32_t>(n_valid * w_row_bytes));
    const int G = (K + a.group - 1) / a.group;     // INT4 groups / NF4 blocks per row
    const int ZW = (G + 7) / 8, GP = ZW * 8;
    rsrc_t rs = make_rsrc(a.codes, 0), rz = rs;  // empty ranges unless the format has metadata
    if constexpr (FMT == FMT_INT4 || FMT == FMT_Q4G || FMT == FMT_Q8G) {
        rs = make_rsrc(static_cast<const uint16_t *>(a.scales) + static_cast<int64_t>(n0) * GP,
                       static_cast<uint32_t>(n_valid) * GP * 2);
    }
    if constexpr (FMT == FMT_INT4) {
        rz = make_rsrc(a.zeros + static_cast<int64_t>(n0) * ZW, static_cast<uint32_t>(n_valid) * ZW * 4);
    } else if constexpr (FMT == FMT_NF4) {
        rs = make_rsrc(static_cast<const float *>(a.scales) + static_cast<int64_t>(n0) * G,
                       static_cast<uint32_t>(n_valid) * G * 4);
    }

    // this thread's x pieces: piece p covers row (tid + p * 256) / 4, chunk (tid % 4)
    // this thread's W part: row wr, bytes [wb, wb + kWBytesThread) of the row's slice
    const int wr = tid / kWThreadsPerRow;
    const int wb = (tid % kWThreadsPerRow) * kWBytesThread;

    struct Regs {
        uint4 x[kXPieces];
        uint32_t w[kWBytesThread / 4];
        uint32_t s, z;  // INT4: f16 scale bits, zero word; NF4: absmax bits; GGUF: d bits
    };
    auto gload = [&](Regs &r, int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int p = 0; p < kXPieces; ++p) {
            const int piece = tid + p * kThreads;
            const int row = piece >> 2, ch = piece & 3;
            r.x[p] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   rx, static_cast<uint32_t>(row * K + k0 + ch * 8) * 2, 0, 0));
        }
        const uint32_t wo = static_cast<uint32_t>(wr * w_row_bytes + (FMT == FMT_INT8 ? k0 : k0 / 2) + wb);
        if constexpr (FMT == FMT_Q4G) {
            // the slice is one block; its 4-byte piece p (elements 8p..8p+7) sits at byte
            // 16 p + 4 (block & 3) of the block's 64-byte chunk
            const uint32_t cb = static_cast<uint32_t>(wr * w_row_bytes + (k0 >> 7) * 64 + 4 * ((k0 >> 5) & 3));
#pragma unroll
            for (int h = 0; h < kWBytesThread / 4; ++h)
                r.w[h] = __builtin_amdgcn_raw_buffer_load_b32(rw, cb + 16 * (wb / 4 + h), 0, 0);
        } else if constexpr (FMT == FMT_Q8G) {
            // the slice is one block; its 8-byte piece p (elements 8p..8p+7) sits at byte
            // 16 p + 8 (block & 1) of the block's 64-byte chunk
            const uint32_t cb = static_cast<uint32_t>(wr * w_row_bytes + (k0 >> 6) * 64 + 8 * ((k0 >> 5) & 1));
#pragma unroll
            for (int h = 0; h < kWBytesThread / 8; ++h) {
                const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                              rw, cb + 16 * (wb / 8 + h), 0, 0));
                r.w[2 * h] = v.x;
                r.w[2 * h + 1] = v.y;
            }
        } else if constexpr (kWBytesThread >= 16) {
#pragma unroll
            for (int h = 0; h < kWBytesThread / 16; ++h) {
                const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo + 16 * h, 0, 0));
                r.w[4 * h] = v.x; r.w[4 * h + 1] = v.y; r.w[4 * h + 2] = v.z; r.w[4 * h + 3] = v.w;
            }
        } else if constexpr (kWBytesThread == 8) {
            const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, wo, 0, 0));
            r.w[0] = v.x; r.w[1] = v.y;
        } else {
            r.w[0] = __builtin_amdgcn_raw_buffer_load_b32(rw, wo, 0, 0);
        }
        // raw metadata words only: decoding them here would wait for the loads
        const int g = k0 / a.group;
        if constexpr (FMT == FMT_INT4 || FMT == FMT_Q4G || FMT == FMT_Q8G)
            r.s = __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<uint32_t>(wr * GP + (g & ~1)) * 2, 0, 0);
        if constexpr (FMT == FMT_INT4) {
            r.z = __builtin_amdgcn_raw_buffer_load_b32(rz, static_cast<uint32_t>(wr * ZW + (g >> 3)) * 4, 0, 0);
        } else if constexpr (FMT == FMT_NF4) {
            r.s = __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<uint32_t>(wr * G + g) * 4, 0, 0);
        }
    };

    // registers of slice kt -> bf16 planes of LDS stage `st`
    auto lwrite = [&](const Regs &r, int kt, int st) {
        uint8_t *base = lds + st * kStage;
        uint8_t *wplane = base;
        uint8_t *xplane = base + P * kWPlane;
#pragma unroll
        for (int p = 0; p < kXPieces; ++p) {
            const int piece = tid + p * kThreads;
            const int row = piece >> 2, ch = piece & 3;
            *reinterpret_cast<uint4 *>(xplane + row * C::kRowBytes + swz(row, ch) * 16) = r.x[p];
        }
        // W: this thread's bytes cover chunks [c0, c0 + nch) of row wr
        if constexpr (FMT == FMT_INT8) {
            // two code words = 8 k = one chunk
#pragma unroll
            for (int t = 0; t < kWBytesThread / 8; ++t) {
                const int ch = wb / 8 + t;
                const uint2 h0 = int8_word_bf16(r.w[2 * t]), h1 = int8_word_bf16(r.w[2 * t + 1]);
                *reinterpret_cast<uint4 *>(wplane + wr * C::kRowBytes + swz(wr, ch) * 16) =
                    make_uint4(h0.x, h0.y, h1.x, h1.y);
            }
        } else {
            // f32 weights as the evaluator forms them, split into P exact bf16 terms
            float d = 0.0f;
            float zf = 0.0f;
            if constexpr (FMT == FMT_NF4) {
                d = __uint_as_float(r.s);
            } else {
                if constexpr (FMT == FMT_INT4) zf = static_cast<float>((r.z >> (4 * ((kt * BK / a.group) & 7))) & 15u);
                const int g = kt * BK / a.group;
                d = f16_to_f32(static_cast<uint16_t>((g & 1) ? (r.s >> 16) : (r.s & 0xFFFFu)));
            }
            constexpr int kWordsPerChunk = FMT == FMT_Q8G ? 2 : 1;
#pragma unroll
            for (int t = 0; t < kWBytesThread / (4 * kWordsPerChunk); ++t) {
                const int ch = wb / (4 * kWordsPerChunk) + t;
                float v[8];
                if constexpr (FMT == FMT_NF4) {
                    const uint32_t w = r.w[t];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint2 e = lut[(w >> (8 * q)) & 255u];
                        v[2 * q] = __uint_as_float(e.x) * d;
                        v[2 * q + 1] = __uint_as_float(e.y) * d;
                    }
                } else if constexpr (FMT == FMT_Q4G || FMT == FMT_INT4) {
                    // exact (q - z) times the f16 scale: 15 significant bits, exact in f32
                    const uint32_t w = r.w[t];
                    const float z = FMT == FMT_Q4G ? 8.0f : zf;
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        v[q] = (static_cast<float>((w >> (4 * q)) & 15u) - z) * d;
                } else {
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            v[4 * h + q] = static_cast<float>(static_cast<int32_t>(r.w[2 * t + h] << (24 - 8 * q)) >> 24) * d;
                }
                uint32_t terms[4][3];
#pragma unroll
                for (int q = 0; q < 4; ++q) split_bf16<P>(v[2 * q], v[2 * q + 1], terms[q]);
                const int off = wr * C::kRowBytes + swz(wr, ch) * 16;
#pragma unroll
                for (int pl = 0; pl < P; ++pl)
                    *reinterpret_cast<uint4 *>(wplane + pl * kWPlane + off) =
                        make_uint4(terms[0][pl], terms[1][pl], terms[2][pl], terms[3][pl]);
            }
        }
    };

    // ---- fragments: row lane % 32 of each 32-row sub-tile, chunk 2 kk + lane / 32 ----
    const int wn = (wave % WN) * C::TN, wm = (wave / WN) * C::TM;
    const int fr = lane & 31, fh = lane >> 5;
    floatx16 acc[C::I][C::J];
#pragma unroll
    for (int i = 0; i < C::I; ++i)
#pragma unroll
        for (int j = 0; j < C::J; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    auto mma_stage = [&](int t) {
        const uint8_t *base = lds + (t & 1) * kStage;
        const uint8_t *wplane = base;
        const uint8_t *xplane = base + P * kWPlane;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int ch = 2 * kk + fh;
            bf16x8_t wf[P][C::I], xf[C::J];
#pragma unroll
            for (int i = 0; i < C::I; ++i) {
                const int r = wn + i * 32 + fr;
#pragma unroll
                for (int p = 0; p < P; ++p)
                    wf[p][i] = *reinterpret_cast<const bf16x8_t *>(wplane + p * kWPlane + r * C::kRowBytes + swz(r, ch) * 16);
            }
#pragma unroll
            for (int j = 0; j < C::J; ++j) {
                const int r = wm + j * 32 + fr;
                xf[j] = *reinterpret_cast<const bf16x8_t *>(xplane + r * C::kRowBytes + swz(r, ch) * 16);
            }
#pragma unroll
            for (int p = 0; p < P; ++p)
#pragma unroll
                for (int i = 0; i < C::I; ++i)
#pragma unroll
                    for (int j = 0; j < C::J; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[p][i], xf[j], acc[i][j], 0, 0, 0);
        }
    };

    const int KT = K / BK;
    // R register sets: set t % R carries slice t from its global loads to its LDS write.
    Regs ring[R];
    if constexpr (FMT == FMT_NF4) __syncthreads();  // LUT ready
    static_for<R>([&](auto II) {
        constexpr int i = decltype(II)::value;
        if (i < KT) gload(ring[i], i);
    });
    lwrite(ring[0], 0, 0);
    __syncthreads();
    // Step t: stage t & 1 holds slice t, sets (t + 1) % R .. hold slices t + 1 .. t + R - 1
    // (loads in flight) and set t % R is free (slice t went to LDS in step t - 1).  Issue
    // slice t + R into set t % R, run slice t's MFMAs, convert slice t + 1 into the other stage
    // (last read in step t - 1), then barrier.  The barrier is a bare s_barrier after the LDS
    // writes retire: __syncthreads() would also wait for the global loads in flight.  Steady
    // steps are branch-free, so the compiler's vmcnt waits cover only the loads being consumed.
    // Small tiles finish a slice quickly, so they keep more slices in flight (larger R).
    auto step = [&](auto steady, auto SI, int t) {
        constexpr bool kSteady = decltype(steady)::value;
        constexpr int si = decltype(SI)::value;
        if (kSteady || t + R < KT) gload(ring[si], t + R);
        mma_stage(t);
        if (kSteady || t + 1 < KT) lwrite(ring[(si + 1) % R], t + 1, (t + 1) & 1);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));
        __builtin_amdgcn_s_barrier();
    };
    int kt = 0;
    for (; kt + 2 * R - 1 < KT; kt += R)
        static_for<R>([&](auto II) { step(std::true_type{}, II, kt + decltype(II)::value); });
    for (; kt < KT; kt += R)
        static_for<R>([&](auto II) {
            if (kt + decltype(II)::value < KT) step(std::false_type{}, II, kt + decltype(II)::value);
        });

    // ---- epilogue: acc[i][j] holds n = wn + 32 i + 8 g + 4 (lane / 32) + q (reg 4 g + q),
    // m = wm + 32 j + lane % 32 ----
    float sc[C::I][4][4];  // INT8: scale of each output column (0 past N)
    if constexpr (FMT == FMT_INT8) {
        const float *sp = static_cast<const float *>(a.scales);
#pragma unroll
        for (int i = 0; i < C::I; ++i)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int n = n0 + wn + i * 32 + g * 8 + fh * 4 + q;
                    sc[i][g][q] = n < N ? sp[a.per_row ? n : 0] : 0.f;
                }
    }
    // a workgroup whose tile lies inside [M, N] with 4-aligned rows stores without checks
    const bool full = a.y_vec && m0 + BM <= M && n0 + BN <= N;
    static_for<C::J>([&](auto JJ) {
        constexpr int j = decltype(JJ)::value;
        const int m = m0 + wm + j * 32 + fr;
        static_for<C::I>([&](auto II) {
            constexpr int i = decltype(II)::value;
            static_for<4>([&](auto GG) {
                constexpr int g = decltype(GG)::value;
                const int n = n0 + wn + i * 32 + g * 8 + fh * 4;
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v[q] = acc[i][j][g * 4 + q];
                    if constexpr (FMT == FMT_INT8) v[q] *= sc[i][g][q];
                }
                const int64_t o = static_cast<int64_t>(m) * N + n;
                if (full) {
                    if (a.y_bf16)
                        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(a.y) + o) =
                            make_uint2(f32x2_to_bf16x2_rne(v[0], v[1]), f32x2_to_bf16x2_rne(v[2], v[3]));
                    else
                        *reinterpret_cast<float4 *>(static_cast<float *>(a.y) + o) = make_float4(v[0], v[1], v[2], v[3]);
                } else if (m < M) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (n + q < N) {
                            if (a.y_bf16) static_cast<uint16_t *>(a.y)[o + q] = f32_to_bf16_rne(v[q]);
                            else static_cast<float *>(a.y)[o + q] = v[q];
                        }
                    }
                }
            });
        });
    });
}

// ---- INT4 (groups of 32, 64 or a multiple of 128), INT8, GGUF Q4_0 / Q8_0 planes: one MFMA per product ----
//
// `prefill_i4_kernel<BM, D, NW, FMT, DW>` feeds the MFMA the exact integer (q - z) as bf16
// (|q - z| <= 15) and x as the bf16 it is.  Per 128-wide K block the MFMAs sum x (q - z) into a fresh f32
// partial, and one fma per accumulator applies the block's f16 group scale:
// y = sum_b s_b * P_b, the GEMV's per-group partial scheme.  Each partial rounds 8 times
// (one per 16-wide MFMA step) over 128 products and the total once per block, against the
// evaluator's one rounding per product (eval.rs:1465-1507).
//   * Tile 256 (n) x BM (m), NW waves.  Wave w owns n rows [256 / NW * w, 256 / NW * (w + 1))
//     (I = 8 / NW MFMA blocks of 32) and all BM rows of x (BM / 32 blocks).  W is the MFMA B
//     operand, so a lane's accumulators hold 16 m of one n and one scale multiplies them all.
//     At NW = 8 two waves share a SIMD: each holds half the accumulators, and one wave's
//     decode and fold run while the other's MFMAs do.
//   * W never touches LDS: each lane loads its row's 32 code bytes of the block (k = 64 h ..
//     64 h + 63 of the block, h = lane / 32) and decodes word kk for MFMA step kk.  The f16
//     pairs 1024 + q (even nibbles, at mantissa bits 0..3) and 64 + q (odd nibbles, at bits
//     4..7) come from one v_and_or_b32 each; v_fma_mix_f32 subtracts 1024 + z or 64 + z from
//     a half, giving q - z in f32 exactly; v_perm packs the bf16 halves.  17 VALU
//     instructions per 8 weights.
//   * x goes global -> LDS (buffer loads, rows past M read zero) in a ring of D + 1 stages of
//     BM rows x 256 bytes; 16-byte chunk c of row r sits at c ^ (r & 15), so the 16 rows that
//     one read phase touches hit 16 distinct chunks.  MFMA step kk reads chunk 8 h + kk, the
//     k range the W lane decoded.
//   * One barrier per block; x of block b + D and W of block b + DW are issued right after it.
//   * The other forms (instances by FMT): GGUF Q4_0 / Q8_0 (a d per 32-wide block, so a fold
//     every two MFMA steps; q - 8 or the signed byte q) and INT4 with groups of 32 / 64 read
//     their words in a step -> k map where no step straddles a group (WSet below); INT8 keeps
//     one f32 sum and applies its row scale once.
#ifndef CFH_PF_I4_DEPTH
#define CFH_PF_I4_DEPTH 2
#endif
// 1: block b - 1's partials are folded pair by pair in block b's first MFMA step; 0: at the
// end of block b - 1 (with 8 waves the first is 1-2 % faster)
#ifndef CFH_PF_I4_FOLD_FIRST
#define CFH_PF_I4_FOLD_FIRST 1
#endif
// prefetch depth of the Q4_0 planes form, and whether it reads x fragments a step ahead
#ifndef CFH_PF_Q4_DEPTH
#define CFH_PF_Q4_DEPTH 2
#endif
#ifndef CFH_PF_Q4_XPREFETCH
#define CFH_PF_Q4_XPREFETCH 0
#endif
// prefetch depths of the Q8_0 planes form: x blocks and W blocks in flight (its 16 code words
// per row block and lane leave registers for two W sets only)
#ifndef CFH_PF_Q8_DEPTH
#define CFH_PF_Q8_DEPTH 2
#endif
#ifndef CFH_PF_Q8_WDEPTH
#define CFH_PF_Q8_WDEPTH 1
#endif
// 1: a step's x fragments are read during the previous step's MFMAs
#ifndef CFH_PF_I4_XPREFETCH
#define CFH_PF_I4_XPREFETCH 1
#endif
// waves per workgroup: 8 (two per SIMD, 32 W rows each; measured 1.13-1.17x faster at
// M = 4096) or 4 (one per SIMD, 64 rows each)
#ifndef CFH_PF_I4_WAVES
#define CFH_PF_I4_WAVES 8
#endif
constexpr int kI4BN = 256;
constexpr int kI4KB = 128;

template <int BM, int D, int NW, int FMT, int DW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4)))
void prefill_i4_kernel(PfArgs a) {
    static_assert(FMT == FMT_INT4 || FMT == FMT_Q4G || FMT == FMT_Q8G || FMT == FMT_INT8 || FMT == FMT_I4G32 ||
                      FMT == FMT_I4G64,
                  "INT4, INT8 or GGUF Q4_0 / Q8_0 planes");
    constexpr bool kI8 = FMT == FMT_INT8;  // one scale per row (or tensor): no per-block fold
    constexpr bool kQ8 = FMT == FMT_Q8G;
    constexpr bool kQ4 = FMT == FMT_Q4G || kQ8;  // a d per 32-wide block (the GGUF forms)
    // INT4 with groups of 32 / 64: canonical codes read in the GGUF forms' step -> k map (a
    // step never straddles a group), a zero point and a scale per group
    constexpr int kSG = FMT == FMT_I4G32 ? 32 : FMT == FMT_I4G64 ? 64 : 0;
    constexpr bool kQmap = kQ4 || kSG;
    static_assert(!kQmap || CFH_PF_I4_FOLD_FIRST, "small groups fold at the start of each group");
    constexpr int J = BM / 32;
    constexpr int I = kI4BN / 32 / NW;  // MFMA row blocks of W per wave
    constexpr int kRowsW = kI4BN / NW;  // W rows per wave
    constexpr int S = D + 1;
    constexpr int kStage = BM * kI4KB * 2;
    constexpr int kRowsX = BM / NW;          // x rows each wave loads
    constexpr int kDma = kRowsX / 4;         // 1 KB buffer -> LDS loads per wave and block
    constexpr int kLoads = kDma + I * (kQ8 ? 9 : kQ4 ? 3 : kSG ? 6 : 4);  // vector-memory loads per wave and block
    static_assert(!kI8 || I * 4 == kLoads - kDma, "INT8: 4 code loads per row block");
    static_assert(I >= 1 && kRowsX % 16 == 0 && S * kStage <= 160 * 1024, "tile / LDS budget");
    extern __shared__ __align__(16) uint8_t lds[];

    const int M = a.M, N = a.N, K = a.K;
    int pid = blockIdx.x;
    const int ntiles = a.tiles_m * a.tiles_n;
    {
        const int per_xcd = ntiles / kXcds, full = per_xcd * kXcds;
        if (pid < full) pid = (pid % kXcds) * per_xcd + pid / kXcds;
    }
    const int group_span = kGroupM * a.tiles_n;
    const int first_m = (pid / group_span) * kGroupM;
    const int gsize = (a.tiles_m - first_m) < kGroupM ? (a.tiles_m - first_m) : kGroupM;
    const int m0 = (first_m + (pid % group_span) % gsize) * BM;
    const int n0 = ((pid % group_span) / gsize) * kI4BN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int fr = lane & 31, h = lane >> 5;
    const int KB = K / kI4KB;
    const int G = K / a.group, ZW = (G + 7) / 8, GP = ZW * 8;
    const int bpg = max(1, a.group / kI4KB);  // K blocks per group (INT4; unused by the others)

    const rsrc_t rx = make_rsrc(a.x + static_cast<int64_t>(m0) * K, static_cast<uint32_t>(min(BM, M - m0)) * K * 2);
    // descriptors over the tile's rows [n0, n0 + n_valid) (rows past N read zero); a lane's
    // row is 64 wave + 32 i + fr of the tile
    const int nw0 = n0 + kRowsW * wave;
    const uint32_t n_valid = static_cast<uint32_t>(min(kI4BN, N - n0));
    const int row_bytes = kQ8 || kI8 ? K : K / 2;
    const rsrc_t rw = make_rsrc(static_cast<const uint8_t *>(a.codes) + static_cast<int64_t>(n0) * row_bytes,
                                n_valid * static_cast<uint32_t>(row_bytes));
    const rsrc_t rs = make_rsrc(static_cast<const uint16_t *>(a.scales) + static_cast<int64_t>(n0) * GP, n_valid * GP * 2);
    const rsrc_t rz = make_rsrc(a.zeros + static_cast<int64_t>(n0) * ZW, n_valid * ZW * 4);
    uint32_t vw[I], vs[I], vz[I];
#pragma unroll
    for (int i = 0; i < I; ++i) {
        const uint32_t row = static_cast<uint32_t>(kRowsW * wave + 32 * i + fr);
        vw[i] = row * static_cast<uint32_t>(row_bytes) + (kI8 ? 64u : kSG ? 8u : 32u) * h;
        vs[i] = row * static_cast<uint32_t>(GP) * 2u;
        vz[i] = row * static_cast<uint32_t>(ZW) * 4u;
    }
    // lane offsets of the x loads: load t writes rows 4 t .. 4 t + 3 of the wave's BM / 4;
    // lane -> row 4 t + lane / 16, physical chunk lane % 16 (logical chunk ^ (row & 15))
    uint32_t lv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int r = 4 * u + (lane >> 4);
        lv[u] = static_cast<uint32_t>((lane >> 4) * K * 2 + (((lane & 15) ^ (r & 15)) * 16));
    }

    // INT4: word t of the lane's 32 code bytes holds k = 64 h + 8 t .. + 7 of the block.
    // Q4_0 planes: 8-element piece p of 32-wide block bb sits at byte 16 p + 4 bb of the row's
    // 64-byte chunk, so word 4 pp + bb (pp = p - 2 h) holds k = 32 bb + 16 h + 8 pp .. + 7.
    // Q8_0 planes: 8-byte piece p of 32-wide block B sits at byte 16 p + 8 (B & 1) of the
    // row's 64-byte chunk B / 2; lane half h loads pieces 2 h and 2 h + 1 of each block
    // (w[i][B]: words 0-1 piece 2 h, 2-3 piece 2 h + 1), k = 32 B + 16 h + 8 pp .. + 7.
    struct WSet {
        uint4 w[I][kQ8 || kI8 ? 4 : 2];  // INT4 / Q4_0 [half]: words 0..3, 4..7 of the lane's 32 code bytes;
                                         // INT8: the lane's 64 code bytes (k = 64 h .. 64 h + 63)
        uint32_t s[I][2], z[I];   // INT4: s[i][0] = the f16 scale pair; GGUF: the block's 4 d
    };
    auto issue_x = [&](int b, uint8_t *stage) __attribute__((always_inline)) {
        uint8_t *dst = stage + kRowsX * wave * (kI4KB * 2);
#pragma unroll
        for (int t = 0; t < kDma; ++t)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rx, reinterpret_cast<__attribute__((address_space(3))) void *>(reinterpret_cast<uintptr_t>(dst + t * 1024)),
                16, lv[t & 3], (kRowsX * wave + 4 * t) * K * 2 + b * (kI4KB * 2), 0, 0);
    };
    auto issue_w = [&](int b, WSet &r) __attribute__((always_inline)) {
        const int g = b / bpg;
#pragma unroll
        for (int i = 0; i < I; ++i) {
            if constexpr (kI8) {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    r.w[i][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vw[i] + b * 128 + 16 * c, 0, 0));
            } else if constexpr (kQ8) {
                // vw = row * K + 32 h; piece 2 h + pp of block B at 64 (B / 2) + 8 (B & 1) + 16 pp
#pragma unroll
                for (int B = 0; B < 4; ++B) {
                    const uint32_t o = vw[i] + b * 128 + 64 * (B >> 1) + 8 * (B & 1);
                    const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, o, 0, 0));
                    const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, o + 16, 0, 0));
                    r.w[i][B] = make_uint4(lo.x, lo.y, hi.x, hi.y);
                }
            } else if constexpr (kSG) {
                // words 4 B + 2 h, 4 B + 2 h + 1 of the row's 16 (vw = row * K / 2 + 8 h): k = 32 B +
                // 16 h .. + 15, kept in step order
#pragma unroll
                for (int B2 = 0; B2 < 2; ++B2) {
                    const uint2 e = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, vw[i] + b * 64 + 32 * B2, 0, 0));
                    const uint2 o = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rw, vw[i] + b * 64 + 32 * B2 + 16, 0, 0));
                    r.w[i][B2] = make_uint4(e.x, e.y, o.x, o.y);
                }
            } else {
                r.w[i][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vw[i] + b * 64, 0, 0));
                r.w[i][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rw, vw[i] + b * 64 + 16, 0, 0));
            }
            if constexpr (kI8) {
            } else if constexpr (kSG) {
                // the block's 4 (g32) or 2 (g64) scales and the zero-point word holding theirs
                if constexpr (kSG == 32) {
                    const uint2 d = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, vs[i] + b * 8, 0, 0));
                    r.s[i][0] = d.x;
                    r.s[i][1] = d.y;
                } else {
                    r.s[i][0] = __builtin_amdgcn_raw_buffer_load_b32(rs, vs[i] + b * 4, 0, 0);
                }
                r.z[i] = __builtin_amdgcn_raw_buffer_load_b32(rz, vz[i] + (kSG == 32 ? (b >> 1) : (b >> 2)) * 4, 0, 0);
            } else if constexpr (kQ4) {
                const uint2 d = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, vs[i] + b * 8, 0, 0));
                r.s[i][0] = d.x;
                r.s[i][1] = d.y;
            } else {
                r.s[i][0] = __builtin_amdgcn_raw_buffer_load_b32(rs, vs[i] + (g & ~1) * 2, 0, 0);
                r.z[i] = __builtin_amdgcn_raw_buffer_load_b32(rz, vz[i] + (g >> 3) * 4, 0, 0);
            }
        }
    };

    floatx16 tot[I][J];
#pragma unroll
    for (int i = 0; i < I; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) tot[i][j][e] = 0.f;

    // opaque constants: kept in registers so the masks fold into v_and_or_b32 and the unit
    // multiplier of v_fma_mix_f32 is not simplified away
    auto opaque = [](uint32_t v) __attribute__((always_inline)) {
        asm("" : "+v"(v));
        return v;
    };
    const uint32_t kM0 = opaque(0x000F000Fu), kM1 = opaque(0x00F000F0u);
    const uint32_t kC0 = opaque(0x64006400u), kC1 = opaque(0x54005400u);  // f16 1024, 64
    const float kOne = __uint_as_float(opaque(0x3F800000u));
    // 8 codes (k order) -> 4 bf16 pairs of exact q - z; ce = -(1024 + z), co = -(64 + z)
    auto decode = [&](uint32_t w, float ce, float co) __attribute__((always_inline)) {
        typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
        const uint32_t w8 = w >> 8;
        const h2_t p0 = __builtin_bit_cast(h2_t, (w & kM0) | kC0), p1 = __builtin_bit_cast(h2_t, (w & kM1) | kC1);
        const h2_t p2 = __builtin_bit_cast(h2_t, (w8 & kM0) | kC0), p3 = __builtin_bit_cast(h2_t, (w8 & kM1) | kC1);
        const float q0 = __builtin_fmaf(static_cast<float>(p0.x), kOne, ce), q4 = __builtin_fmaf(static_cast<float>(p0.y), kOne, ce);
        const float q1 = __builtin_fmaf(static_cast<float>(p1.x), kOne, co), q5 = __builtin_fmaf(static_cast<float>(p1.y), kOne, co);
        const float q2 = __builtin_fmaf(static_cast<float>(p2.x), kOne, ce), q6 = __builtin_fmaf(static_cast<float>(p2.y), kOne, ce);
        const float q3 = __builtin_fmaf(static_cast<float>(p3.x), kOne, co), q7 = __builtin_fmaf(static_cast<float>(p3.y), kOne, co);
        return __builtin_bit_cast(bf16x8_t, make_uint4(pack_hi16(q0, q1), pack_hi16(q2, q3), pack_hi16(q4, q5), pack_hi16(q6, q7)));
    };
    // Q8_0: 8 signed codes (two words, k order) -> 4 bf16 pairs of exact q: (w & 0x00FF00FF) ^
    // 0x64806480 is the f16 pair 1024 + (q + 128), and v_fma_mix_f32 subtracts 1152
    const uint32_t kM8 = opaque(0x00FF00FFu), kC8 = opaque(0x64806480u);
    auto decode8 = [&](uint32_t w0, uint32_t w1) __attribute__((always_inline)) {
        typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
        const float c = -1152.0f;
        const h2_t a0 = __builtin_bit_cast(h2_t, (w0 & kM8) ^ kC8), a1 = __builtin_bit_cast(h2_t, ((w0 >> 8) & kM8) ^ kC8);
        const h2_t b0 = __builtin_bit_cast(h2_t, (w1 & kM8) ^ kC8), b1 = __builtin_bit_cast(h2_t, ((w1 >> 8) & kM8) ^ kC8);
        const float q0 = __builtin_fmaf(static_cast<float>(a0.x), kOne, c), q2 = __builtin_fmaf(static_cast<float>(a0.y), kOne, c);
        const float q1 = __builtin_fmaf(static_cast<float>(a1.x), kOne, c), q3 = __builtin_fmaf(static_cast<float>(a1.y), kOne, c);
        const float q4 = __builtin_fmaf(static_cast<float>(b0.x), kOne, c), q6 = __builtin_fmaf(static_cast<float>(b0.y), kOne, c);
        const float q5 = __builtin_fmaf(static_cast<float>(b1.x), kOne, c), q7 = __builtin_fmaf(static_cast<float>(b1.y), kOne, c);
        return __builtin_bit_cast(bf16x8_t, make_uint4(pack_hi16(q0, q1), pack_hi16(q2, q3), pack_hi16(q4, q5), pack_hi16(q6, q7)));
    };

    // One set of partials.  Block b's first MFMA step overwrites pair (i, j) only right after
    // block b - 1's partials of that pair are scaled into the total, so the VALU work of the
    // fold runs beside the MFMAs of the other pairs.  Block 0's "previous" partials are zero
    // with scale zero.
    floatx16 part[I][J];
#pragma unroll
    for (int i = 0; i < I; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) part[i][j][e] = 0.f;
    float sc_prev[I] = {};
    if constexpr (kI8) {
        // per-channel: scales[n] (0 past N); per tensor: scales[0]
        const float *sp = static_cast<const float *>(a.scales);
#pragma unroll
        for (int i = 0; i < I; ++i) {
            const int n = nw0 + 32 * i + fr;
            sc_prev[i] = n < N ? sp[a.per_row ? n : 0] : 0.f;
        }
    }
    auto fold = [&](int i, int j) __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 16; ++e) tot[i][j][e] = __builtin_fmaf(sc_prev[i], part[i][j][e], tot[i][j][e]);
    };

    auto compute = [&](int b, const uint8_t *__restrict__ stage, const WSet &r) __attribute__((always_inline)) {
        const int g = b / bpg;
        float ce[I], co[I], sc[I];
#pragma unroll
        for (int i = 0; i < I; ++i) {
            const float z = kQ4 || kI8 ? 8.0f : static_cast<float>((r.z[i] >> (4 * (g & 7))) & 15u);
            ce[i] = -(1024.0f + z);
            co[i] = -(64.0f + z);
            sc[i] = kI8 ? 0.f : f16_to_f32(static_cast<uint16_t>((g & 1) ? (r.s[i][0] >> 16) : (r.s[i][0] & 0xFFFFu)));
        }
        // x fragments of step kk + 1 are read while step kk's MFMAs run (two sets); step kk
        // reads the 16-byte chunk holding the k range its W word covers
        bf16x8_t xf[2][J];
        // chunk c ^ (fr & 15) with c = (step constant) | (lane half term).  Q4_0: row offsets
        // are multiples of 256, so a step's offset is one XOR of the lane's offset with the
        // step constant, and the lane offset is hidden from the compiler, which would otherwise
        // keep one precomputed address per step and stage live and spill them (10 % faster);
        // INT4 keeps the precomputed addresses (1.5 % faster there).
        const uint32_t xlane = static_cast<uint32_t>(fr * (kI4KB * 2) + (((fr & 15) ^ (kQmap ? 2 * h : 8 * h)) * 16));
        auto read_x = [&](int kk, bf16x8_t (&dst)[J]) __attribute__((always_inline)) {
            const uint32_t cst = kQmap ? 4 * (kk >> 1) + (kk & 1) : kk;
            uint32_t xo = xlane;
            if constexpr (kQmap) asm volatile("" : "+v"(xo));
            const uint8_t *row = stage + (xo ^ (cst << 4));
#pragma unroll
            for (int j = 0; j < J; ++j)
                dst[j] = *reinterpret_cast<const bf16x8_t *>(row + 32 * j * (kI4KB * 2));
        };
        // (Q4_0 reads each step's fragments in the step by default: with its extra folds a
        // second set spills)
        constexpr bool kXPre = CFH_PF_I4_XPREFETCH && (!kQmap || CFH_PF_Q4_XPREFETCH);
        if (kXPre) read_x(0, xf[0]);
        static_for<8>([&](auto KK) {
            constexpr int kk = decltype(KK)::value;
            constexpr int xs = kXPre ? (kk & 1) : 0;
            bf16x8_t wf[I];
            if (!kXPre) read_x(kk, xf[0]);
            else if (kk + 1 < 8) read_x(kk + 1, xf[xs ^ 1]);
            // INT4: word kk; Q4_0: word 4 (kk & 1) + kk / 2 (block kk / 2, half kk & 1)
            constexpr int half = kQ4 ? (kk & 1) : (kk >> 2), comp = kQ4 ? (kk >> 1) : (kk & 3);
            // Q4_0: nothing moves across a 32-wide block start (the compiler would otherwise
            // hoist later blocks' decodes above the folds and run out of registers)
            if constexpr (kQmap && (kk & 1) == 0 && kk > 0) __builtin_amdgcn_sched_barrier(0);
            // small groups: the zero point of the group this step starts
            if constexpr (kSG && (kk % (kSG / 16)) == 0) {
                const int nib = kSG == 32 ? 4 * (b & 1) + (kk >> 1) : 2 * (b & 3) + (kk >> 2);
#pragma unroll
                for (int i = 0; i < I; ++i) {
                    const float z = static_cast<float>((r.z[i] >> (4 * nib)) & 15u);
                    ce[i] = -(1024.0f + z);
                    co[i] = -(64.0f + z);
                }
            }
#pragma unroll
            for (int i = 0; i < I; ++i) {
                if constexpr (kQ8 || kI8) {
                    // Q8_0: block kk / 2, piece 2 h + (kk & 1); INT8: words 2 kk, 2 kk + 1
                    const uint4 q = r.w[i][kk >> 1];
                    wf[i] = (kk & 1) ? decode8(q.z, q.w) : decode8(q.x, q.y);
                } else {
                    const uint4 q = r.w[i][half];
                    const uint32_t word = comp == 0 ? q.x : comp == 1 ? q.y : comp == 2 ? q.z : q.w;
                    wf[i] = decode(word, ce[i], co[i]);
                }
            }
            // Q4_0: a new 32-wide block (and scale) every two steps
            constexpr bool kStart = kI8 ? false : kQ4 ? (kk & 1) == 0 : kSG ? (kk % (kSG / 16)) == 0 : kk == 0;
#pragma unroll
            for (int i = 0; i < I; ++i)
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    if constexpr (kStart) {
                        // the pair's fold, then its first MFMA; nothing moves across the
                        // barrier, so the reads of the fold stay next to the MFMA that needs
                        // their registers
                        if (CFH_PF_I4_FOLD_FIRST) fold(i, j);
                        floatx16 z{};
                        part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[xs][j], wf[i], z, 0, 0, 0);
                        if (CFH_PF_I4_FOLD_FIRST && !kQmap) __builtin_amdgcn_sched_barrier(0);
                    } else {
                        part[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[xs][j], wf[i], part[i][j], 0, 0, 0);
                    }
                }
            if constexpr (kSG && kStart) {
                // this group's scale multiplies the partial that the next group start folds
#pragma unroll
                for (int i = 0; i < I; ++i) {
                    const uint32_t dw = kSG == 32 ? r.s[i][kk >> 2] : r.s[i][0];
                    const bool hi = kSG == 32 ? (kk & 2) != 0 : (kk & 4) != 0;
                    sc_prev[i] = f16_to_f32(static_cast<uint16_t>(hi ? (dw >> 16) : (dw & 0xFFFFu)));
                }
            }
            if constexpr (kQ4 && kStart) {
                // block kk / 2's d scales the partial that the next block start folds
#pragma unroll
                for (int i = 0; i < I; ++i) {
                    const uint32_t dw = r.s[i][kk >> 2];
                    sc_prev[i] = f16_to_f32(static_cast<uint16_t>((kk & 2) ? (dw >> 16) : (dw & 0xFFFFu)));
                }
            }
        });
        if constexpr (!kQmap && !kI8) {
#pragma unroll
            for (int i = 0; i < I; ++i) sc_prev[i] = sc[i];
        }
        if (!CFH_PF_I4_FOLD_FIRST) {
#pragma unroll
            for (int i = 0; i < I; ++i)
#pragma unroll
                for (int j = 0; j < J; ++j) fold(i, j);
        }
    };

    // Block b: wait for its loads, barrier (every wave's LDS writes of block b landed, every
    // wave is done with block b - 1's stage), issue W of block b + DW into the register set
    // block b - 1 used and x of block b + D into the stage block b - 1 used, compute block b.
    // With DW < D a step issues W before x, so block b's W and x are both in when at most the
    // loads issued after W(b) are outstanding (x of b + 1 .. b + D - DW, then whole steps).
    // Steps are unrolled U-fold (a multiple of both ring sizes) so every index is a constant.
    constexpr int SW = DW + 1;
    constexpr int U = S % SW == 0 ? S : SW % S == 0 ? SW : S * SW;
    constexpr int kAhead = kDma * (D - DW) + (DW - 1) * kLoads;  // loads issued after W(b), steady
    static_assert(DW >= 1 && DW <= D, "W depth within the x depth");
    WSet ws[SW];
    // (with DW == D the order within a step does not change the count; x first there keeps
    // the INT4 form's schedule, which spilled with W first)
    constexpr bool kWFirst = DW < D;
    static_for<D>([&](auto II) {
        constexpr int i = decltype(II)::value;
        if (!kWFirst && i < KB) issue_x(i, lds + i * kStage);
        if (i < DW && i < KB) issue_w(i, ws[i]);
        if (kWFirst && i < KB) issue_x(i, lds + i * kStage);
    });
    // Steady steps (every block of the unrolled group issues its loads) are branch-free, so
    // the compiler's own vmcnt waits cover only the loads being consumed; the last steps wait
    // for everything.
    auto step = [&](auto steady, auto SI, int b) __attribute__((always_inline)) {
        constexpr bool kSteady = decltype(steady)::value;
        constexpr int sx = decltype(SI)::value % S, sw = decltype(SI)::value % SW;
        if (kSteady) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(kAhead) & ~(15 << 8));
        } else {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & ~(15 << 8));
        }
        __builtin_amdgcn_s_barrier();
        if (!kWFirst && (kSteady || b + D < KB)) issue_x(b + D, lds + ((sx + D) % S) * kStage);
        if (kSteady || b + DW < KB) issue_w(b + DW, ws[(sw + DW) % SW]);
        if (kWFirst && (kSteady || b + D < KB)) issue_x(b + D, lds + ((sx + D) % S) * kStage);
        compute(b, lds + sx * kStage, ws[sw]);
    };
    int b0 = 0;
    for (; b0 + U - 1 + D < KB; b0 += U)
        static_for<U>([&](auto SI) { step(std::true_type{}, SI, b0 + decltype(SI)::value); });
    for (; b0 < KB; b0 += U)
        static_for<U>([&](auto SI) {
            if (b0 + decltype(SI)::value < KB) step(std::false_type{}, SI, b0 + decltype(SI)::value);
        });
    // the last block's partials
    if (CFH_PF_I4_FOLD_FIRST) {
#pragma unroll
        for (int i = 0; i < I; ++i)
#pragma unroll
            for (int j = 0; j < J; ++j) fold(i, j);
    }

    // ---- epilogue: tot[i][j] reg 4 g + q holds m = m0 + 32 j + 8 g + 4 h + q, n = nw0 + 32 i + fr ----
#pragma unroll
    for (int i = 0; i < I; ++i) {
        const int n = nw0 + 32 * i + fr;
        if (n >= N) continue;
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + 32 * j + 8 * (e >> 2) + 4 * h + (e & 3);
                if (m < M) {
                    const int64_t o = static_cast<int64_t>(m) * N + n;
                    if (a.y_bf16) static_cast<uint16_t *>(a.y)[o] = f32_to_bf16_rne(tot[i][j][e]);
                    else static_cast<float *>(a.y)[o] = tot[i][j][e];
                }
            }
    }
}

template <int BM, int D, int NW, int FMT, int DW = D>
void launch_i4(PfArgs a, hipStream_t st) {
    constexpr int lds = (D + 1) * BM * kI4KB * 2;
    static std::mutex mu;
    static std::map<int, bool> attr_set;  // per device
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    {
        std::lock_guard<std::mutex> g(mu);
        if (!attr_set[dev]) {
            check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(&prefill_i4_kernel<BM, D, NW, FMT, DW>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, lds),
                      "hipFuncSetAttribute(prefill_i4_kernel)");
            attr_set[dev] = true;
        }
    }
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + kI4BN - 1) / kI4BN;
    const int64_t tiles = static_cast<int64_t>(a.tiles_m) * a.tiles_n;
    require(tiles <= 0x7fffffff, "too many tiles");
    prefill_i4_kernel<BM, D, NW, FMT, DW><<<dim3(static_cast<unsigned>(tiles)), dim3(64 * NW), lds, st>>>(a);
    check_launch("prefill_i4_kernel");
}

template <int FMT, int BM, int BN, int WN, int R>
void launch_cfg(PfArgs a, hipStream_t st) {
    constexpr int lds = 2 * stage_bytes<FMT, BM, BN>();
    static_assert(lds <= 160 * 1024, "LDS budget");
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    const int64_t tiles = static_cast<int64_t>(a.tiles_m) * a.tiles_n;
    require(tiles <= 0x7fffffff, "too many tiles");
    prefill_qgemm_kernel<FMT, BM, BN, WN, R><<<dim3(static_cast<unsigned>(tiles)), dim3(kThreads), lds, st>>>(a);
    check_launch("prefill_qgemm");
}

// Tile shapes, largest first.  The largest square one that still gives every CU a workgroup
// is used; small M or N falls through to smaller tiles rather than leaving CUs idle (NF4 at
// M = 64 over an 11008 x 4096 matrix: 227 us with 256 x 256 tiles, 45 us with 64 x 64).
// CASTFORGE_PREFILL_TILE (e.g. "64x128") forces a shape.
// register sets in flight per tile shape (slices loaded ahead of their LDS write)
#ifndef CFH_PF_R_256
#define CFH_PF_R_256 2
#endif
#ifndef CFH_PF_R_128x256
#define CFH_PF_R_128x256 2
#endif
#ifndef CFH_PF_R_128
#define CFH_PF_R_128 4
#endif
#ifndef CFH_PF_R_64x128
#define CFH_PF_R_64x128 6
#endif
#ifndef CFH_PF_R_64
#define CFH_PF_R_64 8
#endif
enum PfTile { PF_256x256, PF_128x256, PF_128x128, PF_64x128, PF_64x64, PF_NTILES };
constexpr int kPfTileM[PF_NTILES] = {256, 128, 128, 64, 64};
constexpr int kPfTileN[PF_NTILES] = {256, 256, 128, 128, 64};

int pick_tile(int64_t M, int64_t N) {
    if (const char *e = std::getenv("CASTFORGE_PREFILL_TILE")) {
        for (int t = 0; t < PF_NTILES; ++t) {
            char name[16];
            std::snprintf(name, sizeof(name), "%dx%d", kPfTileM[t], kPfTileN[t]);
            if (std::strcmp(e, name) == 0) return t;
        }
    }
    int cus = 256;
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
    }
    // 128 x 256 and 64 x 128 are left to the override: at every shape measured they lost to
    // the next smaller square tile (W_gate / W_down of the 7B block at M = 512 / 1024 / 4096,
    // NF4 / Q8_0 / INT8: e.g. Q8_0 11008 x 4096 at M = 1024 406 against 278 us on 128 x 128,
    // NF4 4096 x 11008 at M = 512 254 on 64 x 128 against 196 us on 64 x 64)
    for (int t : {PF_256x256, PF_128x128, PF_64x64}) {
        const int64_t tiles = ((M + kPfTileM[t] - 1) / kPfTileM[t]) * ((N + kPfTileN[t] - 1) / kPfTileN[t]);
        if (M > kPfTileM[t] / 2 && tiles >= static_cast<int64_t>(cus)) return t;
    }
    return PF_64x64;
}

template <int FMT>
void launch_fmt(const PfArgs &a, hipStream_t st) {
    switch (pick_tile(a.M, a.N)) {
        case PF_256x256: launch_cfg<FMT, 256, 256, 2, CFH_PF_R_256>(a, st); break;
        case PF_128x256: launch_cfg<FMT, 128, 256, 2, CFH_PF_R_128x256>(a, st); break;
        case PF_128x128: launch_cfg<FMT, 128, 128, 2, CFH_PF_R_128>(a, st); break;
        case PF_64x128: launch_cfg<FMT, 64, 128, 2, CFH_PF_R_64x128>(a, st); break;
        default: launch_cfg<FMT, 64, 64, 2, CFH_PF_R_64>(a, st); break;
    }
}

// INT4 whose groups are whole 128-wide K blocks takes the one-MFMA kernel once it has at least
// one 256 x 128 tile per 6 CUs (43 on 256 CUs; other formats below).  Measured against the
// generic kernel's smaller
// tiles: 11008 x 4096 (43 n-tiles) at M = 96 / 512 / 1024: 57 / 61 / 125 us against 65 / 128 /
// 290; 4096 x 11008 (16 n-tiles) at M = 256 / 512: 143 / 143 us against 121 / 199.
// CASTFORGE_PREFILL_I4=0 keeps every INT4 problem on the generic kernel, =1 sends every one
// whose groups allow it to the one-MFMA kernel.
bool i4_eligible(const PfArgs &a, int fmt) {
    if (fmt == FMT_I4G32 || fmt == FMT_I4G64) {
        if (a.K % kI4KB != 0) return false;
    } else if (fmt == FMT_Q4G || fmt == FMT_Q8G || fmt == FMT_INT8 ? a.K % kI4KB != 0
                                                                    : (a.group % kI4KB != 0 || a.K % a.group != 0)) {
        return false;
    }
    if (static_cast<int64_t>(128) * a.K * 2 >= (int64_t{1} << 31)) return false;
    if (const char *e = std::getenv("CASTFORGE_PREFILL_I4")) {
        if (std::strcmp(e, "0") == 0) return false;
        if (std::strcmp(e, "1") == 0) return true;
    }
    int cus = 256, dev = 0;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
    }
    const int64_t tiles = ((a.M + 127) / 128) * static_cast<int64_t>((a.N + kI4BN - 1) / kI4BN);
    // INT4: one tile per 6 CUs.  The GGUF forms fold every two MFMA steps and INT8's generic
    // kernel is already one term, so they switch later (measured on 256 CUs, us generic / one-
    // MFMA): Q4_0 / Q8_0 11008 x 4096 at M = 128 (43 tiles) 65 / 76 and 75 / 92, at M = 256
    // (86) 102 / 77 and 116 / 92; INT8 4096 x 11008 and 4096 x 4096 at M = 1024 (128 tiles)
    // 124 / 136 and 51 / 55, 11008 x 4096 at M = 512 (172) 73 / 56.
    if (fmt == FMT_INT8) return 8 * tiles >= 5 * static_cast<int64_t>(cus);
    if (fmt == FMT_Q4G || fmt == FMT_Q8G || fmt == FMT_I4G32 || fmt == FMT_I4G64) return 3 * tiles >= cus;
    return 6 * tiles >= cus;
}

}  // namespace

// Routes one problem to the prefill MFMA kernel when its shape allows it.
bool prefill_try(int fmt, const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                 const void *codes, const void *scales, const uint32_t *zeros, int per_row, void *y,
                 int y_bf16, hipStream_t st) {
    if (m < 17 || n < 1 || k < BK || k % BK != 0) return false;
    if (fmt != FMT_INT8 && (group < BK || group % BK != 0)) return false;
    if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return false;
    // 32-bit buffer offsets over one tile's rows
    if (256 * k * 2 >= (int64_t{1} << 31) || 256 * k >= (int64_t{1} << 31)) return false;
    if (!aligned(x, 16) || !aligned(codes, 16)) return false;
    PfArgs a{x, codes, scales, zeros, y, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k),
             static_cast<int>(fmt == FMT_INT8 ? BK : group), per_row, y_bf16, (n % 4 == 0 && aligned(y, 16)) ? 1 : 0, 0, 0};
    if (fmt == FMT_INT4 && i4_eligible(a, fmt)) launch_i4<128, CFH_PF_I4_DEPTH, CFH_PF_I4_WAVES, FMT_INT4>(a, st);
    else if (fmt == FMT_INT4 && a.group == 32 && i4_eligible(a, FMT_I4G32))
        launch_i4<128, CFH_PF_Q4_DEPTH, CFH_PF_I4_WAVES, FMT_I4G32, 1>(a, st);  // two W sets: three spill
    else if (fmt == FMT_INT4 && a.group == 64 && i4_eligible(a, FMT_I4G64))
        launch_i4<128, CFH_PF_Q4_DEPTH, CFH_PF_I4_WAVES, FMT_I4G64>(a, st);
    else if (fmt == FMT_INT8 && i4_eligible(a, fmt)) launch_i4<128, CFH_PF_Q8_DEPTH, CFH_PF_I4_WAVES, FMT_INT8, CFH_PF_Q8_WDEPTH>(a, st);
    else if (fmt == FMT_Q4G && i4_eligible(a, fmt)) launch_i4<128, CFH_PF_Q4_DEPTH, CFH_PF_I4_WAVES, FMT_Q4G>(a, st);
    else if (fmt == FMT_Q8G && i4_eligible(a, fmt)) launch_i4<128, CFH_PF_Q8_DEPTH, CFH_PF_I4_WAVES, FMT_Q8G, CFH_PF_Q8_WDEPTH>(a, st);
    else if (fmt == FMT_INT4) launch_fmt<FMT_INT4>(a, st);
    else if (fmt == FMT_NF4) launch_fmt<FMT_NF4>(a, st);
    else if (fmt == FMT_Q4G) launch_fmt<FMT_Q4G>(a, st);
    else if (fmt == FMT_Q8G) launch_fmt<FMT_Q8G>(a, st);
    else launch_fmt<FMT_INT8>(a, st);
    return true;
}

}  // namespace cfh
