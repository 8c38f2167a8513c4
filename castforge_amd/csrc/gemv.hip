// Dequant-fused GEMV / skinny GEMM (M <= 64) for packed INT4 / INT8 / NF4 / GGUF weights, gfx950.
//
// Replaces the evaluation of `castforge.fused_qmatmul` (eval.rs:1145-1179 with
// eval_matmul_2d, eval.rs:1465-1507) and the one-thread-per-row HIP text the reference emits
// for it (gpu_c.rs:208-292): out[m, n] = sum_k x[m, k] * dequant(W)[n, k], W stored [N, K]
// row-major (packed_rhs layout, fold.rs:549-554).
//
// Decode is HBM-bound on the packed weight stream.  Design:
//   * a workgroup (4 waves) owns a tile of 16*R weight rows (R = 1 for M = 1);
//   * a chunk is what one wave-wide load brings for 16 rows: lane%16 = row, lane/16 = part,
//     each lane loads LW bytes (16, 8 or 4), so one chunk spans exactly one quantization
//     group / NF4 block per row and its scale multiplies the fp32 MFMA result (no rounding of
//     the scale into the f16 operand);
//   * v_mfma_f32_16x16x32_f16 with dequantized W rows as B and the activation rows as A; x is
//     converted from bf16 to f16 in the permuted order the nibble extraction produces,
//     each (row, chunk) scaled by an exact power of two that the chunk's f32 partial undoes, so
//     any finite bf16 activation is accepted (x_scale_of);
//   * M = 1 (skinny_m1_split_kernel): each wave owns a contiguous quarter of K, copies its
//     groups' scales / zero points and its x slice into its own LDS region up front, and then
//     streams codes only, decoded to exact (q - z) f16 operands;
//   * M = 2..64 (skinny_gx_kernel): the waves interleave over K in units of NB chunks,
//     double-buffered per wave, each wave reading its chunks' x fragments from global memory
//     and converting them itself; up to 4 x tiles of 16 rows share every decoded weight word;
//     exact (q - z) / q / NF4 hi+lo operands;
//   * problems with the longest K are dispatched first so no long workgroup forms a tail.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
// x staged per workgroup and pass for M > 1 (fewer passes: each pass boundary drains the
// weight loads in flight; 32 KB -> 64 KB took M = 8 / 16 from 48 / 65 to 42 / 55 us per block)
#ifndef CFH_GEMV_LDS_MAX
#define CFH_GEMV_LDS_MAX 65536
#endif
constexpr int kLdsBytesMax = CFH_GEMV_LDS_MAX;  // activation stage per workgroup
constexpr int kLdsBytesSplit = 65536;  // the M = 1 split-K kernel's x slices per workgroup
constexpr int kMaxProblems = 8;
constexpr uint32_t kOobGx = 0x80000000u;  // buffer offset past every range: reads 0, no traffic
// rows-per-workgroup multiplier and chunks in flight per wave for M <= 4 (tuning knobs)
#ifndef CFH_GEMV_R_SMALL
#define CFH_GEMV_R_SMALL 1
#endif
#ifndef CFH_GEMV_NB_SMALL
#define CFH_GEMV_NB_SMALL 4
#endif
// M = 2..16 (skinny_gx_kernel with one x tile): rows per workgroup (16 R) by M, and chunks per unit
#ifndef CFH_GX_R_SMALL
#define CFH_GX_R_SMALL 2
#endif
#ifndef CFH_GX_R_MID
#define CFH_GX_R_MID 2
#endif
#ifndef CFH_GX_R_BIG
#define CFH_GX_R_BIG 4
#endif
#ifndef CFH_GX_NB
#define CFH_GX_NB 2
#endif
// M = 1 decode uses the split-K kernel (0: the per-tile kernel, for comparison)
#ifndef CFH_GEMV_SPLIT
#define CFH_GEMV_SPLIT 1
#endif
// cache policy of the streamed weight-code loads (2 = nt: the codes are read once)
#ifndef CFH_GEMV_CPOL
#define CFH_GEMV_CPOL 0
#endif

// FMT_Q4_0 / FMT_Q8_0: GGUF planes (gguf.hip), 32-element blocks with an f16 d, M = 1 only
// on the MFMA path
enum Fmt { FMT_INT4 = 0, FMT_INT8 = 1, FMT_NF4 = 2, FMT_Q4_0 = 3, FMT_Q8_0 = 4 };

constexpr bool is_gguf(int fmt) { return fmt == FMT_Q4_0 || fmt == FMT_Q8_0; }
// blocks per chunk of the GGUF planes (a chunk is 64 bytes of a row)
constexpr int gguf_bpc(int fmt) { return fmt == FMT_Q4_0 ? 4 : 2; }

struct Problem {
    const uint16_t *x;      // bf16 [M, K]
    const void *codes;      // INT4/NF4: u32 [N, K/8]; INT8: i8 [N, K]
    const void *scales;     // INT4: f16 [N, GP] (GP = 8*ceil(G/8)); INT8: f32 [N] or [1]; NF4: f32 [N, K/block]
    const uint32_t *zeros;  // INT4: u32 [N, ceil(G/8)]
    void *y;                // [M, N] f32 or bf16
    int64_t n, k;
    int32_t group;          // INT4 group / NF4 block
    int32_t scale_per_row;  // INT8: 1 per-channel, 0 per-tensor
    int32_t tile_begin;     // first workgroup index of this problem
    int32_t kc;             // K elements staged per LDS pass (M = 1 split-K: LDS bytes per wave)
    int32_t soff, zoff;     // M = 1 split-K: scale and zero-point pieces within a wave's LDS bytes
    int32_t xsoff;          // M = 1 split-K: per-chunk activation post factors within a wave's LDS bytes
};

struct Batch {
    Problem p[kMaxProblems];
    int32_t count;
    int32_t m;
    int32_t y_bf16;
    int32_t kc_max;  // M > 1 kernel: the largest problem's kc (the activation post factors follow)
};

template <int FMT> constexpr int codes_per_byte() { return FMT == FMT_INT8 || FMT == FMT_Q8_0 ? 1 : 2; }

// Position, within each 8-element k-run, of the element the extraction places in f16 slot i.
// INT4: (n0,n4),(n1,n5),(n2,n6),(n3,n7); INT8 (two words): (b0,b2),(b1,b3) of each word;
// NF4: the table gives natural-order pairs.
__device__ __forceinline__ int perm_src(int fmt, int i) {
    if (fmt == FMT_INT4 || fmt == FMT_Q4_0) return (i >> 1) + ((i & 1) << 2);
    if (fmt == FMT_INT8 || fmt == FMT_Q8_0) return ((i >> 2) << 2) + ((i >> 1) & 1) + ((i & 1) << 1);
    return i;
}

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// A loop-invariant constant held in a VGPR.  gfx9 VOP3 encodings take no literal operand and
// at most one SGPR, so (w & mask) | magic only becomes a single v_and_or_b32 when both
// constants already sit in VGPRs.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
    uint32_t v;
    asm("v_mov_b32 %0, %1" : "=v"(v) : "i"(c));
    return v;
}

// Activation range.  bf16 activations span 2^-133 .. 2^128, f16 operands 2^-24 .. 65504.  Each
// chunk of x (one row, the K elements one chunk of weight codes spans) is multiplied by an
// exact power of two pre = 2^-sh chosen from the chunk's largest bf16 exponent e:
// sh = clamp(e - 141, -126, 126) puts the chunk's largest element in [2^14, 2^15), so every
// element within 2^-28 of it converts to f16 exactly and smaller ones lose at most 2^-25 of
// 2^-sh.  The chunk's f32 partial sum is multiplied by post = 2^sh, which undoes the scale
// exactly: y(2^e x) = 2^e y(x) bit for bit while nothing overflows.  Inf / NaN stay non-finite.
__device__ __forceinline__ uint32_t bf16x8_emax(const uint32_t wv[4]) {
    uint32_t e = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        e = max(e, (wv[q] >> 7) & 0xFFu);
        e = max(e, (wv[q] >> 23) & 0xFFu);
    }
    return e;
}

// Max over aligned groups of R lanes (R = 1, 2, 4, 8 or 16), every lane of a group receiving it.
template <int R>
__device__ __forceinline__ uint32_t lane_group_max(uint32_t v) {
#pragma unroll
    for (int o = 1; o < R; o <<= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), o)));
    return v;
}

__device__ __forceinline__ void x_scale_of(uint32_t emax, float &pre, float &post) {
    int sh = static_cast<int>(emax) - 141;
    sh = sh < -126 ? -126 : sh > 126 ? 126 : sh;
    pre = __uint_as_float(static_cast<uint32_t>(127 - sh) << 23);
    post = __uint_as_float(static_cast<uint32_t>(127 + sh) << 23);
}

// 8 bf16 (4 words) -> 4 f16 pairs of x * pre in the extraction order of FMT.
__device__ __forceinline__ void bf16x8_to_f16_perm(int fmt, const uint32_t wv[4], float pre, uint32_t o[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int s0 = perm_src(fmt, 2 * q), s1 = perm_src(fmt, 2 * q + 1);
        const uint16_t b0 = static_cast<uint16_t>(wv[s0 >> 1] >> (16 * (s0 & 1)));
        const uint16_t b1 = static_cast<uint16_t>(wv[s1 >> 1] >> (16 * (s1 & 1)));
        const half2_t h = {static_cast<_Float16>(bf16_to_f32(b0) * pre), static_cast<_Float16>(bf16_to_f32(b1) * pre)};
        o[q] = __builtin_bit_cast(uint32_t, h);
    }
}

struct Int4Consts {
    uint32_t lo_mask, hi_mask, magic;
};

__device__ __forceinline__ Int4Consts int4_consts() {
    return Int4Consts{vgpr_const(0x000F000Fu), vgpr_const(0x00F000F0u), vgpr_const(0x64006400u)};
}

// INT4 word -> 4 f16 pairs of exact (q - z).  zc1024 = -(1024+z) splat, zc64 = -(64+z) splat.
// (w & 0x000F000F) | 0x6400_6400 is the f16 pair (1024 + n0, 1024 + n4); the 0x00F0 nibbles
// give 1024 + 16 n, scaled back by 1/16.  Every intermediate is an exact f16.
__device__ __forceinline__ void int4_word_to_h(uint32_t w, half2_t zc1024, half2_t zc64,
                                               const Int4Consts &k, uint32_t out[4]) {
    const half2_t sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
    const uint32_t w8 = w >> 8;
    out[0] = as_u(as_h2((w & k.lo_mask) | k.magic) + zc1024);
    out[1] = as_u(as_h2((w & k.hi_mask) | k.magic) * sixteenth + zc64);
    out[2] = as_u(as_h2((w8 & k.lo_mask) | k.magic) + zc1024);
    out[3] = as_u(as_h2((w8 & k.hi_mask) | k.magic) * sixteenth + zc64);
}

// INT8 word (4 signed codes) -> 2 f16 pairs of exact q.
__device__ __forceinline__ void int8_word_to_h(uint32_t w, uint32_t out[2]) {
    const half2_t c1152 = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    const uint32_t u = w ^ 0x80808080u;
    out[0] = as_u(as_h2((u & 0x00FF00FFu) | 0x64006400u) + c1152);
    out[1] = as_u(as_h2(((u >> 8) & 0x00FF00FFu) | 0x64006400u) + c1152);
}

__device__ __forceinline__ half8_t pack8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(half8_t, make_uint4(a, b, c, d));
}

__constant__ float kNf4[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer descriptor over [base, base + bytes): 32-bit offsets, reads past `bytes` return 0.
__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

// The same over values the caller knows to be wave-uniform, moved to scalar registers (a
// descriptor built from values the compiler cannot prove uniform is re-read per lane).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ rsrc_t make_rsrc_u(const void *base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = static_cast<uint32_t>(uni(static_cast<int>(static_cast<uint32_t>(a))));
    const uint32_t hi = static_cast<uint32_t>(uni(static_cast<int>(static_cast<uint32_t>(a >> 32))));
    return make_rsrc(reinterpret_cast<const void *>((static_cast<uint64_t>(hi) << 32) | lo),
                     static_cast<uint32_t>(uni(static_cast<int>(bytes))));
}

// Loads one unit issues: per row tile NB code loads, plus one scale and one zero-point load
// (INT4), one absmax load per chunk (NF4) or one scale load per chunk (GGUF Q4_0 / Q8_0).
template <int FMT, int NB, int R>
constexpr int kVmcntAfterUnit() { return vmcnt_imm(R * (NB + (FMT == 0 ? 2 : (FMT == 2 || FMT == 3 || FMT == 4) ? NB : 0))); }

template <int LW>
__device__ __forceinline__ void load_words(rsrc_t r, uint32_t off, uint32_t *w) {
    if constexpr (LW == 16) {
        const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CFH_GEMV_CPOL));
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (LW == 8) {
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CFH_GEMV_CPOL));
        w[0] = v.x; w[1] = v.y;
    } else {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CFH_GEMV_CPOL);
    }
}

// ONE: M == 1, so only accumulator slot 0 of the lanes with part == 0 is ever stored and the
// per-chunk scale is applied to that slot alone.
template <int FMT, int LW, int R, bool ONE>
__global__ __launch_bounds__(kThreads) void skinny_qgemm_kernel(Batch b) {
    constexpr int WPL = LW / 4;                         // 32-bit code words per lane per chunk
    constexpr int CPB = codes_per_byte<FMT>();
    constexpr int CK = 4 * LW * CPB;                    // K elements per chunk
    constexpr int NB = R == 4 ? 2 : CFH_GEMV_NB_SMALL;  // chunks in flight per wave
    extern __shared__ __align__(16) _Float16 xs[];      // [M][KC], permuted per 8-run
    __shared__ floatx4 red[kWaves - 1][R][64];
    __shared__ uint2 lut[FMT == FMT_NF4 ? 256 : 1];

    int pi = 0;
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
        if (i < b.count && static_cast<int>(blockIdx.x) >= b.p[i].tile_begin) pi = i;
    const Problem &P = b.p[pi];
    const int M = b.m;
    const int64_t N = P.n, K = P.k;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x - P.tile_begin) * 16 * R;
    const int rows_here = static_cast<int>((N - n0) < 16 * R ? (N - n0) : 16 * R);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, part = lane >> 4;
    const uint32_t row_bytes = static_cast<uint32_t>(K / CPB);
    // descriptors over this workgroup's rows only: rows past N read as zero
    const rsrc_t rc = make_rsrc(static_cast<const uint8_t *>(P.codes) + n0 * row_bytes,
                                static_cast<uint32_t>(rows_here) * row_bytes);
    // INT4: scale groups per row; NF4: absmax blocks per row
    const int64_t grp = FMT == FMT_INT8 ? CK : P.group;  // INT8 has no groups (group 0)
    const uint32_t G = static_cast<uint32_t>((K + grp - 1) / grp);
    const uint32_t ZW = (G + 7) / 8, GP = ZW * 8;  // INT4 scale rows are padded to GP groups
    const int gshift = is_gguf(FMT) ? 0 : __builtin_ctz(static_cast<uint32_t>(grp / CK));  // chunks per group = 2^gshift
    rsrc_t rs, rz;
    if constexpr (is_gguf(FMT)) {
        rs = make_rsrc(static_cast<const uint16_t *>(P.scales) + n0 * GP, static_cast<uint32_t>(rows_here) * GP * 2);
    }
    if constexpr (FMT == FMT_INT4) {
        rs = make_rsrc(static_cast<const uint16_t *>(P.scales) + n0 * GP, static_cast<uint32_t>(rows_here) * GP * 2);
        rz = make_rsrc(P.zeros + n0 * ZW, static_cast<uint32_t>(rows_here) * ZW * 4);
    } else if constexpr (FMT == FMT_NF4) {
        rs = make_rsrc(static_cast<const float *>(P.scales) + n0 * G, static_cast<uint32_t>(rows_here) * G * 4);
    }
    uint32_t code_off[R], sc_off[R], z_off[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = 16 * r + lr;
        code_off[r] = row * row_bytes + part * LW;
        sc_off[r] = row * ((FMT == FMT_INT4 || is_gguf(FMT)) ? GP : G);
        z_off[r] = row * ZW;
    }

    // A wave works on "units" of NB consecutive chunks, double-buffered in registers: the
    // next unit's loads are issued before the current unit is consumed.  Raw loaded words
    // only: decoding a scale or zero point at load time would make the wave wait for it.
    // INT4 (one group per chunk): the unit's NB scales are one aligned NB*2-byte load and its
    // zero points one word, instead of two scattered loads per chunk.
    struct Unit {
        uint32_t wq[NB][R][WPL];
        // INT4: f16 scale pairs in [0, NB/2); NF4: f32 absmax bits per chunk; GGUF: the chunk's
        // block scales as f16 pairs (Q4_0: 2 words per chunk, Q8_0: 1)
        uint32_t sv[R][FMT == FMT_Q4_0 ? 2 * NB : NB];
        uint32_t zv[R];      // INT4: the zero-point word of the unit's 8-group block
    };
    Unit ua, ub;

    // Every call issues the same loads (NB code loads per row tile, plus the unit's scale and
    // zero-point loads for INT4 or one absmax load per chunk for NF4), so the loop below is
    // straight-line and the compiler's vmcnt waits only cover the unit being consumed.
    // Chunks at or past `cend` use an offset beyond the descriptor's range: the buffer unit
    // returns zero for them without touching memory.
    constexpr uint32_t kOob = 0x80000000u;
    auto load_unit = [&](Unit &u, int c0, int cend) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int c = c0 + j;
            const bool in = c < cend;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                load_words<LW>(rc, in ? code_off[r] + static_cast<uint32_t>(c) * (CK / CPB) : kOob, u.wq[j][r]);
                if constexpr (FMT == FMT_Q4_0) {
                    const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                                  rs, in ? (sc_off[r] + static_cast<uint32_t>(c) * 4u) * 2u : kOob, 0, 0));
                    u.sv[r][2 * j] = v.x;
                    u.sv[r][2 * j + 1] = v.y;
                } else if constexpr (FMT == FMT_Q8_0) {
                    u.sv[r][j] = __builtin_amdgcn_raw_buffer_load_b32(
                        rs, in ? (sc_off[r] + static_cast<uint32_t>(c) * 2u) * 2u : kOob, 0, 0);
                }
                if constexpr (FMT == FMT_NF4)
                    u.sv[r][j] = __builtin_amdgcn_raw_buffer_load_b32(
                        rs, in ? (sc_off[r] + (static_cast<uint32_t>(c) >> gshift)) * 4 : kOob, 0, 0);
            }
        }
        if constexpr (FMT == FMT_INT4) {
            // a unit past the end reads metadata it never uses (within or past this tile's rows,
            // where the descriptor returns zero): 20 bytes per lane, no branch
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t so = (sc_off[r] + static_cast<uint32_t>(c0)) * 2;
                if constexpr (NB == 8) {
                    const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, so, 0, 0));
                    u.sv[r][0] = v.x; u.sv[r][1] = v.y; u.sv[r][2] = v.z; u.sv[r][3] = v.w;
                } else if constexpr (NB == 4) {
                    const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, so, 0, 0));
                    u.sv[r][0] = v.x; u.sv[r][1] = v.y;
                } else {
                    static_assert(NB == 2, "INT4 units hold 2, 4 or 8 chunks");
                    u.sv[r][0] = __builtin_amdgcn_raw_buffer_load_b32(rs, so, 0, 0);
                }
                u.zv[r] = __builtin_amdgcn_raw_buffer_load_b32(rz, (z_off[r] + (static_cast<uint32_t>(c0) >> 3)) * 4, 0, 0);
            }
        }
    };

    const int KC = P.kc;
    const int KCmax = b.kc_max;  // the largest problem's stage: xpost follows it
    const int nchunks = static_cast<int>(K / CK);
    const int cps = KC / CK;  // chunks per LDS stage

    // Activation staging.  x[:, k0:k0+kc] is copied as raw bf16 straight into LDS
    // (global_load_lds: no VGPRs held), laid out [m][kc].  The copy is issued before the weight
    // loads, so waiting for it (vmcnt drains in issue order) does not wait for HBM.  After a
    // barrier every thread converts its 16-byte runs in place to f16, permuted into the order
    // the code extraction produces, and a second barrier publishes them.
    auto stage_copy = [&](int cs_, int ce_) {
        const int64_t k0 = static_cast<int64_t>(cs_) * CK;
        const int kc = (ce_ - cs_) * CK;
        const int bytes = M * kc * 2;
        for (int blk = wave; blk * 1024 < bytes; blk += kWaves) {  // wave-uniform
            const int e = blk * 1024 + lane * 16;  // byte offset in the stage
            if (e < bytes) {
                const int el = e >> 1;
                const int m = M == 1 ? 0 : el / kc, kk = el - m * kc;
                __builtin_amdgcn_global_load_lds(
                    static_cast<const void *>(P.x + static_cast<int64_t>(m) * K + k0 + kk),
                    reinterpret_cast<__attribute__((address_space(3))) void *>(
                        reinterpret_cast<uintptr_t>(xs) + blk * 1024),
                    16, 0, 0);
            }
        }
    };
    // Each (row m, chunk) is scaled by its own power of two (x_scale_of); its post factor goes
    // to xpost[chunk][m], M4 = M rounded up to 4 slots per chunk.  The CK / 8 runs of a chunk
    // are consecutive iterations, so aligned groups of CK / 8 lanes hold one chunk.
    const int M4 = (M + 3) & ~3;
    float *const xpost = reinterpret_cast<float *>(xs + M * KCmax);
    auto stage_convert = [&](int cs_, int ce_) {
        const int kc = (ce_ - cs_) * CK;
        const int runs = M * kc / 8;
        for (int it = tid; it < runs; it += kThreads) {
            const uint4 raw = *reinterpret_cast<const uint4 *>(xs + it * 8);
            const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
            float pre, post;
            x_scale_of(lane_group_max<CK / 8>(bf16x8_emax(wv)), pre, post);
            uint32_t o[4];
            bf16x8_to_f16_perm(FMT, wv, pre, o);
            *reinterpret_cast<uint4 *>(xs + it * 8) = make_uint4(o[0], o[1], o[2], o[3]);
            const int e = it * 8, m = e / kc, c = (e - m * kc) / CK;
            if ((it & (CK / 8 - 1)) == 0) xpost[c * M4 + m] = post;
        }
    };

    const int ce0 = cps < nchunks ? cps : nchunks;
    stage_copy(0, ce0);
    load_unit(ua, wave * NB, ce0);  // the first weight unit is in flight during the staging

    if constexpr (FMT == FMT_NF4) {
        for (int i = tid; i < 256; i += kThreads) {
            const _Float16 h0 = static_cast<_Float16>(kNf4[i & 15]), h1 = static_cast<_Float16>(kNf4[i >> 4]);
            const _Float16 l0 = static_cast<_Float16>(kNf4[i & 15] - static_cast<float>(h0));
            const _Float16 l1 = static_cast<_Float16>(kNf4[i >> 4] - static_cast<float>(h1));
            half2_t hi = {h0, h1}, lo = {l0, l1};
            lut[i] = make_uint2(as_u(hi), as_u(lo));
        }
    }
    // Wait for this wave's LDS copies only: they were issued before the weight loads and
    // vmcnt drains in issue order.  A bare s_barrier is used because __syncthreads() carries a
    // release fence that would also wait for the weight loads still in flight.
    __builtin_amdgcn_s_waitcnt(kVmcntAfterUnit<FMT, NB, R>());
    __builtin_amdgcn_s_barrier();
    stage_convert(0, ce0);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));  // this wave's LDS writes are done
    __builtin_amdgcn_s_barrier();

    floatx4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = floatx4{0.f, 0.f, 0.f, 0.f};
    // A rows >= M only feed output rows that are never stored, so they read row 0
    const int xr = lr < M ? lr : 0;
    const Int4Consts i4k = int4_consts();

    // the post factors of this lane's output rows m = 4 part + q (rows >= M read row 0's)
    const int mi = part * 4 < M ? part * 4 : 0;
    auto post_of = [&](int c, int cs) -> floatx4 {
        if constexpr (ONE) {
            return floatx4{xpost[(c - cs) * M4], 0.f, 0.f, 0.f};
        } else {
            return *reinterpret_cast<const floatx4 *>(xpost + (c - cs) * M4 + mi);
        }
    };
    auto process = [&](const Unit &u, int cb, int cs, int ce) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int c = cb + j;
            if (c >= ce) break;
            const _Float16 *xa = xs + xr * ((ce - cs) * CK) + (c - cs) * CK + part * (CK / 4);
            const floatx4 post = post_of(c, cs);
            if constexpr (FMT == FMT_INT4) {
                floatx4 pacc[R];
                uint32_t zc1024[R], zc64[R];
                const uint32_t gsh = 4 * (static_cast<uint32_t>(c) & 7u);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    pacc[r] = floatx4{0.f, 0.f, 0.f, 0.f};
                    const uint32_t z = (u.zv[r] >> gsh) & 15u;
                    // f16 bits of -(1024 + z) and -(64 + z), splatted to both halves
                    zc1024[r] = (0xE400u + z) * 0x00010001u;
                    zc64[r] = (0xD400u + (z << 4)) * 0x00010001u;
                }
#pragma unroll
                for (int t = 0; t < WPL; ++t) {
                    const half8_t aop = *reinterpret_cast<const half8_t *>(xa + t * 8);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        uint32_t hb[4];
                        int4_word_to_h(u.wq[j][r][t], as_h2(zc1024[r]), as_h2(zc64[r]), i4k, hb);
                        pacc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(hb[0], hb[1], hb[2], hb[3]),
                                                                        pacc[r], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r)
                {
                    const float sc = f16_to_f32(static_cast<uint16_t>(u.sv[r][j >> 1] >> (16 * (j & 1))));
                    if constexpr (ONE) acc[r][0] += (pacc[r][0] * sc) * post[0];
                    else acc[r] += (pacc[r] * sc) * post;
                }
            } else if constexpr (is_gguf(FMT)) {
                // one MFMA per block (the four parts of a row hold elements 8p..8p+7 of each
                // block of the chunk), scaled in f32 by the block's d
                constexpr int BPC = gguf_bpc(FMT);
                const _Float16 *xg = xs + xr * ((ce - cs) * CK) + (c - cs) * CK + 8 * part;
                floatx4 cacc[R];
#pragma unroll
                for (int r = 0; r < R; ++r) cacc[r] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int q = 0; q < BPC; ++q) {
                    const half8_t aop = *reinterpret_cast<const half8_t *>(xg + 32 * q);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        floatx4 pb = floatx4{0.f, 0.f, 0.f, 0.f};
                        if constexpr (FMT == FMT_Q4_0) {
                            uint32_t hb[4];
                            int4_word_to_h(u.wq[j][r][q], as_h2(0xE408E408u), as_h2(0xD480D480u), i4k, hb);  // -1032, -72
                            pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(hb[0], hb[1], hb[2], hb[3]), pb, 0, 0, 0);
                        } else {
                            uint32_t h0[2], h1[2];
                            int8_word_to_h(u.wq[j][r][2 * q], h0);
                            int8_word_to_h(u.wq[j][r][2 * q + 1], h1);
                            pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(h0[0], h0[1], h1[0], h1[1]), pb, 0, 0, 0);
                        }
                        const uint32_t sw = FMT == FMT_Q4_0 ? u.sv[r][2 * j + (q >> 1)] : u.sv[r][j];
                        const float d = f16_to_f32(static_cast<uint16_t>(sw >> (16 * (q & 1))));
                        if constexpr (ONE) cacc[r][0] += pb[0] * d;
                        else cacc[r] += pb * d;
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if constexpr (ONE) acc[r][0] += cacc[r][0] * post[0];
                    else acc[r] += cacc[r] * post;
                }
            } else if constexpr (FMT == FMT_NF4) {
                floatx4 pacc[R];
#pragma unroll
                for (int r = 0; r < R; ++r) pacc[r] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < WPL; ++t) {
                    const half8_t aop = *reinterpret_cast<const half8_t *>(xa + t * 8);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const uint32_t w = u.wq[j][r][t];
                        const uint2 e0 = lut[w & 255u], e1 = lut[(w >> 8) & 255u];
                        const uint2 e2 = lut[(w >> 16) & 255u], e3 = lut[w >> 24];
                        pacc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(e0.x, e1.x, e2.x, e3.x), pacc[r], 0, 0, 0);
                        pacc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(e0.y, e1.y, e2.y, e3.y), pacc[r], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float am = __builtin_bit_cast(float, u.sv[r][j]);
                    if constexpr (ONE) acc[r][0] += (pacc[r][0] * am) * post[0];
                    else acc[r] += (pacc[r] * am) * post;
                }
            } else {
                floatx4 pacc[R];
#pragma unroll
                for (int r = 0; r < R; ++r) pacc[r] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < WPL / 2; ++t) {
                    const half8_t aop = *reinterpret_cast<const half8_t *>(xa + t * 8);
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        uint32_t h0[2], h1[2];
                        int8_word_to_h(u.wq[j][r][2 * t], h0);
                        int8_word_to_h(u.wq[j][r][2 * t + 1], h1);
                        pacc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(h0[0], h0[1], h1[0], h1[1]),
                                                                        pacc[r], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if constexpr (ONE) acc[r][0] += pacc[r][0] * post[0];
                    else acc[r] += pacc[r] * post;
                }
            }
        }
    };

    constexpr int S = kWaves * NB;  // chunks between a wave's consecutive units
    for (int cs = 0; cs < nchunks; cs += cps) {
        const int ce = cs + cps < nchunks ? cs + cps : nchunks;
        if (cs > 0) {
            __syncthreads();  // every wave is done with the previous stage
            stage_copy(cs, ce);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            stage_convert(cs, ce);
            __syncthreads();
            load_unit(ua, cs + wave * NB, ce);
        }
        // ua holds the unit at cb; the unit at cb + S goes into ub before ua is consumed
        for (int cb = cs + wave * NB; cb < ce; cb += 2 * S) {
            load_unit(ub, cb + S, ce);
            process(ua, cb, cs, ce);
            if (cb + S >= ce) break;
            load_unit(ua, cb + 2 * S, ce);
            process(ub, cb + S, cs, ce);
        }
    }

    // ---- reduce the 4 waves' partial tiles and store ----
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) red[wave - 1][r][lane] = acc[r];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int w = 0; w < kWaves - 1; ++w) acc[r] += red[w][r][lane];
            const int64_t nrow = n0 + 16 * r + lr;
            if (nrow >= N) continue;
            if constexpr (FMT == FMT_INT8) {
                const float *s = static_cast<const float *>(P.scales);
                acc[r] *= P.scale_per_row ? s[nrow] : s[0];
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = part * 4 + q;
                if (m < M) {
                    if (b.y_bf16)
                        static_cast<uint16_t *>(P.y)[static_cast<int64_t>(m) * N + nrow] = f32_to_bf16_rne(acc[r][q]);
                    else
                        static_cast<float *>(P.y)[static_cast<int64_t>(m) * N + nrow] = acc[r][q];
                }
            }
        }
    }
}

// ---- M = 2..64 with x from global memory --------------------------------------------------
// Each wave reads the activation fragments of its own chunks straight from global memory
// (L2: x is a few KB per row) into registers, next to the weight codes of the same unit, and
// converts them to f16 there: per (row, chunk) the power of two of x_scale_of, agreed on by
// the four lanes that hold the row's chunk (xor 16, 32), the post factor of each output row
// fetched from the lane that owns it.  No LDS staging of x, so no pass boundaries and no
// barrier before the final cross-wave sum.  The conversion is shared by the R row tiles of
// the unit; the weight decode and the per-chunk scale handling are those of
// skinny_qgemm_kernel.  Measured (7-matrix block, INT4 g128): M = 2 / 4 / 8 / 16 in 40 / 42 /
// 46 / 52 us, against 57 / 76 us at M = 8 / 16 for the LDS-staged kernel; the limit is the
// VALU work of the x conversion (probe builds without any x or metadata loads run as fast).
// Two waves per SIMD: measured faster than one wave with spill-free registers at R = 4 (52 vs
// 57 us per block at M = 16); the conversion of x is the VALU cost that the second wave hides.
// MT: 16-row tiles of x (M <= 16 MT); each weight word is decoded once for all of them.
template <int FMT, int LW, int R, int NB, int MT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void skinny_gx_kernel(Batch b) {
    constexpr int WPL = LW / 4;
    constexpr int CPB = codes_per_byte<FMT>();
    constexpr int CK = 4 * LW * CPB;   // K elements per chunk
    constexpr int XV = CK / 32;        // 16-byte x loads per lane per chunk
    __shared__ floatx4 red[kWaves - 1][R][MT][64];
    __shared__ uint2 lut[FMT == FMT_NF4 ? 256 : 1];

    int pi = 0;
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
        if (i < b.count && static_cast<int>(blockIdx.x) >= b.p[i].tile_begin) pi = i;
    const Problem &P = b.p[pi];
    const int M = b.m;
    const int64_t N = P.n, K = P.k;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x - P.tile_begin) * 16 * R;
    const int rows_here = static_cast<int>((N - n0) < 16 * R ? (N - n0) : 16 * R);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, part = lane >> 4;
    const uint32_t row_bytes = static_cast<uint32_t>(K / CPB);
    const rsrc_t rc = make_rsrc(static_cast<const uint8_t *>(P.codes) + n0 * row_bytes,
                                static_cast<uint32_t>(rows_here) * row_bytes);
    const int64_t grp = FMT == FMT_INT8 ? CK : P.group;
    const uint32_t G = static_cast<uint32_t>((K + grp - 1) / grp);
    const uint32_t ZW = (G + 7) / 8, GP = ZW * 8;
    const int gshift = is_gguf(FMT) ? 0 : __builtin_ctz(static_cast<uint32_t>(grp / CK));
    rsrc_t rs = make_rsrc(P.codes, 0), rz = rs;
    if constexpr (FMT == FMT_INT4 || is_gguf(FMT))
        rs = make_rsrc(static_cast<const uint16_t *>(P.scales) + n0 * GP, static_cast<uint32_t>(rows_here) * GP * 2);
    if constexpr (FMT == FMT_INT4) {
        rz = make_rsrc(P.zeros + n0 * ZW, static_cast<uint32_t>(rows_here) * ZW * 4);
    } else if constexpr (FMT == FMT_NF4) {
        rs = make_rsrc(static_cast<const float *>(P.scales) + n0 * G, static_cast<uint32_t>(rows_here) * G * 4);
    }
    // x [M, K] bf16: this lane's rows 16 mt + lr (rows >= M read zero) and its part of each
    // chunk (GGUF: elements 8 part .. + 7 of each 32-block; others: a contiguous quarter)
    const rsrc_t rx = make_rsrc(P.x, static_cast<uint32_t>(M * K * 2));
    uint32_t x_off[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int row = 16 * mt + lr;
        x_off[mt] = row < M ? static_cast<uint32_t>(row * K + (is_gguf(FMT) ? 8 * part : part * (CK / 4))) * 2u
                            : kOobGx;
    }
    uint32_t code_off[R], sc_off[R], z_off[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = 16 * r + lr;
        code_off[r] = row * row_bytes + part * LW;
        sc_off[r] = row * ((FMT == FMT_INT4 || is_gguf(FMT)) ? GP : G);
        z_off[r] = row * ZW;
    }

    const int nchunks = static_cast<int>(K / CK);
    struct Unit {
        uint32_t wq[NB][R][WPL];
        uint32_t sv[R][FMT == FMT_Q4_0 ? 2 * NB : NB];
        uint32_t zv[R];
        uint4 xv[NB][MT][XV];
    };
    // unit k of this wave: chunks c0 = (wave + k kWaves) NB .. + NB - 1; chunks past K read
    // nothing (offsets past the descriptors), so every unit issues the same loads
    auto load_unit = [&](Unit &u, int k) {
        const int c0 = (wave + k * kWaves) * NB;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int c = c0 + j;
            const bool in = c < nchunks;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int h = 0; h < XV; ++h) {
                    const uint32_t xo = static_cast<uint32_t>(c * CK + (is_gguf(FMT) ? 32 * h : 8 * h)) * 2u;
                    u.xv[j][mt][h] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                   rx, in ? x_off[mt] + xo : kOobGx, 0, 0));
                }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                load_words<LW>(rc, in ? code_off[r] + static_cast<uint32_t>(c) * (CK / CPB) : kOobGx, u.wq[j][r]);
                if constexpr (FMT == FMT_Q4_0) {
                    const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                                  rs, in ? (sc_off[r] + static_cast<uint32_t>(c) * 4u) * 2u : kOobGx, 0, 0));
                    u.sv[r][2 * j] = v.x;
                    u.sv[r][2 * j + 1] = v.y;
                } else if constexpr (FMT == FMT_Q8_0) {
                    u.sv[r][j] = __builtin_amdgcn_raw_buffer_load_b32(
                        rs, in ? (sc_off[r] + static_cast<uint32_t>(c) * 2u) * 2u : kOobGx, 0, 0);
                } else if constexpr (FMT == FMT_NF4) {
                    u.sv[r][j] = __builtin_amdgcn_raw_buffer_load_b32(
                        rs, in ? (sc_off[r] + (static_cast<uint32_t>(c) >> gshift)) * 4 : kOobGx, 0, 0);
                }
            }
        }
        if constexpr (FMT == FMT_INT4) {
            // the unit's NB scales in one aligned load and its 8-group zero word (a unit past
            // the end reads nothing)
            const uint32_t um = c0 < nchunks ? 0u : kOobGx;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t so = ((sc_off[r] + static_cast<uint32_t>(c0)) * 2) | um;
                if constexpr (NB == 4) {
                    const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, so, 0, 0));
                    u.sv[r][0] = v.x;
                    u.sv[r][1] = v.y;
                } else if constexpr (NB == 2) {
                    u.sv[r][0] = __builtin_amdgcn_raw_buffer_load_b32(rs, so, 0, 0);
                } else {
                    static_assert(NB == 1, "INT4 units hold 1, 2 or 4 chunks");
                    u.sv[r][0] = __builtin_amdgcn_raw_buffer_load_b16(rs, so, 0, 0);
                }
                u.zv[r] = __builtin_amdgcn_raw_buffer_load_b32(rz, ((z_off[r] + (static_cast<uint32_t>(c0) >> 3)) * 4) | um,
                                                               0, 0);
            }
        }
    };

    // units of this wave (the same count for every path through the loop below)
    const int U = __builtin_amdgcn_readfirstlane((nchunks + kWaves * NB - 1) / (kWaves * NB));
    Unit ua, ub;
    load_unit(ua, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (FMT == FMT_NF4) {
        for (int i = tid; i < 256; i += kThreads) {
            const _Float16 h0 = static_cast<_Float16>(kNf4[i & 15]), h1 = static_cast<_Float16>(kNf4[i >> 4]);
            const _Float16 l0 = static_cast<_Float16>(kNf4[i & 15] - static_cast<float>(h0));
            const _Float16 l1 = static_cast<_Float16>(kNf4[i >> 4] - static_cast<float>(h1));
            half2_t hi = {h0, h1}, lo = {l0, l1};
            lut[i] = make_uint2(as_u(hi), as_u(lo));
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));  // the table's LDS writes
        __builtin_amdgcn_s_barrier();
    }

    floatx4 acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[r][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
    const Int4Consts i4k = int4_consts();
    const floatx4 zero4 = floatx4{0.f, 0.f, 0.f, 0.f};

    // a chunk past K read zero codes, zero x and zero metadata; its sums are dropped by a select
    auto process = [&](const Unit &u, int k) {
        const int cb = (wave + k * kWaves) * NB;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int c = cb + j;
            const bool live = c < nchunks;
            // x of this chunk, per x tile: f16 scaled by each row's power of two for the chunk,
            // and the post factor of this lane's output rows 16 mt + 4 part + q (from lane 4 part + q)
            half8_t a[MT][XV];
            floatx4 post[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                uint32_t e = 0;
#pragma unroll
                for (int h = 0; h < XV; ++h) {
                    const uint32_t wv[4] = {u.xv[j][mt][h].x, u.xv[j][mt][h].y, u.xv[j][mt][h].z, u.xv[j][mt][h].w};
                    e = max(e, bf16x8_emax(wv));
                }
                e = max(e, static_cast<uint32_t>(__shfl_xor(static_cast<int>(e), 16)));
                e = max(e, static_cast<uint32_t>(__shfl_xor(static_cast<int>(e), 32)));
                float pre, pst;
                x_scale_of(e, pre, pst);
#pragma unroll
                for (int h = 0; h < XV; ++h) {
                    const uint32_t wv[4] = {u.xv[j][mt][h].x, u.xv[j][mt][h].y, u.xv[j][mt][h].z, u.xv[j][mt][h].w};
                    uint32_t o[4];
                    bf16x8_to_f16_perm(FMT, wv, pre, o);
                    a[mt][h] = pack8(o[0], o[1], o[2], o[3]);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) post[mt][q] = __shfl(pst, 4 * part + q);
            }
            if constexpr (FMT == FMT_INT4) {
                const uint32_t gsh = 4 * (static_cast<uint32_t>(c) & 7u);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t z = (u.zv[r] >> gsh) & 15u;
                    const uint32_t zc1024 = (0xE400u + z) * 0x00010001u, zc64 = (0xD400u + (z << 4)) * 0x00010001u;
                    floatx4 pacc[MT];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) pacc[mt] = zero4;
#pragma unroll
                    for (int t = 0; t < WPL; ++t) {
                        uint32_t hb[4];
                        int4_word_to_h(u.wq[j][r][t], as_h2(zc1024), as_h2(zc64), i4k, hb);
                        const half8_t bw = pack8(hb[0], hb[1], hb[2], hb[3]);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            pacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][t], bw, pacc[mt], 0, 0, 0);
                    }
                    const float sc = f16_to_f32(static_cast<uint16_t>(u.sv[r][j >> 1] >> (16 * (j & 1))));
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const floatx4 v = (pacc[mt] * sc) * post[mt];
                        acc[r][mt] += live ? v : zero4;
                    }
                }
            } else if constexpr (is_gguf(FMT)) {
                constexpr int BPC = gguf_bpc(FMT);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    floatx4 cacc[MT];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) cacc[mt] = zero4;
#pragma unroll
                    for (int q = 0; q < BPC; ++q) {
                        half8_t bw;
                        if constexpr (FMT == FMT_Q4_0) {
                            uint32_t hb[4];
                            int4_word_to_h(u.wq[j][r][q], as_h2(0xE408E408u), as_h2(0xD480D480u), i4k, hb);  // -1032, -72
                            bw = pack8(hb[0], hb[1], hb[2], hb[3]);
                        } else {
                            uint32_t h0[2], h1[2];
                            int8_word_to_h(u.wq[j][r][2 * q], h0);
                            int8_word_to_h(u.wq[j][r][2 * q + 1], h1);
                            bw = pack8(h0[0], h0[1], h1[0], h1[1]);
                        }
                        const uint32_t sw = FMT == FMT_Q4_0 ? u.sv[r][2 * j + (q >> 1)] : u.sv[r][j];
                        const float d = f16_to_f32(static_cast<uint16_t>(sw >> (16 * (q & 1))));
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            cacc[mt] += __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][q], bw, zero4, 0, 0, 0) * d;
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const floatx4 v = cacc[mt] * post[mt];
                        acc[r][mt] += live ? v : zero4;
                    }
                }
            } else if constexpr (FMT == FMT_NF4) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    floatx4 pacc[MT];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) pacc[mt] = zero4;
#pragma unroll
                    for (int t = 0; t < WPL; ++t) {
                        const uint32_t w = u.wq[j][r][t];
                        const uint2 e0 = lut[w & 255u], e1 = lut[(w >> 8) & 255u];
                        const uint2 e2 = lut[(w >> 16) & 255u], e3 = lut[w >> 24];
                        const half8_t bh = pack8(e0.x, e1.x, e2.x, e3.x), bl = pack8(e0.y, e1.y, e2.y, e3.y);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            pacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][t], bh, pacc[mt], 0, 0, 0);
                            pacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][t], bl, pacc[mt], 0, 0, 0);
                        }
                    }
                    const float am = __builtin_bit_cast(float, u.sv[r][j]);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const floatx4 v = (pacc[mt] * am) * post[mt];
                        acc[r][mt] += live ? v : zero4;
                    }
                }
            } else {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    floatx4 pacc[MT];
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) pacc[mt] = zero4;
#pragma unroll
                    for (int t = 0; t < WPL / 2; ++t) {
                        uint32_t h0[2], h1[2];
                        int8_word_to_h(u.wq[j][r][2 * t], h0);
                        int8_word_to_h(u.wq[j][r][2 * t + 1], h1);
                        const half8_t bw = pack8(h0[0], h0[1], h1[0], h1[1]);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
                            pacc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mt][t], bw, pacc[mt], 0, 0, 0);
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        const floatx4 v = pacc[mt] * post[mt];
                        acc[r][mt] += live ? v : zero4;
                    }
                }
            }
        }
    };

    // unit k in ua, unit k + 1 in ub: one exit, no branch and no load under a branch in the
    // body, so the compiler's vmcnt waits cover only the unit being consumed
    for (int k = 0; k < U; k += 2) {
        load_unit(ub, k + 1);
        __builtin_amdgcn_sched_barrier(0);
        process(ua, k);
        load_unit(ua, k + 2);
        __builtin_amdgcn_sched_barrier(0);
        process(ub, k + 1);
    }

    // ---- reduce the 4 waves' partial tiles and store ----
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) red[wave - 1][r][mt][lane] = acc[r][mt];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t nrow = n0 + 16 * r + lr;
            float s = 1.0f;
            if constexpr (FMT == FMT_INT8) {
                const float *sp = static_cast<const float *>(P.scales);
                s = nrow < N ? sp[P.scale_per_row ? nrow : 0] : 0.0f;
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                floatx4 v = acc[r][mt];
#pragma unroll
                for (int w = 0; w < kWaves - 1; ++w) v += red[w][r][mt][lane];
                if (nrow >= N) continue;
                if constexpr (FMT == FMT_INT8) v *= s;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int m = 16 * mt + part * 4 + q;
                    if (m < M) {
                        if (b.y_bf16)
                            static_cast<uint16_t *>(P.y)[static_cast<int64_t>(m) * N + nrow] = f32_to_bf16_rne(v[q]);
                        else
                            static_cast<float *>(P.y)[static_cast<int64_t>(m) * N + nrow] = v[q];
                    }
                }
            }
        }
    }
}

// ---- M = 1 split-K kernel ------------------------------------------------------------------
// Decode (M = 1): one workgroup per 16-row tile, each of its 4 waves owning a contiguous
// quarter of K (whole units of NB chunks) and its own LDS region, so no wave waits for
// another before the final cross-wave sum.  A wave first copies, straight into its region
// (buffer loads to LDS, 16 bytes per lane), the scales and zero points of its groups for the
// 16 rows and its slice of x; then it issues the code loads of its first kSplitDepth units,
// waits for the copies alone (vmcnt drains in issue order), converts the x slice in place to
// permuted f16, and from then on keeps kSplitDepth - 1 units in flight while it consumes one.
// The main loop loads codes only: metadata read per unit would be a 4-byte access to each of
// 16 rows, as many memory requests as the codes themselves.  The loop has one exit, no branch
// inside and no load under a branch, so the compiler's vmcnt waits cover only the unit being
// consumed (an early exit, even a uniform one, turns the loop into exec-mask flow whose
// merges wait for loads in flight).
#ifndef CFH_GEMV_NB_SPLIT
#define CFH_GEMV_NB_SPLIT 2
#endif
#ifndef CFH_GEMV_DEPTH_SPLIT
#define CFH_GEMV_DEPTH_SPLIT 2
#endif
constexpr int kSplitDepth = CFH_GEMV_DEPTH_SPLIT;

// Metadata copies: bytes [lo, lo + 16 * pieces) of each of the 16 rows' metadata arrays, in
// 16-byte pieces; copy i moves pieces 4i .. 4i + 3 of every row into 1 KB of LDS, lane
// (row r, part p) writing piece 4i + p of row r at i * 1024 + (16 p + r) * 16.
__device__ __forceinline__ uint32_t meta_lds_off(uint32_t b, int r) {
    const uint32_t p = b >> 4;
    return (p >> 2) * 1024u + ((p & 3u) * 16u + static_cast<uint32_t>(r)) * 16u + (b & 15u);
}

// Sum over aligned groups of N lanes (N = 4 or 8), every lane of a group receiving it: DPP
// quad permutations (xor 1, xor 2) and the half-row mirror (lane i <-> 7 - i within 8 lanes,
// which pairs each quad with the other quad of its 8) instead of LDS permutes.
template <int N>
__device__ __forceinline__ float lane_group_sum(float v) {
    static_assert(N == 4 || N == 8, "group of 4 or 8 lanes");
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    if constexpr (N == 8)
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    return v;
}

// waves per SIMD the split kernel's register budget is sized for (0: the compiler's choice)
#ifndef CFH_GEMV_SPLIT_WPE
#define CFH_GEMV_SPLIT_WPE 5
#endif
template <int FMT, int LW>
__global__ __launch_bounds__(kThreads)
#if CFH_GEMV_SPLIT_WPE
// (INT4 with 16-byte lanes decodes four words per chunk to exact (q - z): 4 waves per SIMD
// give it the registers to do so without spilling)
__attribute__((amdgpu_waves_per_eu(FMT == FMT_INT4 && LW == 16 ? 4 : CFH_GEMV_SPLIT_WPE)))
#endif
void skinny_m1_split_kernel(Batch b) {
    constexpr int WPL = LW / 4;
    constexpr int CPB = codes_per_byte<FMT>();
    constexpr int CK = 4 * LW * CPB;
    constexpr int NB = CFH_GEMV_NB_SPLIT;
    constexpr int D = kSplitDepth;
    constexpr uint32_t kOob = 0x80000000u;  // past every descriptor's range: reads zero, no traffic
    extern __shared__ __align__(16) uint8_t lds[];  // [kWaves][region]: x slice, scales, zero points
    __shared__ float red[kWaves][64];
    __shared__ uint2 lut[FMT == FMT_NF4 ? kWaves * 256 : 1];  // NF4: one table per wave

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = uni(tid >> 6);
    const int lr = lane & 15, part = lane >> 4;

    int pi = 0;
#pragma unroll
    for (int i = 1; i < kMaxProblems; ++i)
        if (i < b.count && static_cast<int>(blockIdx.x) >= b.p[i].tile_begin) pi = i;
    const Problem &P = b.p[pi];
    const int64_t N = P.n, K = P.k;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x - P.tile_begin) * 16;
    const uint32_t rows = static_cast<uint32_t>((N - n0) < 16 ? (N - n0) : 16);
    const uint32_t row_bytes = static_cast<uint32_t>(uni(static_cast<int>(K / CPB)));
    const rsrc_t rc = make_rsrc_u(static_cast<const uint8_t *>(P.codes) + n0 * row_bytes, rows * row_bytes);
    const int64_t grp = FMT == FMT_INT8 ? CK : P.group;  // INT8 has no groups (group 0)
    const uint32_t Gr = static_cast<uint32_t>(uni(static_cast<int>((K + grp - 1) / grp)));
    const uint32_t ZW = (Gr + 7) / 8, GP = ZW * 8;
    const int gshift = is_gguf(FMT) ? 0 : uni(__builtin_ctz(static_cast<uint32_t>(grp / CK)));
    const uint32_t code_off = static_cast<uint32_t>(lr) * row_bytes + part * LW;

    // this wave's units [u0, u1) and chunks [c_lo, c_hi)
    const int nchunks = uni(static_cast<int>(K / CK));
    const int nunits = (nchunks + NB - 1) / NB;
    const int u0 = uni(wave * nunits / kWaves), u1 = uni((wave + 1) * nunits / kWaves);
    const int U = u1 - u0;
    const int c_lo = u0 * NB;
    const int c_hi = u1 * NB < nchunks ? u1 * NB : nchunks;
    uint8_t *const reg = lds + wave * P.kc;  // kc: region bytes per wave
    _Float16 *const xw = reinterpret_cast<_Float16 *>(reg);
    const uint8_t *const ms = reg + P.soff;  // scale (INT4) / absmax (NF4) pieces
    const uint8_t *const mz = reg + P.zoff;  // zero-point pieces (INT4)
    float *const xpost = reinterpret_cast<float *>(reg + P.xsoff);  // per chunk of the slice
    uint2 *const wl = lut + (FMT == FMT_NF4 ? wave * 256 : 0);

    // NF4 decode table (hi, lo f16 pairs of two codes), written before any copy into LDS is
    // issued: an LDS write after an LDS-bound copy is made to wait for every load in flight
    if constexpr (FMT == FMT_NF4) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int i = lane + 64 * q;
            const _Float16 h0 = static_cast<_Float16>(kNf4[i & 15]), h1 = static_cast<_Float16>(kNf4[i >> 4]);
            const _Float16 l0 = static_cast<_Float16>(kNf4[i & 15] - static_cast<float>(h0));
            const _Float16 l1 = static_cast<_Float16>(kNf4[i >> 4] - static_cast<float>(h1));
            half2_t hi = {h0, h1}, lo = {l0, l1};
            wl[i] = make_uint2(as_u(hi), as_u(lo));
        }
    }

    // metadata of the wave's groups: first byte (16-byte aligned) of the span in each row
    uint32_t s_lo = 0, z_lo = 0;
    if (c_hi > c_lo) {
        auto copy_span = [&](const void *base, uint32_t row_stride, uint32_t lo, uint32_t hi, const uint8_t *dst) {
            const rsrc_t r = make_rsrc_u(static_cast<const uint8_t *>(base) + n0 * row_stride, rows * row_stride);
            const int pieces = static_cast<int>((hi - lo + 15) / 16);
            for (int i = 0; i * 4 < pieces; ++i) {  // wave-uniform
                const int p = 4 * i + part;
                const uint32_t off = (static_cast<uint32_t>(lr) * row_stride + lo + 16u * p) | (p < pieces ? 0u : kOob);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    r, reinterpret_cast<__attribute__((address_space(3))) void *>(reinterpret_cast<uintptr_t>(dst) + i * 1024),
                    16, off, 0, 0, 0);
            }
        };
        if constexpr (FMT == FMT_INT4) {
            s_lo = (static_cast<uint32_t>(c_lo) * 2u) & ~15u;
            copy_span(P.scales, GP * 2, s_lo, static_cast<uint32_t>(c_hi) * 2u, ms);
            z_lo = (static_cast<uint32_t>(c_lo >> 3) * 4u) & ~15u;
            copy_span(P.zeros, ZW * 4, z_lo, static_cast<uint32_t>(((c_hi - 1) >> 3) + 1) * 4u, mz);
        } else if constexpr (FMT == FMT_NF4) {
            s_lo = (static_cast<uint32_t>(c_lo >> gshift) * 4u) & ~15u;
            copy_span(P.scales, Gr * 4, s_lo, static_cast<uint32_t>(((c_hi - 1) >> gshift) + 1) * 4u, ms);
        } else if constexpr (is_gguf(FMT)) {
            constexpr uint32_t SB = 2 * gguf_bpc(FMT);  // scale bytes per chunk
            s_lo = (static_cast<uint32_t>(c_lo) * SB) & ~15u;
            copy_span(P.scales, GP * 2, s_lo, static_cast<uint32_t>(c_hi) * SB, ms);
        }
    }
    // x slice: bf16 x[c_lo * CK, c_hi * CK) copied straight into the region
    {
        const int bytes = (c_hi > c_lo ? c_hi - c_lo : 0) * CK * 2;
        const uint16_t *src = P.x + static_cast<int64_t>(c_lo) * CK;
        for (int blk = 0; blk * 1024 < bytes; ++blk) {  // wave-uniform
            const int e = blk * 1024 + lane * 16;
            if (e < bytes)
                __builtin_amdgcn_global_load_lds(
                    static_cast<const void *>(src + (e >> 1)),
                    reinterpret_cast<__attribute__((address_space(3))) void *>(reinterpret_cast<uintptr_t>(xw) + blk * 1024),
                    16, 0, 0);
        }
    }

    struct Unit {
        uint32_t wq[NB][WPL];
    };
    // Unit k of this wave (k >= U: past the wave's range, reads nothing).  Offsets are computed
    // unconditionally and pushed out of range by OR-ing in kOob (every real offset is below
    // 2^31): a select between an offset and kOob would be compiled as a branch.
    auto load_unit = [&](Unit &u, int k) {
        const uint32_t c0 = static_cast<uint32_t>((u0 + k) * NB);
        const uint32_t okm = k < U ? 0u : kOob;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint32_t m = (static_cast<int>(c0) + j < nchunks) ? okm : kOob;
            load_words<LW>(rc, (code_off + (c0 + j) * (CK / CPB)) | m, u.wq[j]);
        }
    };
    Unit ub[D];
#pragma unroll
    for (int i = 0; i < D; ++i) {
        load_unit(ub[i], i);
        __builtin_amdgcn_sched_barrier(0);  // unit by unit, in the order they are consumed
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(D * NB));  // the copies into LDS have landed
    {
        // x slice -> f16 in the extraction order, each chunk scaled by its own power of two
        // (x_scale_of); the CK / 8 runs of a chunk sit on CK / 8 consecutive lanes
        const int runs = (c_hi > c_lo ? c_hi - c_lo : 0) * CK / 8;
        for (int it = lane; it < runs; it += 64) {
            const uint4 raw = *reinterpret_cast<const uint4 *>(xw + it * 8);
            const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
            float pre, post;
            x_scale_of(lane_group_max<CK / 8>(bf16x8_emax(wv)), pre, post);
            uint32_t o[4];
            bf16x8_to_f16_perm(FMT, wv, pre, o);
            *reinterpret_cast<uint4 *>(xw + it * 8) = make_uint4(o[0], o[1], o[2], o[3]);
            if ((it & (CK / 8 - 1)) == 0) xpost[it / (CK / 8)] = post;
        }
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));  // this wave's LDS writes are done

    const Int4Consts i4k = int4_consts();
    float acc = 0.0f;  // slot 0 of the 16x16 MFMA tile: row lr of this tile (lanes with part 0)
    // A chunk past K (the last unit may be partial) or of a unit past the wave's range reads
    // zero codes and takes its x and metadata from the wave's first chunk; its sum is dropped
    // by a select (no branch, so no path leaves a unit's registers unread).
    auto process = [&](const Unit &u, int k) {
        const int cb = (u0 + k) * NB;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const bool live = k < U && cb + j < nchunks;
            const int c = live ? cb + j : c_lo;
            const _Float16 *xa = xw + (c - c_lo) * CK + part * (CK / 4);
            const float post = xpost[c - c_lo];
            floatx4 pacc = floatx4{0.f, 0.f, 0.f, 0.f};
            if constexpr (FMT == FMT_INT4) {  // exact (q - z) codes
                const uint32_t zw = *reinterpret_cast<const uint32_t *>(
                    mz + meta_lds_off(static_cast<uint32_t>(c >> 3) * 4u - z_lo, lr));
                const uint32_t z = (zw >> (4 * (static_cast<uint32_t>(c) & 7u))) & 15u;
                const uint32_t zc1024 = (0xE400u + z) * 0x00010001u, zc64 = (0xD400u + (z << 4)) * 0x00010001u;
#pragma unroll
                for (int q = 0; q < WPL; ++q) {
                    const half8_t aop = *reinterpret_cast<const half8_t *>(xa + q * 8);
                    uint32_t hb[4];
                    int4_word_to_h(u.wq[j][q], as_h2(zc1024), as_h2(zc64), i4k, hb);
                    pacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(hb[0], hb[1], hb[2], hb[3]), pacc, 0, 0, 0);
                }
                const float sc = f16_to_f32(*reinterpret_cast<const uint16_t *>(
                    ms + meta_lds_off(static_cast<uint32_t>(c) * 2u - s_lo, lr)));
                const float v = (pacc[0] * sc) * post;
                acc += live ? v : 0.0f;
            } else if constexpr (FMT == FMT_NF4) {
#pragma unroll
                for (int q = 0; q < WPL; ++q) {
                    const half8_t aop = *reinterpret_cast<const half8_t *>(xa + q * 8);
                    const uint32_t w = u.wq[j][q];
                    const uint2 e0 = wl[w & 255u], e1 = wl[(w >> 8) & 255u];
                    const uint2 e2 = wl[(w >> 16) & 255u], e3 = wl[w >> 24];
                    pacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(e0.x, e1.x, e2.x, e3.x), pacc, 0, 0, 0);
                    pacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(e0.y, e1.y, e2.y, e3.y), pacc, 0, 0, 0);
                }
                const float am = *reinterpret_cast<const float *>(
                    ms + meta_lds_off(static_cast<uint32_t>(c >> gshift) * 4u - s_lo, lr));
                const float v = (pacc[0] * am) * post;
                acc += live ? v : 0.0f;
            } else if constexpr (is_gguf(FMT)) {
                // One MFMA per 32-element block: the four parts of a row hold elements 8p..8p+7
                // of each block of the chunk, so the MFMA's K sum is that block's exact-code dot
                // product, scaled in f32 by the block's d.  Q4_0 codes decode to q - 8 exactly.
                constexpr int BPC = gguf_bpc(FMT);
                const uint8_t *sp = ms + meta_lds_off(static_cast<uint32_t>(c) * (2u * BPC) - s_lo, lr);
                uint32_t sv[BPC / 2];
                if constexpr (BPC == 4) {
                    const uint2 s2 = *reinterpret_cast<const uint2 *>(sp);
                    sv[0] = s2.x;
                    sv[1] = s2.y;
                } else {
                    sv[0] = *reinterpret_cast<const uint32_t *>(sp);
                }
                const _Float16 *xc = xw + (c - c_lo) * CK + 8 * part;
                float cs = 0.0f;
#pragma unroll
                for (int q = 0; q < BPC; ++q) {
                    const half8_t aop = *reinterpret_cast<const half8_t *>(xc + 32 * q);
                    floatx4 pb = floatx4{0.f, 0.f, 0.f, 0.f};
                    if constexpr (FMT == FMT_Q4_0) {
                        uint32_t hb[4];
                        int4_word_to_h(u.wq[j][q], as_h2(0xE408E408u), as_h2(0xD480D480u), i4k, hb);  // -1032, -72
                        pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(hb[0], hb[1], hb[2], hb[3]), pb, 0, 0, 0);
                    } else {
                        uint32_t h0[2], h1[2];
                        int8_word_to_h(u.wq[j][2 * q], h0);
                        int8_word_to_h(u.wq[j][2 * q + 1], h1);
                        pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(h0[0], h0[1], h1[0], h1[1]), pb, 0, 0, 0);
                    }
                    const float d = f16_to_f32(static_cast<uint16_t>(sv[q >> 1] >> (16 * (q & 1))));
                    cs += pb[0] * d;
                }
                const float v = cs * post;
                acc += live ? v : 0.0f;
            } else {
#pragma unroll
                for (int q = 0; q < WPL / 2; ++q) {
                    const half8_t aop = *reinterpret_cast<const half8_t *>(xa + q * 8);
                    uint32_t h0[2], h1[2];
                    int8_word_to_h(u.wq[j][2 * q], h0);
                    int8_word_to_h(u.wq[j][2 * q + 1], h1);
                    pacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, pack8(h0[0], h0[1], h1[0], h1[1]), pacc, 0, 0, 0);
                }
                const float v = pacc[0] * post;
                acc += live ? v : 0.0f;
            }
        }
    };

    // unit k sits in ub[k % D]: consumed, then refilled with unit k + D (past the wave's range
    // the refill reads nothing and the unit adds zero)
    for (int k = 0; k < U; k += D) {
#pragma unroll
        for (int i = 0; i < D; ++i) {
            process(ub[i], k + i);
            load_unit(ub[i], k + i + D);
            __builtin_amdgcn_sched_barrier(0);  // the refill stays ahead of the next unit's waits
        }
    }

    // cross-wave sum; lanes 0..15 of wave 0 store rows n0 .. n0 + 15 (a store past N, or from
    // a lane without a row, goes to an offset the descriptor drops)
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        float v = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
        if constexpr (FMT == FMT_INT8) {
            const rsrc_t rs = P.scale_per_row ? make_rsrc_u(static_cast<const float *>(P.scales) + n0, rows * 4)
                                              : make_rsrc_u(P.scales, 4);
            v *= __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                               rs, lane < 16 ? (P.scale_per_row ? lane * 4u : 0u) : kOob, 0, 0));
        }
        const int esz = b.y_bf16 ? 2 : 4;
        const rsrc_t ry = make_rsrc_u(static_cast<const uint8_t *>(P.y) + n0 * esz, rows * esz);
        const uint32_t off = lane < 16 ? static_cast<uint32_t>(lane * esz) : kOob;
        if (b.y_bf16) __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_rne(v), ry, off, 0, 0);
        else __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry, off, 0, 0);
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
    const int64_t G = (FMT == FMT_INT4) ? (K + P.group - 1) / P.group : 0, ZW = (G + 7) / 8, GP = ZW * 8;
    const int64_t NBLK = (FMT == FMT_NF4) ? (K + P.group - 1) / P.group : 0;
    const int64_t GPg = (K / 32 + 7) / 8 * 8;  // GGUF planes: scale row stride
    for (int64_t k = lane; k < K; k += 64) {
        float w;
        if constexpr (is_gguf(FMT)) {
            // element k sits in chunk k / CKg, block q, part p, slot i of the GGUF planes
            constexpr int BPC = gguf_bpc(FMT), CKg = 32 * BPC;
            const int64_t c = k / CKg;
            const int r = static_cast<int>(k % CKg), q = r >> 5, p = (r & 31) >> 3, i = r & 7;
            const uint8_t *row = static_cast<const uint8_t *>(P.codes) + n * (FMT == FMT_Q4_0 ? K / 2 : K);
            const float d = f16_to_f32(static_cast<const uint16_t *>(P.scales)[n * GPg + (k >> 5)]);
            if constexpr (FMT == FMT_Q4_0) {
                const uint32_t b = row[c * 64 + 16 * p + 4 * q + (i >> 1)];
                w = static_cast<float>(static_cast<int32_t>((b >> (4 * (i & 1))) & 15u) - 8) * d;
            } else {
                w = static_cast<float>(static_cast<const int8_t *>(static_cast<const void *>(row))[c * 64 + 16 * p + 8 * q + i]) * d;
            }
        } else if constexpr (FMT == FMT_INT8) {
            w = static_cast<float>(static_cast<const int8_t *>(P.codes)[n * K + k]);
        } else {
            const uint32_t word = static_cast<const uint32_t *>(P.codes)[n * (K / 8) + k / 8];
            const uint32_t q = (word >> (4 * (k & 7))) & 15u;
            if constexpr (FMT == FMT_INT4) {
                const int64_t g = k / P.group;
                const int32_t z = static_cast<int32_t>((P.zeros[n * ZW + (g >> 3)] >> (4 * (g & 7))) & 15u);
                w = static_cast<float>(static_cast<int32_t>(q) - z) *
                    f16_to_f32(static_cast<const uint16_t *>(P.scales)[n * GP + g]);
            } else {
                w = kNf4[q] * static_cast<const float *>(P.scales)[n * NBLK + k / P.group];
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

// Bytes each lane loads per chunk for this format / group (0 = no MFMA path).
int lw_for(int fmt, int64_t group) {
    if (fmt == FMT_INT8) return 16;
    if (is_gguf(fmt)) return group == 32 ? 16 : 0;
    // the chunk index maps to the group by a shift: group / chunk must be a power of two
    if (group >= 128 && group % 128 == 0 && ((group / 128) & (group / 128 - 1)) == 0) return 16;
    if (group == 64) return 8;
    if (group == 32) return 4;
    return 0;
}

int chunk_k(int fmt, int lw) { return 4 * lw * (fmt == FMT_INT8 || fmt == FMT_Q8_0 ? 1 : 2); }

// LDS bytes of one wave of the M = 1 split-K kernel: its x slice, then its groups' scale and
// zero-point pieces (1 KB per copy of 4 pieces of 16 bytes per row); bounds over the waves'
// ranges.  Sets the problem's region offsets.
int64_t split_region(int fmt, int lw, Problem &p) {
    const int ck = chunk_k(fmt, lw);
    auto copies = [](int64_t span) { return ((span + 15) / 16 + 3) / 4; };
    const int64_t nunits = (p.k / ck + CFH_GEMV_NB_SPLIT - 1) / CFH_GEMV_NB_SPLIT;
    const int64_t cw = (nunits + kWaves - 1) / kWaves * CFH_GEMV_NB_SPLIT;  // chunks per wave, at most
    const int64_t xbytes = (cw * ck * 2 + 255) / 256 * 256;
    const int64_t tbytes = (cw * 4 + 255) / 256 * 256;  // activation post factor per chunk
    int64_t sbytes = 0, zbytes = 0;
    if (fmt == FMT_INT4) {
        sbytes = 1024 * copies(2 * cw + 14);
        zbytes = 1024 * copies(4 * ((cw + 7) / 8 + 1) + 12);
    } else if (fmt == FMT_NF4) {
        const int64_t cpb = p.group / ck;  // chunks per absmax block
        sbytes = 1024 * copies(4 * ((cw + cpb - 1) / cpb + 1) + 12);
    } else if (is_gguf(fmt)) {
        sbytes = 1024 * copies(2 * gguf_bpc(fmt) * cw + 14);
    }
    p.kc = static_cast<int32_t>(xbytes + tbytes + sbytes + zbytes);
    p.xsoff = static_cast<int32_t>(xbytes);
    p.soff = static_cast<int32_t>(xbytes + tbytes);
    p.zoff = static_cast<int32_t>(xbytes + tbytes + sbytes);
    return xbytes + tbytes + sbytes + zbytes;
}

// M = 1..64 (M = 1: split or per-tile kernel; M = 2..64: skinny_gx_kernel, whose x descriptor
// spans M * K bf16 with 32-bit offsets)
bool skinny_ok(int fmt, const Problem &p, int64_t m) {
    if (m < 1 || m > 64 || m * p.k * 2 >= (int64_t{1} << 31)) return false;
    if (is_gguf(fmt)) {
        if (p.group != 32) return false;
        if (p.k % chunk_k(fmt, 16) != 0 || p.k >= (int64_t{1} << 24)) return false;
        return aligned(p.x, 16) && aligned(p.codes, 16) && aligned(p.scales, 16);
    }
    const int lw = lw_for(fmt, p.group);
    if (lw == 0) return false;
    if (p.k % chunk_k(fmt, lw) != 0) return false;
    // INT4 metadata is loaded per unit of consecutive groups: one group per chunk
    if (fmt == FMT_INT4 && p.group != chunk_k(fmt, lw)) return false;
    if (p.k >= (int64_t{1} << 24)) return false;  // 32-bit buffer offsets over 64 rows
    return aligned(p.x, 16) && aligned(p.codes, 16);
}

// Bytes of the per-(chunk, row) activation post factors that follow a stage of kc elements.
int64_t xpost_bytes(int64_t kc, int64_t m, int ck) { return kc / ck * ((m + 3) / 4 * 4) * 4; }

// K elements staged per LDS pass: a whole number of units (unit = nb chunks of ck elements);
// the stage (m rows of kc f16) fills kLdsBytesMax, its post factors come on top
int32_t kc_for(int64_t k, int64_t m, int ck, int nb) {
    const int64_t unit = static_cast<int64_t>(ck) * nb;
    int64_t kc = (kLdsBytesMax / 2) / m;
    kc = (kc / unit) * unit;
    if (kc < unit) kc = unit;
    return static_cast<int32_t>(kc < k ? kc : k);
}

template <int FMT, int LW, int R>
void launch_one(const Batch &b, int64_t tiles, int64_t lds, hipStream_t st) {
    if (R != 4 && b.m == 1)
        skinny_qgemm_kernel<FMT, LW, R, true><<<dim3(static_cast<unsigned>(tiles)), dim3(kThreads),
                                                static_cast<size_t>(lds), st>>>(b);
    else
        skinny_qgemm_kernel<FMT, LW, R, false><<<dim3(static_cast<unsigned>(tiles)), dim3(kThreads),
                                                 static_cast<size_t>(lds), st>>>(b);
}

template <int FMT, int R>
void launch_lw(int lw, const Batch &b, int64_t tiles, int64_t lds, hipStream_t st) {
    if (lw == 16) launch_one<FMT, 16, R>(b, tiles, lds, st);
    else if constexpr (FMT != FMT_INT8 && !is_gguf(FMT)) {
        if (lw == 8) launch_one<FMT, 8, R>(b, tiles, lds, st);
        else launch_one<FMT, 4, R>(b, tiles, lds, st);
    }
}

template <int FMT, int LW, int R, int MT>
void launch_gx(const Batch &b, int64_t tiles, hipStream_t st) {
    // one chunk per unit beyond one x tile (the x fragments of a unit grow with MT)
    constexpr int NB = MT == 1 ? CFH_GX_NB : 1;
    skinny_gx_kernel<FMT, LW, R, NB, MT><<<dim3(static_cast<unsigned>(tiles)), dim3(kThreads), 0, st>>>(b);
}

template <int FMT, int R, int MT>
void launch_gx_lw(int lw, const Batch &b, int64_t tiles, hipStream_t st) {
    if (lw == 16) launch_gx<FMT, 16, R, MT>(b, tiles, st);
    else if constexpr (FMT != FMT_INT8 && !is_gguf(FMT)) {
        if (lw == 8) launch_gx<FMT, 8, R, MT>(b, tiles, st);
        else launch_gx<FMT, 4, R, MT>(b, tiles, st);
    }
}

// rows per workgroup 16 R and x tiles MT for M: R from the CFH_GX_R_* knobs up to M = 16;
// beyond, 32 rows and 2 or 4 x tiles
template <int FMT>
void launch_gx_r(int r, int64_t m, int lw, const Batch &b, int64_t tiles, hipStream_t st) {
    if (m > 32) launch_gx_lw<FMT, 2, 4>(lw, b, tiles, st);
    else if (m > 16) launch_gx_lw<FMT, 2, 2>(lw, b, tiles, st);
    else if (r == 1) launch_gx_lw<FMT, 1, 1>(lw, b, tiles, st);
    else if (r == 2) launch_gx_lw<FMT, 2, 1>(lw, b, tiles, st);
    else launch_gx_lw<FMT, 4, 1>(lw, b, tiles, st);
}

template <int FMT, int LW>
void launch_split(const Batch &b, int64_t tiles, int64_t lds, hipStream_t st) {
    skinny_m1_split_kernel<FMT, LW><<<dim3(static_cast<unsigned>(tiles)), dim3(kThreads), static_cast<size_t>(lds), st>>>(b);
}

// Launch problems that share the format, M and chunk width; all must pass skinny_ok.
void launch_skinny(int fmt, Problem *ps, int count, int64_t m, int y_bf16, hipStream_t st) {
    const int lw = lw_for(fmt, ps[0].group);
    const int ck = chunk_k(fmt, lw);
    if (m == 1 && CFH_GEMV_SPLIT) {
        // LDS bytes of one wave: its x slice, then its groups' scale and zero-point pieces
        // (1 KB per copy of 4 pieces of 16 bytes per row); bounds over the waves' ranges
        std::stable_sort(ps, ps + count, [](const Problem &a, const Problem &c) { return a.k > c.k; });
        Batch b{};
        int64_t region_max = 0, tiles = 0;
        for (int i = 0; i < count; ++i) {
            require(lw_for(fmt, ps[i].group) == lw, "batched problems must share the group size class");
            b.p[i] = ps[i];
            b.p[i].tile_begin = static_cast<int32_t>(tiles);
            region_max = std::max(region_max, split_region(fmt, lw, b.p[i]));
            tiles += (ps[i].n + 15) / 16;
        }
        if (region_max * kWaves <= kLdsBytesSplit) {
            require(tiles <= 0x7fffffff, "too many rows for one launch");
            if (tiles == 0) return;
            b.count = count;
            b.m = 1;
            b.y_bf16 = y_bf16;
            const int64_t lds = region_max * kWaves;
            if (fmt == FMT_INT4) {
                if (lw == 16) launch_split<FMT_INT4, 16>(b, tiles, lds, st);
                else if (lw == 8) launch_split<FMT_INT4, 8>(b, tiles, lds, st);
                else launch_split<FMT_INT4, 4>(b, tiles, lds, st);
            } else if (fmt == FMT_NF4) {
                if (lw == 16) launch_split<FMT_NF4, 16>(b, tiles, lds, st);
                else if (lw == 8) launch_split<FMT_NF4, 8>(b, tiles, lds, st);
                else launch_split<FMT_NF4, 4>(b, tiles, lds, st);
            } else if (fmt == FMT_Q4_0) {
                launch_split<FMT_Q4_0, 16>(b, tiles, lds, st);
            } else if (fmt == FMT_Q8_0) {
                launch_split<FMT_Q8_0, 16>(b, tiles, lds, st);
            } else {
                launch_split<FMT_INT8, 16>(b, tiles, lds, st);
            }
            check_launch("skinny_m1_split");
            return;
        }
    }
    // 16-row tiles up to M = 4, 32 rows up to M = 8, 64 rows beyond (x is shared by more rows)
    const int R = m <= 4 ? CFH_GEMV_R_SMALL : m <= 8 ? 2 : 4;
    if (m >= 2) {
        // NF4 and Q4_0 at M = 9..16: 32 rows (NF4 62 against 72 us per gate / up / down at
        // M = 16; Q4_0 spills registers at 64 rows)
        const int rbig = fmt == FMT_NF4 || fmt == FMT_Q4_0 ? 2 : CFH_GX_R_BIG;
        const int Rg = m <= 4 ? CFH_GX_R_SMALL : m <= 8 ? CFH_GX_R_MID : m <= 16 ? rbig : 2;
        // x read per wave from global memory (skinny_gx_kernel)
        std::stable_sort(ps, ps + count, [](const Problem &a, const Problem &c) { return a.k > c.k; });
        Batch b{};
        int64_t tiles = 0;
        for (int i = 0; i < count; ++i) {
            require(lw_for(fmt, ps[i].group) == lw, "batched problems must share the group size class");
            b.p[i] = ps[i];
            b.p[i].tile_begin = static_cast<int32_t>(tiles);
            tiles += (ps[i].n + 16 * Rg - 1) / (16 * Rg);
        }
        require(tiles <= 0x7fffffff, "too many rows for one launch");
        if (tiles == 0) return;
        b.count = count;
        b.m = static_cast<int32_t>(m);
        b.y_bf16 = y_bf16;
        if (fmt == FMT_INT4) launch_gx_r<FMT_INT4>(Rg, m, lw, b, tiles, st);
        else if (fmt == FMT_NF4) launch_gx_r<FMT_NF4>(Rg, m, lw, b, tiles, st);
        else if (fmt == FMT_Q4_0) launch_gx_r<FMT_Q4_0>(Rg, m, lw, b, tiles, st);
        else if (fmt == FMT_Q8_0) launch_gx_r<FMT_Q8_0>(Rg, m, lw, b, tiles, st);
        else launch_gx_r<FMT_INT8>(Rg, m, lw, b, tiles, st);
        check_launch("skinny_gx");
        return;
    }
    // longest K first: its workgroups run longest, so they start first
    std::stable_sort(ps, ps + count, [](const Problem &a, const Problem &c) { return a.k > c.k; });
    Batch b{};
    int64_t tiles = 0, kc_max = 0;
    for (int i = 0; i < count; ++i) {
        require(lw_for(fmt, ps[i].group) == lw, "batched problems must share the group size class");
        b.p[i] = ps[i];
        b.p[i].tile_begin = static_cast<int32_t>(tiles);
        b.p[i].kc = kc_for(ps[i].k, m, ck, R == 4 ? 2 : CFH_GEMV_NB_SMALL);
        tiles += (ps[i].n + 16 * R - 1) / (16 * R);
        kc_max = std::max<int64_t>(kc_max, b.p[i].kc);
    }
    require(tiles <= 0x7fffffff, "too many rows for one launch");
    // the stage of the largest problem, then its post factors
    const int64_t max_lds = m * kc_max * 2 + xpost_bytes(kc_max, m, ck);
    b.kc_max = static_cast<int32_t>(kc_max);
    b.count = count;
    b.m = static_cast<int32_t>(m);
    b.y_bf16 = y_bf16;
    if (tiles == 0) return;
    if (fmt == FMT_INT4) {
        if (R == CFH_GEMV_R_SMALL) launch_lw<FMT_INT4, CFH_GEMV_R_SMALL>(lw, b, tiles, max_lds, st);
        else if (R == 2) launch_lw<FMT_INT4, 2>(lw, b, tiles, max_lds, st);
        else launch_lw<FMT_INT4, 4>(lw, b, tiles, max_lds, st);
    } else if (fmt == FMT_NF4) {
        if (R == CFH_GEMV_R_SMALL) launch_lw<FMT_NF4, CFH_GEMV_R_SMALL>(lw, b, tiles, max_lds, st);
        else if (R == 2) launch_lw<FMT_NF4, 2>(lw, b, tiles, max_lds, st);
        else launch_lw<FMT_NF4, 4>(lw, b, tiles, max_lds, st);
    } else if (fmt == FMT_Q4_0) {
        if (R == CFH_GEMV_R_SMALL) launch_lw<FMT_Q4_0, CFH_GEMV_R_SMALL>(lw, b, tiles, max_lds, st);
        else if (R == 2) launch_lw<FMT_Q4_0, 2>(lw, b, tiles, max_lds, st);
        else launch_lw<FMT_Q4_0, 4>(lw, b, tiles, max_lds, st);
    } else if (fmt == FMT_Q8_0) {
        if (R == CFH_GEMV_R_SMALL) launch_lw<FMT_Q8_0, CFH_GEMV_R_SMALL>(lw, b, tiles, max_lds, st);
        else if (R == 2) launch_lw<FMT_Q8_0, 2>(lw, b, tiles, max_lds, st);
        else launch_lw<FMT_Q8_0, 4>(lw, b, tiles, max_lds, st);
    } else {
        if (R == CFH_GEMV_R_SMALL) launch_lw<FMT_INT8, CFH_GEMV_R_SMALL>(lw, b, tiles, max_lds, st);
        else if (R == 2) launch_lw<FMT_INT8, 2>(lw, b, tiles, max_lds, st);
        else launch_lw<FMT_INT8, 4>(lw, b, tiles, max_lds, st);
    }
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

// NF4 on one bf16 MFMA pair per product (gemm_nf4.hip), for M > 16.
bool nf4_mfma_ok(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t block, const void *codes);
void nf4_mfma_launch(const cfh_nf4_problem_t *ps, int count, int64_t m, int y_bf16, hipStream_t st);

// CASTFORGE_NF4_MFMA=0 keeps NF4 at M > 16 on the skinny / prefill kernels (for comparison).
bool nf4_mfma_enabled() {
    const char *e = std::getenv("CASTFORGE_NF4_MFMA");
    return !(e && std::strcmp(e, "0") == 0);
}

// Prefill MFMA kernel (gemm_prefill.hip); false when the shape does not fit it.
bool prefill_try(int fmt, const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                 const void *codes, const void *scales, const uint32_t *zeros, int per_row, void *y,
                 int y_bf16, hipStream_t st);

// Largest M a single problem runs on the skinny kernels; beyond it the prefill kernel is
// faster (measured on W_gate / W_up / W_down of a 7B block: INT8 and Q4_0 at M = 48 / 64 take
// 138 / 149 and 309 / 323 us there against 103 / 100 and 200 / 197 us on the prefill kernel;
// INT4, NF4 and Q8_0 stay faster on the skinny kernel up to M = 64).  Batched calls take the
// skinny kernels up to M = 64 for every format.
int64_t skinny_m_max(int fmt) { return fmt == FMT_INT8 || fmt == FMT_Q4_0 ? 32 : 64; }

// Routes one problem to the skinny MFMA kernels when its shape allows it.
bool gemv_try_skinny(int fmt, const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                     const void *codes, const void *scales, const uint32_t *zeros, int per_row,
                     void *y, int y_bf16, hipStream_t st) {
    Problem p{x, codes, scales, zeros, y, n, k, static_cast<int32_t>(group), per_row, 0, 0};
    if (m > skinny_m_max(fmt) || !skinny_ok(fmt, p, m)) return false;
    launch_skinny(fmt, &p, 1, m, y_bf16, st);
    return true;
}

void gemv_generic(int fmt, const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t group,
                  const void *codes, const void *scales, const uint32_t *zeros, int per_row, void *y,
                  int y_bf16, hipStream_t st) {
    Problem p{x, codes, scales, zeros, y, n, k, static_cast<int32_t>(group), per_row, 0, 0};
    if (fmt == FMT_INT4) launch_generic<FMT_INT4>(p, m, y_bf16, st);
    else if (fmt == FMT_INT8) launch_generic<FMT_INT8>(p, m, y_bf16, st);
    else if (fmt == FMT_Q4_0) launch_generic<FMT_Q4_0>(p, m, y_bf16, st);
    else if (fmt == FMT_Q8_0) launch_generic<FMT_Q8_0>(p, m, y_bf16, st);
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
        if (!gemv_try_skinny(FMT_INT4, x, m, n, k, group, codes, scales_f16, zeros, 1, y, yb, st) &&
            !prefill_try(FMT_INT4, x, m, n, k, group, codes, scales_f16, zeros, 1, y, yb, st))
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
        if (!gemv_try_skinny(FMT_INT8, x, m, n, k, 0, codes, scales, nullptr, pr, y, yb, st) &&
            !prefill_try(FMT_INT8, x, m, n, k, 0, codes, scales, nullptr, pr, y, yb, st))
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
        if (nf4_mfma_enabled() && nf4_mfma_ok(x, m, n, k, block, codes)) {
            const cfh_nf4_problem_t p{x, codes, absmax, y, n, k, block};
            nf4_mfma_launch(&p, 1, m, yb, st);
            return;
        }
        if (!gemv_try_skinny(FMT_NF4, x, m, n, k, block, codes, absmax, nullptr, 1, y, yb, st) &&
            !prefill_try(FMT_NF4, x, m, n, k, block, codes, absmax, nullptr, 1, y, yb, st))
            gemv_generic(FMT_NF4, x, m, n, k, block, codes, absmax, nullptr, 1, y, yb, st);
    });
}

int32_t castforge_hip_gemv_gguf(int32_t ggml_type, const uint16_t *x, int64_t m, int64_t n, int64_t k,
                                const void *codes, const uint16_t *scales_f16, void *y, int32_t y_dtype,
                                void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(ggml_type == CFH_GGML_Q4_0 || ggml_type == CFH_GGML_Q8_0,
                "ggml_type must be CFH_GGML_Q4_0 or CFH_GGML_Q8_0");
        common_checks(x, m, n, k, codes, y, y_dtype);
        const int fmt = ggml_type == CFH_GGML_Q4_0 ? FMT_Q4_0 : FMT_Q8_0;
        require(k % chunk_k(fmt, 16) == 0, fmt == FMT_Q4_0 ? "Q4_0 planes need k % 128 == 0"
                                                           : "Q8_0 planes need k % 64 == 0");
        if (m == 0 || n == 0) return;
        require(k == 0 || scales_f16, "scales must not be NULL");
        require(aligned(codes, 16) && aligned(scales_f16, 16), "codes and scales must be 16-byte aligned");
        hipStream_t st = static_cast<hipStream_t>(stream);
        const int yb = y_dtype == CFH_DTYPE_BF16;
        Problem p{x, codes, scales_f16, nullptr, y, n, k, 32, 1, 0, 0};
        if (m == 2 && skinny_ok(fmt, p, 1)) {
            // two rows as two M = 1 problems of one split-K launch (measured faster than the
            // skinny kernel at M = 2; the second row re-reads the planes from the MALL)
            const int esz = yb ? 2 : 4;
            Problem ps[2] = {p, p};
            ps[1].x = x + k;
            ps[1].y = static_cast<uint8_t *>(y) + n * esz;
            launch_skinny(fmt, ps, 2, 1, yb, st);
            return;
        }
        // split-K kernel at M = 1, the skinny kernel (x read per wave) beyond
        if (gemv_try_skinny(fmt, x, m, n, k, 32, codes, scales_f16, nullptr, 1, y, yb, st)) return;
        // larger M: the prefill MFMA kernel reads the planes directly
        if (prefill_try(fmt, x, m, n, k, 32, codes, scales_f16, nullptr, 1, y, yb, st)) return;
        gemv_generic(fmt, x, m, n, k, 32, codes, scales_f16, nullptr, 1, y, yb, st);
    });
}

int32_t castforge_hip_gemv_gguf_batched(int32_t ggml_type, const cfh_gguf_problem_t *problems, int32_t count,
                                        int64_t m, int32_t y_dtype, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(ggml_type == CFH_GGML_Q4_0 || ggml_type == CFH_GGML_Q8_0,
                "ggml_type must be CFH_GGML_Q4_0 or CFH_GGML_Q8_0");
        require(m >= 1 && m <= 64, "batched GEMV requires 1 <= m <= 64");
        require(count >= 0 && count <= CFH_MAX_BATCH, "count must be in [0, CFH_MAX_BATCH]");
        require(count == 0 || problems != nullptr, "problems must not be NULL");
        require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
        const int fmt = ggml_type == CFH_GGML_Q4_0 ? FMT_Q4_0 : FMT_Q8_0;
        Problem ps[kMaxProblems];
        int used = 0;
        for (int i = 0; i < count; ++i) {
            const cfh_gguf_problem_t &q = problems[i];
            common_checks(q.x, m, q.n, q.k, q.codes, q.y, y_dtype);
            if (q.n == 0) continue;
            require(q.k > 0 && q.scales_f16, "problem buffers must not be NULL");
            Problem p{q.x, q.codes, q.scales_f16, nullptr, q.y, q.n, q.k, 32, 1, 0, 0};
            require(skinny_ok(fmt, p, m),
                    "batched GGUF GEMV needs k % 128 == 0 (Q4_0) or k % 64 == 0 (Q8_0), k below 2^24 "
                    "and 16-byte aligned x / codes / scales");
            ps[used++] = p;
        }
        if (used) launch_skinny(fmt, ps, used, m, y_dtype == CFH_DTYPE_BF16, static_cast<hipStream_t>(stream));
    });
}

int32_t castforge_hip_gemv_w4a16_batched(const cfh_w4a16_problem_t *problems, int32_t count,
                                         int64_t m, int32_t y_dtype, void *stream,
                                         char **out_error) {
    return guarded(out_error, [&] {
        require(count >= 0 && count <= CFH_MAX_BATCH, "count must be in [0, CFH_MAX_BATCH]");
        require(count == 0 || problems != nullptr, "problems must not be NULL");
        require(m >= 1 && m <= 64, "batched GEMV requires 1 <= m <= 64");
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
            require(q.group % 128 == 0 && skinny_ok(FMT_INT4, p, m),
                    "batched GEMV needs k % 128 == 0, group % 128 == 0 and 16-byte aligned x/codes");
            ps[used++] = p;
        }
        if (used) launch_skinny(FMT_INT4, ps, used, m, y_dtype == CFH_DTYPE_BF16,
                                static_cast<hipStream_t>(stream));
    });
}

int32_t castforge_hip_gemv_w8a16_batched(const cfh_w8a16_problem_t *problems, int32_t count,
                                         int64_t m, int32_t y_dtype, void *stream,
                                         char **out_error) {
    return guarded(out_error, [&] {
        require(count >= 0 && count <= CFH_MAX_BATCH, "count must be in [0, CFH_MAX_BATCH]");
        require(count == 0 || problems != nullptr, "problems must not be NULL");
        require(m >= 1 && m <= 64, "batched GEMV requires 1 <= m <= 64");
        require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
        Problem ps[kMaxProblems];
        int used = 0;
        for (int i = 0; i < count; ++i) {
            const cfh_w8a16_problem_t &q = problems[i];
            common_checks(q.x, m, q.n, q.k, q.codes, q.y, y_dtype);
            require(q.granularity == CFH_GRAN_TENSOR || q.granularity == CFH_GRAN_CHANNEL,
                    "granularity must be CFH_GRAN_TENSOR or CFH_GRAN_CHANNEL");
            if (q.n == 0) continue;
            require(q.k > 0 && q.scales, "problem buffers must not be NULL");
            Problem p{q.x, q.codes, q.scales, nullptr, q.y, q.n, q.k, 0,
                      q.granularity == CFH_GRAN_CHANNEL ? 1 : 0, 0, 0};
            require(skinny_ok(FMT_INT8, p, m), "batched GEMV needs k % 64 == 0 and 16-byte aligned x/codes");
            ps[used++] = p;
        }
        if (used) launch_skinny(FMT_INT8, ps, used, m, y_dtype == CFH_DTYPE_BF16, static_cast<hipStream_t>(stream));
    });
}

int32_t castforge_hip_gemv_nf4_batched(const cfh_nf4_problem_t *problems, int32_t count, int64_t m,
                                       int32_t y_dtype, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        require(count >= 0 && count <= CFH_MAX_BATCH, "count must be in [0, CFH_MAX_BATCH]");
        require(count == 0 || problems != nullptr, "problems must not be NULL");
        require(m >= 1 && m <= 64, "batched GEMV requires 1 <= m <= 64");
        require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
        Problem ps[kMaxProblems];
        cfh_nf4_problem_t mf[kMaxProblems];
        int used = 0;
        bool mfma = nf4_mfma_enabled();
        for (int i = 0; i < count; ++i) {
            const cfh_nf4_problem_t &q = problems[i];
            common_checks(q.x, m, q.n, q.k, q.codes, q.y, y_dtype);
            require(q.block == problems[0].block, "batched problems must share the block size");
            if (q.n == 0) continue;
            require(q.k > 0 && q.absmax, "problem buffers must not be NULL");
            mfma = mfma && nf4_mfma_ok(q.x, m, q.n, q.k, q.block, q.codes);
            mf[used] = q;
            Problem p{q.x, q.codes, q.absmax, nullptr, q.y, q.n, q.k, static_cast<int32_t>(q.block), 1, 0, 0};
            require(q.block >= 32 && skinny_ok(FMT_NF4, p, m),
                    "batched GEMV needs block 32, 64 or a power-of-two multiple of 128, k a multiple "
                    "of the chunk (block 32: 32, 64: 64, else 128) and 16-byte aligned x/codes");
            ps[used++] = p;
        }
        if (used && mfma) nf4_mfma_launch(mf, used, m, y_dtype == CFH_DTYPE_BF16, static_cast<hipStream_t>(stream));
        else if (used) launch_skinny(FMT_NF4, ps, used, m, y_dtype == CFH_DTYPE_BF16, static_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
