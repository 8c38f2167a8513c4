// FP8 E4M3 W8A8 GEMM for gfx950: Y[m, n] = bf16((sum_k A[m, k] * W[n, k]) * sa[m] * sw[n]).
//
// A: fp8 [M, K] activations with per-token scales sa[M]; W: fp8 [N, K] weights with per-row
// scales sw[N]; both K-contiguous (the packed_rhs layout, passes/weights/fold.rs:549-554).
// This is the prefill GEMM the FP8 variant of `castforge.fused_qmatmul` lowers to
// (codegen/eval.rs:1145-1179 semantics: dequantize then eval_matmul_2d, eval.rs:1465-1507).
//
// Design (compute-bound, AI ~2.4k flop/B):
//   * workgroup tile 256 (n) x 256 (m), 4 waves in a 2 x 2 grid, 128 x 128 per wave, so each
//     LDS byte feeds 256 flops; 16 accumulator tiles of 32 x 32 (256 f32 per lane) live in
//     the accumulation registers at one wave per SIMD;
//   * v_mfma_f32_32x32x64_f8f6f4 (OCP E4M3 operands) with W as the row operand, so each lane
//     ends with 4 consecutive n of one m: 8-byte bf16 stores;
//   * operands move global -> LDS with buffer_load ... lds (no VGPR staging, out-of-range rows
//     read 0), NSTAGE-deep ring of BK-byte K slices, one barrier per slice;
//   * 16-byte chunks are XOR-swizzled by row inside the LDS rows so the fragment reads
//     (ds_read_b128, 8 lanes on 8 rows) hit distinct banks;
//   * XCD-aware tile order: consecutive tiles run on the same XCD (shared L2), grouped by
//     kGroupM m-tiles so an XCD reuses the same A and W panels.
#include <atomic>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

typedef int int32x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

#ifndef CFH_FP8_BK
#define CFH_FP8_BK 64
#endif
#ifndef CFH_FP8_NSTAGE
#define CFH_FP8_NSTAGE 4
#endif
#ifndef CFH_FP8_INTERLEAVE
#define CFH_FP8_INTERLEAVE 1
#endif
#ifndef CFH_FP8_RS
#define CFH_FP8_RS 0  // 1: global -> VGPR -> ds_write staging; 0: buffer_load ... lds ring
#endif
#ifndef CFH_FP8_SCHED
#define CFH_FP8_SCHED 0
#endif
#ifndef CFH_FP8_GROUP_M
#define CFH_FP8_GROUP_M 4
#endif

constexpr int BM = 256, BN = 256, BK = CFH_FP8_BK, NSTAGE = CFH_FP8_NSTAGE;
#ifndef CFH_FP8_WAVES
#define CFH_FP8_WAVES 4
#endif
constexpr int kWaves = CFH_FP8_WAVES;                  // 4: 128 x 128 per wave; 8: 128 x 64
constexpr int kThreads = 64 * kWaves;
constexpr int kWaveM = 512 / kWaves;                   // m extent of a wave's tile
constexpr int JT = kWaveM / 32;                        // 32-wide m sub-tiles per wave
constexpr int kChunks = BK / 16;                       // 16-byte chunks per tile row
constexpr int kRowsPerLoad = 64 / kChunks;             // rows one wave-wide 1 KB load covers
constexpr int kTileBytes = BM * BK;                    // one operand, one stage
constexpr int kStageBytes = 2 * kTileBytes;            // W tile, then A tile
constexpr int kPipeLdsBytes = (CFH_FP8_RS ? 2 : NSTAGE) * kStageBytes;
constexpr int kEpiLdsBytes = kWaves * kWaveM * 256;    // bf16 output block of every wave
constexpr int kLdsBytes = kPipeLdsBytes > kEpiLdsBytes ? kPipeLdsBytes : kEpiLdsBytes;
constexpr int kLoadsPerWave = 2 * kTileBytes / 1024 / kWaves;  // 1 KB loads per wave per stage
constexpr int kXcds = 8;
constexpr int kGroupM = CFH_FP8_GROUP_M;
static_assert(BK == 64 || BK == 128, "BK must be 64 or 128");
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(NSTAGE >= 2 && (NSTAGE - 1) * kLoadsPerWave <= 63, "stages / vmcnt range");

// Physical 16-byte chunk of logical chunk c in tile row r.  Sixteen lanes reading the same
// logical chunk of sixteen consecutive rows land on sixteen distinct 16-byte slots of a
// 256-byte bank window (CFH_FP8_SWZ 1; 0 spreads eight rows over a 128-byte window).
#ifndef CFH_FP8_SWZ
#define CFH_FP8_SWZ 1
#endif
__device__ __forceinline__ int swz(int r, int c) {
    if (CFH_FP8_SWZ == 1) return BK == 128 ? (c ^ ((r >> 1) & 7)) : (c ^ ((r >> 2) & 3));
    return BK == 128 ? (c ^ (r & 7)) : (c ^ ((r >> 1) & 3));
}

// Waits until at most N vector-memory loads are outstanding and every LDS read has returned.
template <int N>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(N) & ~(15 << 8));
}

// Issues this wave's 1 KB buffer->LDS loads of one operand slice (K bytes [k0, k0 + BK) of
// the panel) into dst.
__device__ __forceinline__ void fp8_issue(__amdgpu_buffer_rsrc_t rsrc, uint8_t *__restrict__ dst,
                                          int first_block, int lvoff, int K, int k0) {
#pragma unroll
    for (int t = 0; t < kLoadsPerWave; ++t) {
        const int blk = first_block + t;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc, (__attribute__((address_space(3))) void *)(dst + blk * 1024), 16, lvoff,
            blk * kRowsPerLoad * K + k0, 0, 0);
    }
}

struct Fp8Frags {
    int32x8 w[BK / 64][4], a[BK / 64][JT];
};

// Reads the wave's fragments of one K slice from LDS.
__device__ __forceinline__ void fp8_read_frags(const uint8_t *__restrict__ cur, int wn, int wm, int fr,
                                               int fc, Fp8Frags &f) {
    const uint8_t *sw_ = cur;
    const uint8_t *sa_ = cur + kTileBytes;
#pragma unroll
    for (int kk = 0; kk < BK / 64; ++kk) {
        const int c0 = kk * 4 + fc;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = wn + i * 32 + fr;
            const uint4 lo = *reinterpret_cast<const uint4 *>(sw_ + r * BK + swz(r, c0) * 16);
            const uint4 hi = *reinterpret_cast<const uint4 *>(sw_ + r * BK + swz(r, c0 + 1) * 16);
            f.w[kk][i] = int32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int j = 0; j < JT; ++j) {
            const int r = wm + j * 32 + fr;
            const uint4 lo = *reinterpret_cast<const uint4 *>(sa_ + r * BK + swz(r, c0) * 16);
            const uint4 hi = *reinterpret_cast<const uint4 *>(sa_ + r * BK + swz(r, c0 + 1) * 16);
            f.a[kk][j] = int32x8{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
    }
}

// Eight E4M3 codes (bytes 8 c .. 8 c + 7 of a lane's 32-byte fragment) -> eight exact f16
// (every E4M3 value, subnormals included, is an f16 normal; scale 1.0 leaves it unchanged).
__device__ __forceinline__ half8_t e4m3x8_to_f16(const int32x8 &v, int c) {
    const uint32_t lo = static_cast<uint32_t>(v[2 * c]), hi = static_cast<uint32_t>(v[2 * c + 1]);
    const half2_t p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false);
    const half2_t p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true);
    const half2_t p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false);
    const half2_t p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true);
    return half8_t{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// MFMAs of one slice on W sub-tiles [I0, I1).
//   kExact false: v_mfma_scale_f32_32x32x64_f8f6f4 on the E4M3 codes.  The fp8 MFMAs sum
//     their products in a fixed-point adder aligned to the largest product of a block of
//     eight, keeping about 13 bits below it: 256 + 2^-6 returns 256, and a block holding one
//     x30 outlier product truncates its small neighbours to ~2^-8 of a typical product.
//   kExact true: the codes are widened to exact f16 and fed to v_mfma_f32_32x32x16_f16,
//     whose products are exact and whose sum keeps f32-like precision (measured on gfx950:
//     256 + 15 x 2^-6 returns 256.234375 exactly).  Twice the MFMA time of the fp8 form.
//   A lane's 32-byte fragment holds K bytes [32 (lane / 32), + 32) of a 64-wide step; f16
//   chunk c gives the lane K bytes 32 (lane / 32) + 8 c + 0..7 of both operands, so the
//   16-wide f16 MFMA c sums a matching set of products and four of them cover the step.
template <bool kExact, int I0, int I1>
__device__ __forceinline__ void fp8_mma_range(const Fp8Frags &f, floatx16 (&acc)[4][JT]) {
#pragma unroll
    for (int kk = 0; kk < BK / 64; ++kk) {
        if constexpr (kExact) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                half8_t wv[I1 - I0], av[JT];
#pragma unroll
                for (int i = I0; i < I1; ++i) wv[i - I0] = e4m3x8_to_f16(f.w[kk][i], c);
#pragma unroll
                for (int j = 0; j < JT; ++j) av[j] = e4m3x8_to_f16(f.a[kk][j], c);
#pragma unroll
                for (int i = I0; i < I1; ++i)
#pragma unroll
                    for (int j = 0; j < JT; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wv[i - I0], av[j], acc[i][j], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int i = I0; i < I1; ++i)
#pragma unroll
                for (int j = 0; j < JT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.w[kk][i], f.a[kk][j], acc[i][j],
                                                                                0, 0, 0, 0, 0, 0);
        }
    }
}

template <bool kExact>
__device__ __forceinline__ void fp8_mma(const Fp8Frags &f, floatx16 (&acc)[4][JT]) {
    fp8_mma_range<kExact, 0, 4>(f, acc);
}

// MFMAs of W sub-tiles [2 H, 2 H + 2) (half of a slice's work).
template <bool kExact, int H>
__device__ __forceinline__ void fp8_mma_half(const Fp8Frags &f, floatx16 (&acc)[4][JT]) {
    fp8_mma_range<kExact, 2 * H, 2 * H + 2>(f, acc);
}

// One pipeline step: refill ring slot `nxt` with a later slice (LDS-DMA), read the fragments
// of the following slice from `cur` into `fn`, and run the MFMAs of the fragments already in
// `f`.  The pointers are restrict-qualified: the compiler then knows that the fragment reads
// do not depend on the LDS-DMA writes into `nxt` and need not wait for them.
template <bool kExact>
__device__ __forceinline__ void fp8_step(const uint8_t *__restrict__ cur, uint8_t *__restrict__ nxt,
                                         bool refill, bool read_next, __amdgpu_buffer_rsrc_t rsrc,
                                         int first_block, int lvoff, int K, int k_next, int wn, int wm,
                                         int fr, int fc, const Fp8Frags &f, Fp8Frags &fn,
                                         floatx16 (&acc)[4][JT]) {
    if (refill) fp8_issue(rsrc, nxt, first_block, lvoff, K, k_next);
    if (read_next) fp8_read_frags(cur, wn, wm, fr, fc, fn);
    fp8_mma<kExact>(f, acc);
    if constexpr (kExact) {
        // 64 f16 MFMAs and 128 conversions per slice: spread the 16 LDS reads and the loads
        // over the first MFMAs, each behind its share of conversions
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);  // 8 VALU (conversions)
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // 4 MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
            if (q < kLoadsPerWave) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // 1 VMEM load
        }
        return;
    }
#if CFH_FP8_INTERLEAVE
    // one wave per SIMD feeds the MFMA pipe: start the MFMAs at once and slot the LDS reads
    // and the LDS-DMA loads between them instead of issuing every read first
    // CFH_FP8_SCHED 0: a load after each of the first 8 MFMAs; 1: after every second MFMA;
    // 2: after each of the last 8 MFMAs
#pragma unroll
    for (int q = 0; q < 4 * JT * (BK / 64); ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
        const bool load_here = CFH_FP8_SCHED == 0 ? q < kLoadsPerWave
                             : CFH_FP8_SCHED == 1 ? (q & 1) == 1
                                                  : q >= 4 * JT * (BK / 64) - kLoadsPerWave;
        if (load_here) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // 1 VMEM load
    }
#endif
}

template <bool kExact>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kWaves / 4, kWaves / 4)))
void fp8_gemm_kernel(const uint8_t *__restrict__ A, const float *__restrict__ sa,
                     const uint8_t *__restrict__ W, const float *__restrict__ sw,
                     void *__restrict__ Y, int y_bf16, int y_vec /* 0 scalar, 1 vector, 2 bf16 via LDS */, int sw_vec,
                     int M, int N, int K,
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

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // ---- global -> LDS loads: waves 0-1 bring the W tile, waves 2-3 the A tile ----
    const bool loads_w = wave < kWaves / 2;
    const int rows_valid = loads_w ? min(BN, N - n0) : min(BM, M - m0);
    const uint8_t *base = loads_w ? W + static_cast<int64_t>(n0) * K : A + static_cast<int64_t>(m0) * K;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, rows_valid * K, 0x00020000);
    // lane i of a 1 KB load writes LDS bytes [16 i, 16 i + 16): row i / kChunks of the load's
    // rows, physical chunk i % kChunks, which holds logical chunk swz(row, i % kChunks).
    const int lrow = lane / kChunks;
    const int lvoff = lrow * K + swz(lrow, lane % kChunks) * 16;

    // ---- fragments: lane reads 32 bytes (2 chunks) of row lane % 32 per K=64 step ----
    const int wn = (wave / (kWaves / 2)) * 128, wm = (wave % (kWaves / 2)) * kWaveM;
    const int fr = lane & 31;
    const int fc = (lane >> 5) * 2;  // first logical chunk within a 64-byte K step

    floatx16 acc[4][JT];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int tile_off = loads_w ? 0 : kTileBytes;
    const int first_block = (wave % (kWaves / 2)) * kLoadsPerWave;  // this wave's first 1 KB block
    const int KT = K / BK;
#if CFH_FP8_RS
    // Two LDS slots (slot s & 1 holds slice s) and two register staging sets.  A slice is
    // loaded into registers two steps before it is written to LDS, and read into fragments
    // right after the barrier that follows its write.
    typedef uint4 Stage[kLoadsPerWave];
    auto gload = [&](Stage &st, int kt) {
#pragma unroll
        for (int t = 0; t < kLoadsPerWave; ++t)
            st[t] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                rsrc, lvoff, (first_block + t) * kRowsPerLoad * K + kt * BK, 0));
    };
    auto lwrite = [&](const Stage &st, int slot) {
        uint8_t *dst = lds + slot * kStageBytes + tile_off + first_block * 1024 + lane * 16;
#pragma unroll
        for (int t = 0; t < kLoadsPerWave; ++t) *reinterpret_cast<uint4 *>(dst + t * 1024) = st[t];
    };
    Stage stg0, stg1;
    Fp8Frags fa, fb;
    gload(stg0, 0);
    if (KT > 1) gload(stg1, 1);
    if (KT > 1) wait_vm<kLoadsPerWave>();
    else wait_vm<0>();
    lwrite(stg0, 0);
    if (KT > 2) gload(stg0, 2);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));
    __builtin_amdgcn_s_barrier();
    fp8_read_frags(lds, wn, wm, fr, fc, fa);

    // Step t: fragments of slice t in f; slice t + 1 in staging set sn (landing), slice t + 2
    // in the other set (in flight).  Write slice t + 1 to slot (t + 1) & 1 (last read two
    // steps ago), reload sn with slice t + 3, barrier, read slice t + 1's fragments; slice t's
    // MFMAs are split around the barrier so the pipe is busy while the wave waits.
    auto step = [&](auto steady, int t, const Fp8Frags &f, Fp8Frags &fn, Stage &sn) {
        constexpr bool kSteady = decltype(steady)::value;
        // no explicit vmcnt wait: the LDS writes below consume the staging registers, so the
        // compiler waits for exactly the loads they need
        fp8_mma_half<kExact, 0>(f, acc);
        if (kSteady || t + 1 < KT) lwrite(sn, (t + 1) & 1);
        if (kSteady || t + 3 < KT) gload(sn, t + 3);
#if CFH_FP8_INTERLEAVE
        if (kSteady) {
#pragma unroll
            for (int q = 0; q < 2 * JT * (BK / 64); ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // 1 MFMA
                if (q < kLoadsPerWave) __builtin_amdgcn_sched_group_barrier(0x200, 1, 1);  // 1 LDS write
                if (q < kLoadsPerWave) __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);  // 1 VMEM load
            }
        }
#endif
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));
        __builtin_amdgcn_s_barrier();
        if (kSteady || t + 1 < KT) fp8_read_frags(lds + ((t + 1) & 1) * kStageBytes, wn, wm, fr, fc, fn);
        fp8_mma_half<kExact, 1>(f, acc);
#if CFH_FP8_INTERLEAVE
        if (kSteady) {
#pragma unroll
            for (int q = 0; q < 2 * JT * (BK / 64); ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);  // 1 MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 2);  // 2 LDS reads
            }
        }
#endif
    };
    int kt = 0;
    for (; kt + 4 < KT; kt += 2) {
        step(std::true_type{}, kt, fa, fb, stg1);
        step(std::true_type{}, kt + 1, fb, fa, stg0);
    }
    for (; kt < KT; kt += 2) {
        step(std::false_type{}, kt, fa, fb, stg1);
        if (kt + 1 < KT) step(std::false_type{}, kt + 1, fb, fa, stg0);
    }
#else
    // ring of NSTAGE slots: slot s % NSTAGE holds slice s.  All slots are filled up front.
#pragma unroll
    for (int s = 0; s < NSTAGE; ++s)
        if (s < KT) fp8_issue(rsrc, lds + s * kStageBytes + tile_off, first_block, lvoff, K, s * BK);

    // slice 0's fragments: wait for this wave's slice-0 loads, then for everyone's
    Fp8Frags fa, fb;
    if (KT >= NSTAGE) wait_vm<(NSTAGE - 1) * kLoadsPerWave>();
    else wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    fp8_read_frags(lds, wn, wm, fr, fc, fa);

    // Step t: slice t's fragments are in registers.  Wait until slice t + 1 has landed (at
    // most NSTAGE - 2 younger slices outstanding) and barrier -- after which no wave reads
    // slot t % NSTAGE any more (slice t's fragments were read in step t - 1) -- then refill
    // that slot with slice t + NSTAGE, read slice t + 1's fragments and run slice t's MFMAs.
    // Unrolled by two so the fragment sets alternate between fa and fb without copies.
    auto step = [&](auto steady, int t, const Fp8Frags &f, Fp8Frags &fn) {
        constexpr bool kSteady = decltype(steady)::value;
        if (kSteady || t + NSTAGE - 1 < KT) wait_vm<(NSTAGE - 2) * kLoadsPerWave>();
        else wait_vm<0>();
        // unconditional, so the compiler's own wait tracking sees every LDS read retired on
        // all paths (the branchy vmcnt waits above hide that from it)
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));
        __builtin_amdgcn_s_barrier();
        const int nk = t + NSTAGE;
        // steady steps are branch-free, so the scheduler can interleave loads, reads and MFMAs
        fp8_step<kExact>(lds + ((t + 1) % NSTAGE) * kStageBytes, lds + (t % NSTAGE) * kStageBytes + tile_off,
                 kSteady || nk < KT, kSteady || t + 1 < KT, rsrc, first_block, lvoff, K, nk * BK, wn, wm,
                 fr, fc, f, fn, acc);
    };
    int kt = 0;
    for (; kt + 1 + NSTAGE < KT; kt += 2) {
        step(std::true_type{}, kt, fa, fb);
        step(std::true_type{}, kt + 1, fb, fa);
    }
    for (; kt < KT; kt += 2) {
        step(std::false_type{}, kt, fa, fb);
        if (kt + 1 < KT) step(std::false_type{}, kt + 1, fb, fa);
    }

#endif

    // ---- epilogue: D[n][m] of tile (i, j): lane holds m = lane % 32 and, for g = 0..3,
    // the 4 consecutive n = 8 g + 4 (lane / 32) + 0..3 ----
    // all scales first (one round trip)
    float s_m[JT], s_n[4][4][4];
#pragma unroll
    for (int j = 0; j < JT; ++j) {
        const int m = m0 + wm + j * 32 + fr;
        s_m[j] = m < M ? sa[m] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn + i * 32 + g * 8 + (lane >> 5) * 4;
            if (sw_vec && n + 3 < N) {  // sw_vec: sw 16-byte aligned and N % 4 == 0
                const float4 v = *reinterpret_cast<const float4 *>(sw + n);
                s_n[i][g][0] = v.x, s_n[i][g][1] = v.y, s_n[i][g][2] = v.z, s_n[i][g][3] = v.w;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) s_n[i][g][q] = n + q < N ? sw[n + q] : 0.f;
            }
        }
    if (y_vec == 2) {
        // bf16 output through LDS: each wave writes its 128 (m) x 128 (n) bf16 block (256 B
        // rows, 16-byte chunks XOR-swizzled by row) and reads it back as whole rows, so every
        // global store is a full 256-byte row segment.
        static_assert(kLdsBytes >= kWaves * kWaveM * 256, "epilogue stage fits in LDS");
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));
        __syncthreads();  // every wave is done with the operand slots
        uint8_t *eb = lds + wave * kWaveM * 256;
        static_for<JT>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const int ml = j * 32 + fr;  // row within the wave block
            static_for<4>([&](auto I) {
                constexpr int i = decltype(I)::value;
                static_for<4>([&](auto G) {
                    constexpr int g = decltype(G)::value;
                    uint2 p;
                    p.x = f32x2_to_bf16x2_rne(acc[i][j][g * 4 + 0] * s_m[j] * s_n[i][g][0],
                                              acc[i][j][g * 4 + 1] * s_m[j] * s_n[i][g][1]);
                    p.y = f32x2_to_bf16x2_rne(acc[i][j][g * 4 + 2] * s_m[j] * s_n[i][g][2],
                                              acc[i][j][g * 4 + 3] * s_m[j] * s_n[i][g][3]);
                    const int chunk = (i * 4 + g) ^ (ml & 15);
                    *reinterpret_cast<uint2 *>(eb + ml * 256 + chunk * 16 + (lane >> 5) * 8) = p;
                });
            });
        });
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));  // own LDS writes done
        const int cl = lane & 15;
#pragma unroll 4
        for (int rb = 0; rb < kWaveM; rb += 4) {
            const int ml = rb + (lane >> 4);
            const uint4 v = *reinterpret_cast<const uint4 *>(eb + ml * 256 + ((cl ^ (ml & 15)) * 16));
            const int m = m0 + wm + ml, n = n0 + wn + cl * 8;
            if (m < M && n < N)
                *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(Y) + static_cast<int64_t>(m) * N + n) = v;
        }
        return;
    }
    const bool vec = y_vec != 0;  // N % 4 == 0 and Y 16-byte aligned
    static_for<JT>([&](auto J) {
        constexpr int j = decltype(J)::value;
        const int m = m0 + wm + j * 32 + fr;
        static_for<4>([&](auto I) {
            constexpr int i = decltype(I)::value;
            static_for<4>([&](auto G) {
                constexpr int g = decltype(G)::value;
                const int n = n0 + wn + i * 32 + g * 8 + (lane >> 5) * 4;
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = acc[i][j][g * 4 + q] * s_m[j] * s_n[i][g][q];
                if (m >= M || n >= N) return;
                const int64_t o = static_cast<int64_t>(m) * N + n;
                if (vec) {
                    if (y_bf16) {
                        uint2 p;
                        p.x = f32x2_to_bf16x2_rne(v[0], v[1]);
                        p.y = f32x2_to_bf16x2_rne(v[2], v[3]);
                        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(Y) + o) = p;
                    } else {
                        *reinterpret_cast<float4 *>(static_cast<float *>(Y) + o) = make_float4(v[0], v[1], v[2], v[3]);
                    }
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        if (n + q < N) {
                            if (y_bf16) static_cast<uint16_t *>(Y)[o + q] = f32_to_bf16_rne(v[q]);
                            else static_cast<float *>(Y)[o + q] = v[q];
                        }
                    }
                }
            });
        });
    });
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

// devices (bit = device ordinal < 64) on which each variant's dynamic-LDS limit has been raised
std::atomic<uint64_t> lds_attr_devices[2];

int32_t gemm_fp8(const uint8_t *qa, const float *sa, int64_t m, const uint8_t *qw, const float *sw,
                 int64_t n, int64_t k, void *y, int32_t y_dtype, void *stream, char **out_error,
                 bool exact) {
    return guarded(out_error, [&] {
        require(m >= 0 && n >= 0 && k >= 0, "m, n, k must be non-negative");
        if (m == 0 || n == 0) return;
        require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
        require(qa && sa && qw && sw && y, "buffers must not be NULL");
        const int yb = y_dtype == CFH_DTYPE_BF16;
        require(m <= 0x7fffffff && n <= 0x7fffffff && k <= 0x7fffffff, "dimensions must fit in int32");
        hipStream_t st = static_cast<hipStream_t>(stream);
        // buffer resources address one 256-row panel: 256 * k bytes must fit in 31 bits
        const bool fast = k > 0 && k % BK == 0 && k < (1 << 23) && aligned(qa, 16) && aligned(qw, 16);
        if (fast) {
            int dev = 0;
            check_hip(hipGetDevice(&dev), "hipGetDevice");
            const uint64_t bit = dev < 64 ? (uint64_t{1} << dev) : 0;
            const auto kern = exact ? fp8_gemm_kernel<true> : fp8_gemm_kernel<false>;
            std::atomic<uint64_t> &done = lds_attr_devices[exact ? 1 : 0];
            if (bit == 0 || !(done.load(std::memory_order_acquire) & bit)) {
                check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes),
                          "hipFuncSetAttribute(fp8_gemm_kernel)");
                done.fetch_or(bit, std::memory_order_acq_rel);
            }
            const int tiles_m = static_cast<int>((m + BM - 1) / BM), tiles_n = static_cast<int>((n + BN - 1) / BN);
            kern<<<dim3(tiles_m * tiles_n), dim3(kThreads), kLdsBytes, st>>>(
                qa, sa, qw, sw, y, yb,
                (yb && n % 8 == 0 && aligned(y, 16)) ? 2 : (n % 4 == 0 && aligned(y, 16)) ? 1 : 0,
                (n % 4 == 0 && aligned(sw, 16)) ? 1 : 0, static_cast<int>(m),
                static_cast<int>(n), static_cast<int>(k), tiles_m, tiles_n);
            check_launch(exact ? "fp8_gemm_exact" : "fp8_gemm");
        } else {
            const int64_t tot = m * n;
            require((tot + 255) / 256 <= 0x7fffffff, "shape too large for the generic FP8 kernel");
            fp8_gemm_generic_kernel<<<dim3(static_cast<unsigned>((tot + 255) / 256)), dim3(256), 0, st>>>(
                qa, sa, qw, sw, y, yb, m, n, k);
            check_launch("fp8_gemm_generic");
        }
    });
}

}  // namespace
}  // namespace cfh

extern "C" int32_t castforge_hip_gemm_fp8(const uint8_t *qa, const float *sa, int64_t m,
                                          const uint8_t *qw, const float *sw, int64_t n, int64_t k,
                                          void *y, int32_t y_dtype, void *stream, char **out_error) {
    return cfh::gemm_fp8(qa, sa, m, qw, sw, n, k, y, y_dtype, stream, out_error, false);
}

extern "C" int32_t castforge_hip_gemm_fp8_exact(const uint8_t *qa, const float *sa, int64_t m,
                                                const uint8_t *qw, const float *sw, int64_t n, int64_t k,
                                                void *y, int32_t y_dtype, void *stream, char **out_error) {
    return cfh::gemm_fp8(qa, sa, m, qw, sw, n, k, y, y_dtype, stream, out_error, true);
}
