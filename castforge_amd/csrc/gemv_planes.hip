// W4A16 decode GEMV (M = 1..16) over INT4 g128 weights in the GEMV planes layout, and the M = 1
// decode GEMV over NF4 planes and GGUF Q4_0 GEMV planes, gfx950.  planes_kernel serves INT4 at
// M = 2..4 wherever x fits LDS; planes_xr_kernel (after it) serves M = 5..16, and M = 2..4
// beyond; planes_m1_kernel serves M = 1 for the three formats; planes_i8_kernel serves INT4 at
// M = 1 on the integer MFMA wherever its x pieces fit LDS (planes_m1_kernel's INT4 form, with
// the same arithmetic as planes_kernel, beyond).
//
// Replaces the evaluation of `castforge.fused_qmatmul` at decode (eval.rs:1145-1179 with
// eval_matmul_2d, eval.rs:1465-1507; packed_rhs [N, K] weights, fold.rs:549-554) for the
// asymmetric INT4 group-128 format: y[m, n] = sum_k x[m, k] * (q[n, k] - z[n, g]) * s[n, g].
//
// GEMV planes.  The canonical INT4g arrays (codes u32 [N, K/8], f16 scales [N, GP], u4 zero
// points [N, ceil(G/8)]) are rewritten once, at load time, so that one wave-wide 16-byte load
// reads one contiguous kilobyte: the 64-byte group slice of 16 consecutive rows.
//   codes : T x G chunks of 1024 B (T = ceil(N/16) row tiles, G = K/128 groups); chunk (t, g)
//           holds, at byte 16 * (16 p + r), canonical words 16 g + 4 p .. 16 g + 4 p + 3 of
//           row 16 t + r (p = 0..3: the four 32-code parts of the group);
//   scales: f16 [T][G][16], the scale of row 16 t + r and group g at [t][g][r];
//   zeros : u8 [T][G][8], byte j = zero point of row 16 t + 2 j (low nibble) and 2 j + 1.
// Rows past N are zero.  castforge_hip_int4g_from_planes restores the canonical arrays bit for
// bit.
//
// Kernel.  One workgroup of 16 waves per CU (its LDS request keeps a second one off the CU)
// runs for the whole launch: launch overhead and x staging are paid once per CU instead of
// once per 16-row tile.
//   * Work split: each problem gets a number of workgroups in proportion to its code bytes, and
//     spreads its rows over them in units of 8 rows, so every CU streams about the same number
//     of bytes of one matrix.  A workgroup's chunk sequence is, tile after tile, each tile's G
//     chunks; wave i processes positions i, i + 16, i + 32, ... (balanced to one chunk), with
//     a D-deep ring of loads that runs across tile boundaries.
//   * x (bf16, M rows) is copied into LDS once and converted to f16 in the order the nibble
//     decode produces, with a per-(row, chunk) power of two that brings the chunk's largest |x|
//     into [2^14, 2^15): every finite bf16 x is then exact in f16 (down to 2^-38 of the chunk's
//     largest value), and the scale is undone on the chunk's f32 partial.
//   * M = 1: every row of the MFMA's A operand is x (a broadcast LDS read); M = 2..4: A row i
//     is x row min(i mod 4, M - 1), rows 16 B apart in LDS beyond their G * 256 bytes so that
//     the 16 distinct fragments of a read fall in distinct banks; D rows 0..M-1 (lanes 0..15)
//     are the outputs, the other rows are discarded.  The MFMA count per chunk is the same
//     for every M, so M = 2..4 costs little more than M = 1.
//   * Decode: (w & 0x000F000F) | 0x64006400 is the f16 pair (1024 + q, 1024 + q'), the 0x00F0
//     nibbles give 1024 + 16 q; one packed f16 add of -(1024 + z) (or fma by 1/16 and add of
//     -(64 + z)) leaves the exact integers q - z, so every product x (q - z) is exact and the
//     MFMA's f32 sums carry the only rounding, as the reference's f32 loop does.
//   * Each wave keeps MR f32 partials per row of its current tile (lanes 0..15 of the MFMA
//     result) and stores them into its own LDS slot of that tile when it moves to another tile;
//     no barrier inside the loop.  After the loop one barrier, then the workgroup sums each
//     row's partials in wave order (the same bits on every run) and stores its rows.
#include <algorithm>
#include <map>
#include <type_traits>
#include <mutex>
#include <vector>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr int kGroup = 128;
constexpr uint32_t kOob = 0x80000000u;  // past every descriptor's range: reads 0, no traffic
#ifndef CFH_PLANES_WAVES
#define CFH_PLANES_WAVES 16
#endif
#ifndef CFH_PLANES_DEPTH
#define CFH_PLANES_DEPTH 3
#endif
constexpr int kWaves = CFH_PLANES_WAVES;
constexpr int kDepth = CFH_PLANES_DEPTH;
// workgroups per CU (their LDS request keeps any more off a CU) and the cache policy of the
// streamed loads (2 = non-temporal: each byte is read once)
#ifndef CFH_PLANES_WG_PER_CU
#define CFH_PLANES_WG_PER_CU 1
#endif
#ifndef CFH_PLANES_CPOL
#define CFH_PLANES_CPOL 2
#endif
constexpr int kWgPerCu = CFH_PLANES_WG_PER_CU;
constexpr int kLdsMax = 160 * 1024;
constexpr int kLdsFloor = kLdsMax / (kWgPerCu + 1) + 2048;

struct PProblem {
    const uint8_t *codes;
    const uint16_t *scales;
    const uint8_t *zeros;
    const uint16_t *x;  // bf16 [M, K]
    void *y;
    int32_t n, G;       // rows, groups (K / 128)
    int32_t units;      // ceil(n / 8)
    int32_t wg0, wgs;   // this problem's workgroups [wg0, wg0 + wgs)
    int32_t m;          // rows of x (and y) of this problem
};

template <int NP>
struct PBatch {
    PProblem p[NP];
    int32_t count, y_bf16;
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
    uint32_t v;
    asm("v_mov_b32 %0, %1" : "=v"(v) : "i"(c));
    return v;
}

__device__ __forceinline__ half8_t pack8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(half8_t, make_uint4(a, b, c, d));
}

// Workgroup barrier for LDS data: this wave's LDS operations done (lgkmcnt(0)) and at most VM
// vector-memory loads still in flight, then s_barrier.  Unlike __syncthreads() it does not
// wait for the loads in flight (its release fence would); the single-thread fences only keep
// the compiler from moving memory accesses across it.
template <int VM>
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(VM) & ~(15 << 8));
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t as_u(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

struct Stage {
    uint32_t w[4];
    uint32_t sc, zb;
};

// x rows staged in LDS (M = 1: one row; otherwise up to MR = 4 fragment rows) and their row
// stride
template <int MR>
__host__ __device__ constexpr uint32_t x_row_stride(uint32_t G) { return MR == 1 ? G * 256 : G * 256 + 16; }

// LDS: [x as f16, M rows of G * 256 B at x_row_stride][per (chunk, row) 2^sh, G * MR * 4 B
// (16-byte padded)][partials: tiles x NW x 16 x MR f32]
template <int NW, int D, int MR>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW * kWgPerCu / 4)))
void planes_kernel(PBatch<CFH_MAX_BATCH> b) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = uni(tid >> 6);
    const int w = blockIdx.x;
    const int r16 = lane & 15, part = lane >> 4;

    // this workgroup's problem and rows [rlo, rhi): units of 8 rows spread over the problem's
    // workgroups (host-checked: wgs * units < 2^31)
    int pi = 0;
#pragma unroll
    for (int i = 1; i < CFH_MAX_BATCH; ++i)
        if (i < b.count && w >= b.p[i].wg0) pi = i;
    const PProblem &P = b.p[pi];
    const int G = P.G, local = w - P.wg0;
    const int u0 = static_cast<int>(static_cast<uint32_t>(local * P.units) / static_cast<uint32_t>(P.wgs));
    const int u1 = static_cast<int>(static_cast<uint32_t>((local + 1) * P.units) / static_cast<uint32_t>(P.wgs));
    const int rlo = 8 * u0, rhi = min(8 * u1, P.n);
    const int t0 = u0 >> 1, t1 = u1 > u0 ? (u1 + 1) >> 1 : t0;
    const int ntiles = t1 - t0, npos = ntiles * G;
    const int M = MR == 1 ? 1 : P.m;
    const uint32_t rowb = static_cast<uint32_t>(G) * (kGroup * 2), RS = x_row_stride<MR>(static_cast<uint32_t>(G));
    const uint32_t soff = (RS * static_cast<uint32_t>(M) + 15) & ~15u;
    const uint32_t aoff = soff + ((static_cast<uint32_t>(G) * MR * 4 + 15) & ~15u);
    float *const accs = reinterpret_cast<float *>(lds + aoff);

    // partials to zero, before any copy into LDS is in flight (an LDS write after an LDS-bound
    // copy is made to wait for every load in flight)
    for (int i = tid; i < ntiles * NW * 16 * MR; i += 64 * NW) accs[i] = 0.0f;

    // x (bf16) straight into LDS, 1 KB per wave-wide copy, row m at m * RS
    const int nblk = static_cast<int>((rowb + 1023u) / 1024u);
    for (int i = wave; i < M * nblk; i += NW) {
        const int m = i / nblk, blk = i - m * nblk;
        const uint32_t e = blk * 1024u + lane * 16u;
        if (e < rowb)
            __builtin_amdgcn_global_load_lds(
                static_cast<const void *>(P.x + static_cast<size_t>(m) * G * kGroup + (e >> 1)),
                reinterpret_cast<__attribute__((address_space(3))) void *>(reinterpret_cast<uintptr_t>(lds) + m * RS +
                                                                           blk * 1024),
                16, 0, 0);
    }

    // the first D positions of this wave: positions wave, wave + NW, ... of the sequence of
    // the workgroup's tiles (t0 + t) and their chunks g
    const uint32_t chunks = static_cast<uint32_t>(((P.n + 15) >> 4) * G);
    const rsrc_t rcode = make_rsrc(P.codes, chunks * 1024u);
    const rsrc_t rscale = make_rsrc(P.scales, chunks * 32u);
    const rsrc_t rzero = make_rsrc(P.zeros, chunks * 8u);
    int lt = 0, lg = wave;  // load cursor (tile relative to t0, chunk)
    while (lg >= G) {
        lg -= G;
        ++lt;
    }
    int pt = lt, pg = lg;  // process cursor
    // per-lane offsets within a chunk, pushed out of range (OR kOob) for rows outside
    // [rlo, rhi) and for positions past the workgroup's tiles: recomputed when the tile changes.
    // Every lane needs its row's zero point (its codes are decoded as exact q - z); the scale
    // multiplies the MFMA result, whose output rows lanes 0..15 hold.
    uint32_t vcode, vscale, vzero;
    auto lane_offsets = [&]() __attribute__((always_inline)) {
        const int row = (t0 + lt) * 16 + r16;
        const bool ok = lt < ntiles && row >= rlo && row < rhi;
        const uint32_t m = ok ? 0u : kOob;
        vcode = (static_cast<uint32_t>(lane) * 16u) | m;
        vscale = (static_cast<uint32_t>(r16) * 2u) | (lane < 16 ? m : kOob);
        vzero = static_cast<uint32_t>(r16 >> 1) | m;
    };
    lane_offsets();
    auto load = [&](Stage &st) __attribute__((always_inline)) {
        const uint32_t chunk = static_cast<uint32_t>((t0 + lt) * G + lg);
        const uint4 v = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rcode, vcode + chunk * 1024u, 0, CFH_PLANES_CPOL));
        st.w[0] = v.x;
        st.w[1] = v.y;
        st.w[2] = v.z;
        st.w[3] = v.w;
        st.sc = __builtin_amdgcn_raw_buffer_load_b16(rscale, vscale + chunk * 32u, 0, 0);
        st.zb = __builtin_amdgcn_raw_buffer_load_b8(rzero, vzero + chunk * 8u, 0, 0);
        lg += NW;
        if (lg >= G) {
            do {
                lg -= G;
                ++lt;
            } while (lg >= G);
            lane_offsets();
        }
    };
    Stage st[D];
    static_for<D>([&](auto i) __attribute__((always_inline)) {
        load(st[i]);
        __builtin_amdgcn_sched_barrier(0);
    });
    // this wave's copies of x have landed (the D positions issued after them may still be in
    // flight) and its LDS writes are done
    lds_barrier<3 * D>();

    // x to f16 in the decode's order: per 8 values the pairs (0, 4), (1, 5), (2, 6), (3, 7) of
    // one code word.  Eight lanes (16 values each) hold one chunk of 128 values: they agree on
    // the power of two 2^-sh that brings its largest |x| into [2^14, 2^15) (every finite bf16
    // is then exact in f16 down to 2^-38 of that value); 2^sh is kept per chunk.
    {
        constexpr int kPerm[16] = {0, 4, 1, 5, 2, 6, 3, 7, 8, 12, 9, 13, 10, 14, 11, 15};
        const int per_row = G * 8, total = M * per_row;
        for (int base = 0; base < total; base += 64 * NW) {  // uniform trip count
            const int i = base + tid;
            const bool act = i < total;
            const int ii = act ? i : 0;
            const int m = ii / per_row, j = ii - m * per_row;  // 8 | per_row: a chunk's 8 lanes share m
            uint16_t *px = reinterpret_cast<uint16_t *>(lds + m * RS) + j * 16;
            const uint4 r0 = *reinterpret_cast<const uint4 *>(px);
            const uint4 r1 = *reinterpret_cast<const uint4 *>(px + 8);
            const uint32_t wv[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
            uint32_t emax = 0;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                emax = max(emax, (wv[q] >> 7) & 0xFFu);
                emax = max(emax, (wv[q] >> 23) & 0xFFu);
            }
            {  // over the chunk's 8 lanes (DPP: xor 1, xor 2, half-row mirror)
                int e = static_cast<int>(emax);
                e = max(e, __builtin_amdgcn_mov_dpp(e, 0xB1, 0xF, 0xF, false));
                e = max(e, __builtin_amdgcn_mov_dpp(e, 0x4E, 0xF, 0xF, false));
                e = max(e, __builtin_amdgcn_mov_dpp(e, 0x141, 0xF, 0xF, false));
                emax = static_cast<uint32_t>(e);
            }
            // largest |x| < 2^(emax - 126): scale by 2^-sh so that it lands in [2^14, 2^15)
            int sh = static_cast<int>(emax) - 127 - 14;
            sh = sh < -126 ? -126 : (sh > 126 ? 126 : sh);
            const float pre = __uint_as_float(static_cast<uint32_t>(127 - sh) << 23);
            const float post = __uint_as_float(static_cast<uint32_t>(127 + sh) << 23);
            uint32_t o[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int s0 = kPerm[2 * q], s1 = kPerm[2 * q + 1];
                const float f0 = bf16_to_f32(static_cast<uint16_t>(wv[s0 >> 1] >> (16 * (s0 & 1)))) * pre;
                const float f1 = bf16_to_f32(static_cast<uint16_t>(wv[s1 >> 1] >> (16 * (s1 & 1)))) * pre;
                o[q] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f0))) |
                       (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f1))) << 16);
            }
            if (act) {
                *reinterpret_cast<uint4 *>(px) = make_uint4(o[0], o[1], o[2], o[3]);
                *reinterpret_cast<uint4 *>(px + 8) = make_uint4(o[4], o[5], o[6], o[7]);
                if ((i & 7) == 0) reinterpret_cast<float *>(lds + soff)[(j >> 3) * MR + m] = post;
            }
        }
    }
    lds_barrier<63>();

    const uint32_t LO = vgpr_const(0x000F000Fu), HI = vgpr_const(0x00F000F0u), MG = vgpr_const(0x64006400u);
    // this lane's x fragment row (D rows 0..M-1 of lanes 0..4 MR - 1 are the outputs) and the
    // first of the 4 D rows it holds
    const uint32_t xrow = MR == 1 ? 0u : static_cast<uint32_t>(min(r16 & (MR - 1), M - 1)) * RS;
    const uint32_t prow = MR == 1 ? 0u : 4u * static_cast<uint32_t>(part & (MR / 4 - 1));
    // per lane: the running partial of D rows 0..MR-1 (MR = 1: a scalar, as D rows are equal)
    typedef typename std::conditional<MR == 1, float, floatx4>::type acc_t;
    acc_t acc = acc_t{};
    const int steps = npos > wave ? (npos - wave + NW - 1) / NW : 0;
    // the oldest stage is consumed, then refilled with the position D steps ahead (keeping
    // about 48 KB in flight per CU: deeper rings measured slower); every step of the loop runs
    // (steps past the wave's last position read zero codes and add nothing), so the number of
    // loads in flight is the same on every path
    for (int k = 0; k < steps; k += D) {
        static_for<D>([&](auto ii) __attribute__((always_inline)) {
            constexpr int i = decltype(ii)::value;
            const bool live = pt < ntiles;
            const Stage &s = st[i];
            const int g = live ? pg : 0;  // a step past the end reads chunk 0 (in range)
            const uint8_t *xa = lds + xrow + g * (kGroup * 2) + part * 64;
            const half8_t a0 = *reinterpret_cast<const half8_t *>(xa);
            const half8_t a1 = *reinterpret_cast<const half8_t *>(xa + 16);
            const half8_t a2 = *reinterpret_cast<const half8_t *>(xa + 32);
            const half8_t a3 = *reinterpret_cast<const half8_t *>(xa + 48);
            // 2^sh of rows 0..MR-1 for this chunk
            acc_t post;
            if constexpr (MR == 1) post = reinterpret_cast<const float *>(lds + soff)[g];
            else post = *reinterpret_cast<const floatx4 *>(lds + soff + (g * MR + prow) * 4);
            const uint32_t w0 = s.w[0], w1 = s.w[1], w2 = s.w[2], w3 = s.w[3];
            const uint32_t w08 = w0 >> 8, w18 = w1 >> 8, w28 = w2 >> 8, w38 = w3 >> 8;
            const uint32_t zi = (s.zb >> (4 * (r16 & 1))) & 15u;
            const float sc = f16_to_f32(static_cast<uint16_t>(s.sc));
            acc_t part_sum;
            {
                // (1024 + q) - (1024 + z) and (1024 + 16 q) / 16 - (64 + z): exact small integers
                const half2_t zc1024 = as_h2((0xE400u + zi) * 0x00010001u);
                const half2_t zc64 = as_h2((0xD400u + (zi << 4)) * 0x00010001u);
                const half2_t sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
                auto dec = [&](uint32_t ww, uint32_t w8) __attribute__((always_inline)) {
                    return pack8(as_u(as_h2((ww & LO) | MG) + zc1024), as_u(as_h2((ww & HI) | MG) * sixteenth + zc64),
                                 as_u(as_h2((w8 & LO) | MG) + zc1024), as_u(as_h2((w8 & HI) | MG) * sixteenth + zc64));
                };
                // two accumulation chains halve the MFMA dependency latency
                floatx4 pa = floatx4{0.f, 0.f, 0.f, 0.f}, pb = pa;
                pa = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, dec(w0, w08), pa, 0, 0, 0);
                pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, dec(w1, w18), pb, 0, 0, 0);
                pa = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, dec(w2, w28), pa, 0, 0, 0);
                pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(a3, dec(w3, w38), pb, 0, 0, 0);
                // a separate multiply and add (no contraction): chunk results that cancel
                // exactly sum to exactly zero
                if constexpr (MR == 1) {
                    part_sum = __fmul_rn(pa[0] + pb[0], sc * post);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) part_sum[q] = __fmul_rn(pa[q] + pb[q], sc * post[q]);
                }
            }
            if constexpr (MR == 1) {
                acc = __fadd_rn(acc, live ? part_sum : 0.0f);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) acc[q] = __fadd_rn(acc[q], live ? part_sum[q] : 0.0f);
            }
            // next position; a wave's positions in one tile are consecutive steps, so one store
            // of its partials per tile
            const int tile = pt;
            pg += NW;
            while (pg >= G) {
                pg -= G;
                ++pt;
            }
            if (live && pt != tile) {
                if (lane < (MR == 1 ? 16 : 4 * MR)) {
                    float *dst = accs + (tile * NW + wave) * 16 * MR + (MR == 1 ? lane : 4 * lane);
                    if constexpr (MR == 1) dst[0] = acc;
                    else *reinterpret_cast<floatx4 *>(dst) = acc;
                }
                acc = acc_t{};
            }
            load(st[i]);
            __builtin_amdgcn_sched_barrier(0);
        });
    }
    lds_barrier<63>();  // every wave's partials are in LDS

    // rows of this workgroup: the waves' partials in wave order (the same bits on every run)
    for (int i = tid; i < ntiles * 16 * M; i += 64 * NW) {
        const int r = i / M, m = i - r * M;
        const int row = (t0 + (r >> 4)) * 16 + (r & 15);
        if (row >= rlo && row < rhi) {
            const float *pa = accs + (r >> 4) * NW * 16 * MR +
                              (MR == 1 ? (r & 15) : ((r & 15) + 16 * (m >> 2)) * 4 + (m & 3));
            float v = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) v += pa[w2 * 16 * MR];
            const int64_t o = static_cast<int64_t>(m) * P.n + row;
            if (b.y_bf16) static_cast<uint16_t *>(P.y)[o] = f32_to_bf16_rne(v);
            else static_cast<float *>(P.y)[o] = v;
        }
    }
}

// ---- M = 2..16: x in registers --------------------------------------------------------------------
// planes_xr_kernel: the design above with x held in registers instead of LDS, so that x's size
// bounds neither K nor M and every matrix streams its planes once.  A row of x is an A row of
// the MFMA (A row i is x row min(i mod MR, M - 1), MR = 4, 8 or 16), so one chunk costs the same
// 4 MFMAs at every M up to 16.
//   * Each wave owns chunks g = wave, wave + NW, ... of its workgroup's tiles and walks them
//     chunk by chunk, every tile of a chunk in turn.  A chunk's x fragment (64 bytes a lane: the
//     32 values of the lane's A row that its part of the MFMA reads) is loaded with the chunk's
//     first position, ahead of that position's codes in the same ring stage, and converted to
//     f16 with the per-(row, chunk) power of two when the wave reaches that position; the
//     chunk's other tiles reuse it.  Per workgroup x is read once, from L2.
//   * Each position's partial (D rows 0..MR-1: 16 bytes a lane) is added into the wave's own LDS
//     slot of its tile, in the wave's chunk order; only the wave itself touches its slots, so
//     there is no barrier until the end, where the workgroup sums each row's slots in wave
//     order (the same bits on every run).
//   * LDS holds only the slots: tiles x NW x 16 x MR f32 per workgroup.
// waves and ring depth: 16 waves at MR = 4 and 8; at MR = 16 the slots of 16 waves would not
// fit LDS next to the waves' x areas for the row counts of a 7B block, so 8 with a deeper ring
#ifndef CFH_PLANES_XR_WAVES
#define CFH_PLANES_XR_WAVES 16
#endif
#ifndef CFH_PLANES_XR_DEPTH
#define CFH_PLANES_XR_DEPTH 3
#endif
#ifndef CFH_PLANES_XR_WAVES16
#define CFH_PLANES_XR_WAVES16 8
#endif
#ifndef CFH_PLANES_XR_DEPTH16
#define CFH_PLANES_XR_DEPTH16 4
#endif
// the cost of converting one x value in streamed bytes, for the work split (MR = 4, 8 / MR = 16;
// measured at M = 8: 1.0 best of 1..3; at M = 16: 39.3 / 37.3 / 36.7 / 36.6 us for 1 / 1.5 / 2 /
// 2.5)
#ifndef CFH_PLANES_XR_XCOST
#define CFH_PLANES_XR_XCOST 1.0
#endif
#ifndef CFH_PLANES_XR_XCOST16
#define CFH_PLANES_XR_XCOST16 2.0
#endif
// one ring stage: one position's codes, scale and zero point and, when it is its chunk's last
// tile, the next chunk's x
template <int MR>
struct XStage {
    uint32_t w[4];
    uint32_t sc, zb;
    uint4 x[MR / 4];
};

template <int NW, int D, int MR>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW * kWgPerCu / 4)))
void planes_xr_kernel(PBatch<CFH_MAX_BATCH> b) {
    // a chunk's partial is rounded on its own before it is added (no contraction into an fma):
    // chunk results that cancel exactly sum to exactly zero
#pragma clang fp contract(off)
    static_assert(MR == 4 || MR == 8 || MR == 16, "MR is 4, 8 or 16");
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = uni(tid >> 6);
    const int w = blockIdx.x;
    const int r16 = lane & 15, part = lane >> 4;

    int pi = 0;
#pragma unroll
    for (int i = 1; i < CFH_MAX_BATCH; ++i)
        if (i < b.count && w >= b.p[i].wg0) pi = i;
    const PProblem &P = b.p[pi];
    const int G = P.G, M = P.m, local = w - P.wg0;
    const int u0 = static_cast<int>(static_cast<uint32_t>(local * P.units) / static_cast<uint32_t>(P.wgs));
    const int u1 = static_cast<int>(static_cast<uint32_t>((local + 1) * P.units) / static_cast<uint32_t>(P.wgs));
    const int rlo = 8 * u0, rhi = min(8 * u1, P.n);
    const int t0 = u0 >> 1, t1 = u1 > u0 ? (u1 + 1) >> 1 : t0;
    const int ntiles = t1 - t0;
    constexpr int kSlot = 16 * MR;        // floats of one (tile, wave) slot
    const bool out_lane = lane < 4 * MR;  // lanes holding D rows 0..MR-1
    float *const accs = reinterpret_cast<float *>(lds);
    float *const mine = accs + wave * kSlot + 4 * lane;  // slot (t, wave) at mine + t * NW * kSlot
    // this wave's x area after the slots: MR rows of a chunk as f16 (256 bytes each), then their
    // post factors
    uint8_t *const xarea = lds + ntiles * NW * kSlot * 4 + wave * (MR * 256 + 64);

    for (int t = 0; t < ntiles; ++t)
        if (out_lane) *reinterpret_cast<floatx4 *>(mine + t * NW * kSlot) = floatx4{0.f, 0.f, 0.f, 0.f};

    const int nc = G > wave ? (G - wave + NW - 1) / NW : 0;  // chunks of this wave
    const int nsteps = nc * ntiles;
    const uint32_t chunks = static_cast<uint32_t>(((P.n + 15) >> 4) * G);
    const rsrc_t rcode = make_rsrc(P.codes, chunks * 1024u);
    const rsrc_t rscale = make_rsrc(P.scales, chunks * 32u);
    const rsrc_t rzero = make_rsrc(P.zeros, chunks * 8u);
    const uint32_t rowb = static_cast<uint32_t>(G) * (kGroup * 2);
    const rsrc_t rx = make_rsrc(P.x, static_cast<uint32_t>(M) * rowb);
    // a chunk's x: load i brings rows 4 i .. 4 i + 3 (clamped to M - 1), 16 bytes a lane
    auto xrow = [&](int i) __attribute__((always_inline)) { return min(4 * i + part, M - 1); };

    int lc = 0, lt = 0;  // load cursor: the wave's chunk index, tile (relative to t0)
    auto load_x = [&](uint4 (&xr)[MR / 4], int c) __attribute__((always_inline)) {
        const uint32_t xo = c < nc ? static_cast<uint32_t>(wave + c * NW) * (kGroup * 2) + static_cast<uint32_t>(r16) * 16u : kOob;
        static_for<MR / 4>([&](auto jj) __attribute__((always_inline)) {
            constexpr int j = decltype(jj)::value;
            xr[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  rx, xo + static_cast<uint32_t>(xrow(j)) * rowb, 0, 0));
        });
    };
    auto load = [&](XStage<MR> &st) __attribute__((always_inline)) {
        const uint32_t g = static_cast<uint32_t>(wave + lc * NW);
        if (lt == ntiles - 1) load_x(st.x, lc + 1);  // the chunk's last tile: the next chunk's x first
        // rows outside [rlo, rhi) and chunks past the wave's read zeros (offsets pushed out of
        // range) and add nothing
        const int row = (t0 + lt) * 16 + r16;
        const uint32_t m = lc < nc && row >= rlo && row < rhi ? 0u : kOob;
        const uint32_t chunk = static_cast<uint32_t>(t0 + lt) * static_cast<uint32_t>(G) + g;
        const uint4 v = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rcode, ((static_cast<uint32_t>(lane) * 16u) | m) + chunk * 1024u, 0,
                                                         CFH_PLANES_CPOL));
        st.w[0] = v.x;
        st.w[1] = v.y;
        st.w[2] = v.z;
        st.w[3] = v.w;
        st.sc = __builtin_amdgcn_raw_buffer_load_b16(
            rscale, ((static_cast<uint32_t>(r16) * 2u) | (out_lane ? m : kOob)) + chunk * 32u, 0, 0);
        st.zb = __builtin_amdgcn_raw_buffer_load_b8(rzero, (static_cast<uint32_t>(r16 >> 1) | m) + chunk * 8u, 0, 0);
        if (++lt == ntiles) {
            lt = 0;
            ++lc;
        }
    };

    // a chunk's x to f16 in the decode's order (per 8 values the pairs (0, 4), (1, 5), (2, 6),
    // (3, 7)), scaled by 2^-sh so that the largest |x| of the row's chunk (its 16 lanes of a load)
    // lands in [2^14, 2^15), written to the wave's x area; then each lane reads its A fragment
    // (row r16 mod MR, values 32 part .. 32 part + 31) and the post factors 2^sh of its D rows
    // 4 (part mod MR / 4) + q
    const int prow = 4 * (part & (MR / 4 - 1));
    half8_t xa[4];
    floatx4 post;
    auto convert = [&](const uint4 (&xr)[MR / 4]) __attribute__((always_inline)) {
        static_for<MR / 4>([&](auto ii) __attribute__((always_inline)) {
            constexpr int i = decltype(ii)::value;
            const uint32_t wv[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
            uint32_t emax = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t a = (wv[q] >> 7) & 0xFFu, c = (wv[q] >> 23) & 0xFFu;
                emax = emax > a ? emax : a;
                emax = emax > c ? emax : c;
            }
            {  // over the row's 16 lanes (DPP row rotations by 1, 2, 4, 8)
                int e = static_cast<int>(emax);
                e = max(e, __builtin_amdgcn_mov_dpp(e, 0x121, 0xF, 0xF, false));
                e = max(e, __builtin_amdgcn_mov_dpp(e, 0x122, 0xF, 0xF, false));
                e = max(e, __builtin_amdgcn_mov_dpp(e, 0x124, 0xF, 0xF, false));
                e = max(e, __builtin_amdgcn_mov_dpp(e, 0x128, 0xF, 0xF, false));
                emax = static_cast<uint32_t>(e);
            }
            int sh = static_cast<int>(emax) - 127 - 14;
            sh = sh < -126 ? -126 : (sh > 126 ? 126 : sh);
            const float pre = __uint_as_float(static_cast<uint32_t>(127 - sh) << 23);
            auto h = [&](int e) __attribute__((always_inline)) {
                const uint32_t u = wv[e >> 1];
                const float f = __uint_as_float((e & 1) ? (u & 0xFFFF0000u) : (u << 16)) * pre;
                return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f)));
            };
            const int row = 4 * i + part;
            *reinterpret_cast<uint4 *>(xarea + row * 256 + r16 * 16) =
                make_uint4(h(0) | (h(4) << 16), h(1) | (h(5) << 16), h(2) | (h(6) << 16), h(3) | (h(7) << 16));
            if (r16 == 0)
                reinterpret_cast<float *>(xarea + MR * 256)[row] = __uint_as_float(static_cast<uint32_t>(127 + sh) << 23);
        });
        const uint8_t *xs = xarea + (r16 & (MR - 1)) * 256 + part * 64;
        static_for<4>([&](auto jj) __attribute__((always_inline)) {
            constexpr int j = decltype(jj)::value;
            xa[j] = *reinterpret_cast<const half8_t *>(xs + 16 * j);
        });
        post = *reinterpret_cast<const floatx4 *>(xarea + MR * 256 + prow * 4);
    };

    // the first chunk's x, then the ring; each stage of a chunk's last tiles carries the next
    // chunk's x, converted right after that stage's refill is issued (while the wave waits for
    // the next stage's loads)
    uint4 x0[MR / 4];
    load_x(x0, 0);
    XStage<MR> st[D];
    static_for<D>([&](auto i) __attribute__((always_inline)) {
        load(st[i]);
        __builtin_amdgcn_sched_barrier(0);
    });
    convert(x0);

    const uint32_t LO = vgpr_const(0x000F000Fu), HI = vgpr_const(0x00F000F0u), MG = vgpr_const(0x64006400u);
    int pc = 0, pt = 0;  // process cursor: the wave's chunk index, tile
    const int steps = (nsteps + D - 1) / D * D;
    for (int k = 0; k < steps; k += D) {
        static_for<D>([&](auto ii) __attribute__((always_inline)) {
            constexpr int i = decltype(ii)::value;
            XStage<MR> &s = st[i];
            {
                const uint32_t w0 = s.w[0], w1 = s.w[1], w2 = s.w[2], w3 = s.w[3];
                const uint32_t w08 = w0 >> 8, w18 = w1 >> 8, w28 = w2 >> 8, w38 = w3 >> 8;
                const uint32_t zi = (s.zb >> (4 * (r16 & 1))) & 15u;
                const float sc = f16_to_f32(static_cast<uint16_t>(s.sc));
                // (1024 + q) - (1024 + z) and (1024 + 16 q) / 16 - (64 + z): exact small integers
                const half2_t zc1024 = as_h2((0xE400u + zi) * 0x00010001u);
                const half2_t zc64 = as_h2((0xD400u + (zi << 4)) * 0x00010001u);
                const half2_t sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
                auto dec = [&](uint32_t ww, uint32_t w8) __attribute__((always_inline)) {
                    return pack8(as_u(as_h2((ww & LO) | MG) + zc1024), as_u(as_h2((ww & HI) | MG) * sixteenth + zc64),
                                 as_u(as_h2((w8 & LO) | MG) + zc1024), as_u(as_h2((w8 & HI) | MG) * sixteenth + zc64));
                };
                // two accumulation chains halve the MFMA dependency latency
                floatx4 pa = floatx4{0.f, 0.f, 0.f, 0.f}, pb = pa;
                pa = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[0], dec(w0, w08), pa, 0, 0, 0);
                pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[1], dec(w1, w18), pb, 0, 0, 0);
                pa = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[2], dec(w2, w28), pa, 0, 0, 0);
                pb = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[3], dec(w3, w38), pb, 0, 0, 0);
                if (pc < nc && out_lane) {
                    floatx4 *dst = reinterpret_cast<floatx4 *>(mine + pt * NW * kSlot);
                    floatx4 a = *dst;
#pragma unroll
                    for (int q = 0; q < 4; ++q) a[q] = a[q] + (pa[q] + pb[q]) * (sc * post[q]);
                    *dst = a;
                }
            }
            const bool last = pt == ntiles - 1;
            // the next chunk's x moved out of the stage (opaque copies: the refill may then load
            // into the stage's own registers, none rotate between iterations)
            uint4 xn[MR / 4];
            if (last) {
#pragma unroll
                for (int j = 0; j < MR / 4; ++j) {
                    uint32_t a = s.x[j].x, c = s.x[j].y, d = s.x[j].z, e = s.x[j].w;
                    asm volatile("v_mov_b32 %0, %1" : "=v"(xn[j].x) : "v"(a));
                    asm volatile("v_mov_b32 %0, %1" : "=v"(xn[j].y) : "v"(c));
                    asm volatile("v_mov_b32 %0, %1" : "=v"(xn[j].z) : "v"(d));
                    asm volatile("v_mov_b32 %0, %1" : "=v"(xn[j].w) : "v"(e));
                }
            }
            if (++pt == ntiles) {
                pt = 0;
                ++pc;
            }
            load(s);
            if (last) convert(xn);
            __builtin_amdgcn_sched_barrier(0);
        });
    }
    lds_barrier<63>();  // every wave's slots are final

    for (int i = tid; i < ntiles * 16 * M; i += 64 * NW) {
        const int r = i / M, m = i - r * M;
        const int row = (t0 + (r >> 4)) * 16 + (r & 15);
        if (row >= rlo && row < rhi) {
            const float *pa = accs + (r >> 4) * NW * kSlot + ((r & 15) + 16 * (m >> 2)) * 4 + (m & 3);
            float v = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) v += pa[w2 * kSlot];
            const int64_t o = static_cast<int64_t>(m) * P.n + row;
            if (b.y_bf16) static_cast<uint16_t *>(P.y)[o] = f32_to_bf16_rne(v);
            else static_cast<float *>(P.y)[o] = v;
        }
    }
}

// ---- M = 1: INT4 g128, NF4 and GGUF Q4_0 planes ------------------------------------------------
// planes_m1_kernel: the design above specialised to one row of x (a scalar partial per lane, a
// 64-byte problem record, 8 problems per launch), with the decode and metadata of its KIND.
//
// NF4 planes.  Codes: the same T x G chunks of 1024 bytes, but the piece of lane (p, r) holds
// canonical words 16 g + p, 16 g + 4 + p, 16 g + 8 + p, 16 g + 12 + p of row 16 t + r, so that
// the q-th words of the four parts, which one MFMA takes, are codes 32 q .. 32 q + 31 of the
// chunk: one block for every block size >= 32.  absmax: f32 [T][G][16][NBPC], NBPC = max(1,
// 128 / block) values per chunk and row (a block longer than a chunk repeats its absmax in each
// of its chunks).  Rows past N are zero.
//
// The decode table (code byte -> f16 hi and lo of its two codes' table values, 8 bytes, so
// hi + lo is the f32 table value exactly) is kept in LDS as 32 interleaved copies: lane l reads
// entry e at (e * 32 + l % 32) * 8, so the 32 lanes an LDS cycle serves hit 32 distinct bank
// pairs whatever the codes.  The persistent grid writes the 64 KB once per CU.
#ifndef CFH_NF4_PLANES_DEPTH
#define CFH_NF4_PLANES_DEPTH 2  // positions in flight per wave (3 and 4 measured slower)
#endif
constexpr int kNf4Depth = CFH_NF4_PLANES_DEPTH;
#ifndef CFH_PLANES_I4_DEPTH
#define CFH_PLANES_I4_DEPTH 2  // the INT4 kind of the kernel below (M = 1 over INT4 GEMV planes)
#endif
constexpr int kI4Depth = CFH_PLANES_I4_DEPTH;
#ifndef CFH_PLANES_M1_SPLIT
#define CFH_PLANES_M1_SPLIT 1  // M = 1 INT4 work split: 1 whole tiles, least largest share; 0 by bytes, 8-row units
#endif
#ifndef CFH_PLANES_XR_FROM
#define CFH_PLANES_XR_FROM 5  // M from which planes_xr_kernel serves every batch (2..5)
#endif
#ifndef CFH_PLANES_M1_GENERIC
#define CFH_PLANES_M1_GENERIC 1  // M = 1 over INT4 GEMV planes on planes_m1_kernel (0: planes_kernel)
#endif
constexpr int kXRegs = 2;  // x loads (four chunks each) a wave issues ahead of its ring (K <= 16384)
constexpr int kNf4LutCopies = 32;
constexpr int kNf4LutBytes = 256 * kNf4LutCopies * 8;
constexpr float kNf4Values[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

struct NProblem {
    const uint8_t *codes;
    const float *absmax;   // NF4: absmax planes; Q4_0: d planes; INT4: scale planes
    const uint8_t *zeros;  // INT4: zero-point planes
    const uint16_t *x;     // bf16 [1, K]
    void *y;
    int32_t n, G, units, wg0, wgs;
    int32_t ush;  // a unit is 8 << ush rows (0: half tiles, 1: whole tiles)
};
static_assert(sizeof(NProblem) == 64, "one problem record, 64 bytes");

// what planes_m1_kernel decodes
constexpr int kKindNf4 = 0;   // NF4 planes, table decode
constexpr int kKindQ40 = 1;   // GGUF Q4_0 GEMV planes, exact q - 8
constexpr int kKindInt4 = 2;  // INT4 g128 GEMV planes, exact q - z (the M = 1 form of planes_kernel)

struct NBatch {
    NProblem p[CFH_MAX_BATCH];
    int32_t count, y_bf16;
};

struct NStage {
    uint32_t w[4];
    uint32_t am[4];
};

// LDS: [decode table, 64 KB (NF4 only)][x as f16, G * 256 B][per chunk 2^sh, G * 4 B (16-byte
// padded)][partials: tiles x NW x 16 f32]
// Q4_0 GEMV planes (castforge_hip_gguf_q4_0_to_gemv_planes): chunk (t, g) holds at byte
// 16 * (16 p + r) the 16-byte part p of chunk g of row 16 t + r of the GGUF planes (elements
// 8p..8p+7 of its four blocks, so MFMA q takes block q), d f16 [T][G][16][4].
// Q40: the GGUF Q4_0 form over Q4_0 GEMV planes (below): codes decoded to the exact f16
// q - 8 like INT4, one f16 d per block of 32 (NBPC = 4 blocks per chunk), x in the INT4
// decode's order.
// INT4 (NBPC = 1): the INT4 g128 GEMV planes (planes_kernel's layout and arithmetic at M = 1,
// bit for bit: per chunk two MFMA chains over words 0, 2 and 1, 3, then RN(RN(pa + pb) * RN(s *
// post))), with x in the INT4 decode's order.
template <int NW, int D, int NBPC, int KIND = kKindNf4>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW / 4)))
void planes_m1_kernel(NBatch b) {
    constexpr bool Q40 = KIND == kKindQ40, I4 = KIND == kKindInt4;
    static_assert(!I4 || NBPC == 1, "INT4: one group per chunk");
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = uni(tid >> 6);
    const int w = blockIdx.x;
    const int r16 = lane & 15, part = lane >> 4;

    int pi = 0;
#pragma unroll
    for (int i = 1; i < CFH_MAX_BATCH; ++i)
        if (i < b.count && w >= b.p[i].wg0) pi = i;
    const NProblem &P = b.p[pi];
    const int G = P.G, local = w - P.wg0;
    const int u0 = static_cast<int>(static_cast<uint32_t>(local * P.units) / static_cast<uint32_t>(P.wgs));
    const int u1 = static_cast<int>(static_cast<uint32_t>((local + 1) * P.units) / static_cast<uint32_t>(P.wgs));
    const int r0 = u0 << (3 + P.ush), r1 = u1 << (3 + P.ush);
    const int rlo = r0, rhi = min(r1, P.n);
    const int t0 = r0 >> 4, t1 = u1 > u0 ? (r1 + 15) >> 4 : t0;
    const int ntiles = t1 - t0, npos = ntiles * G;
    const uint32_t rowb = static_cast<uint32_t>(G) * (kGroup * 2);
    constexpr uint32_t xoff = KIND == kKindNf4 ? kNf4LutBytes : 0u;
    const uint32_t soff = xoff + rowb;
    const uint32_t aoff = soff + ((static_cast<uint32_t>(G) * 4 + 15) & ~15u);
    float *const accs = reinterpret_cast<float *>(lds + aoff);

    // x first (straight into registers, 16 bytes a lane: wave load i holds chunks 4 i .. 4 i + 3,
    // lane (c4, j) elements 8 j .. 8 j + 7 of chunk 4 i + c4), then the ring; the LDS work and the
    // conversion run while both are in flight
    const int nxl = (G + 3) >> 2;
    const rsrc_t rx = make_rsrc(P.x, rowb);
    uint4 xr[kXRegs];
    static_for<kXRegs>([&](auto ii) __attribute__((always_inline)) {
        constexpr int i = decltype(ii)::value;
        const int xl = wave + i * NW;
        xr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rx, (xl < nxl ? 0u : kOob) | (lane * 16u), static_cast<uint32_t>(xl) * 1024u, 0));
    });

    const uint32_t chunks = static_cast<uint32_t>(((P.n + 15) >> 4) * G);
    const rsrc_t rcode = make_rsrc(P.codes, chunks * 1024u);
    constexpr uint32_t kMetaRow = Q40 ? 8u : I4 ? 2u : 4u * NBPC;  // metadata bytes per row and chunk
    const rsrc_t ramax = make_rsrc(P.absmax, chunks * 16u * kMetaRow);
    const rsrc_t rzero = make_rsrc(P.zeros, I4 ? chunks * 8u : 0u);
    int lt = 0, lg = wave;
    while (lg >= G) {
        lg -= G;
        ++lt;
    }
    int pt = lt, pg = lg;
    // per-lane offsets, pushed out of range (OR kOob) for rows outside [rlo, rhi) and past the
    // workgroup's tiles; the chunk's own offset is wave-uniform (the loads' scalar offset).  The
    // absmax values multiply the MFMA result, whose rows lanes 0..15 hold (INT4: every lane
    // needs its row's zero point for the exact q - z decode).  A position past the workgroup's
    // tiles reads scale 0 (out of range): its partial is 0 times a finite value or, for
    // non-finite x, lands after the workgroup's last store of its running sum.
    uint32_t vcode, vam, vzero;
    auto lane_offsets = [&]() __attribute__((always_inline)) {
        const int row = (t0 + lt) * 16 + r16;
        const bool ok = lt < ntiles && row >= rlo && row < rhi;
        const uint32_t m = ok ? 0u : kOob;
        vcode = (static_cast<uint32_t>(lane) * 16u) | m;
        vam = (static_cast<uint32_t>(r16) * kMetaRow) | (lane < 16 ? m : kOob);
        vzero = static_cast<uint32_t>((r16 >> 3) * 4) | m;  // the dword with rows 8 (r / 8) .. + 7
    };
    lane_offsets();
    auto load = [&](NStage &st) __attribute__((always_inline)) {
        const uint32_t chunk = static_cast<uint32_t>((t0 + lt) * G + lg);
        const uint4 v = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rcode, vcode, chunk * 1024u, CFH_PLANES_CPOL));
        st.w[0] = v.x;
        st.w[1] = v.y;
        st.w[2] = v.z;
        st.w[3] = v.w;
        const uint32_t ao = chunk * (16u * kMetaRow);
        if constexpr (I4) {  // the group's f16 scale (lanes 0..15) and zero-point byte (all lanes)
            st.am[0] = __builtin_amdgcn_raw_buffer_load_b16(ramax, vam, ao, 0);
            st.am[1] = __builtin_amdgcn_raw_buffer_load_b32(rzero, vzero, chunk * 8u, 0);
        } else if constexpr (Q40) {  // the 4 blocks' f16 d
            const uint2 a = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ramax, vam, ao, 0));
            st.am[0] = a.x;
            st.am[1] = a.y;
        } else if constexpr (NBPC == 1) {
            st.am[0] = __builtin_amdgcn_raw_buffer_load_b32(ramax, vam, ao, 0);
        } else if constexpr (NBPC == 2) {
            const uint2 a = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ramax, vam, ao, 0));
            st.am[0] = a.x;
            st.am[1] = a.y;
        } else {
            const uint4 a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ramax, vam, ao, 0));
            st.am[0] = a.x;
            st.am[1] = a.y;
            st.am[2] = a.z;
            st.am[3] = a.w;
        }
        lg += NW;
        if (lg >= G) {
            do {
                lg -= G;
                ++lt;
            } while (lg >= G);
            lane_offsets();
        }
    };
    NStage st[D];
    static_for<D>([&](auto i) __attribute__((always_inline)) {
        load(st[i]);
        __builtin_amdgcn_sched_barrier(0);
    });

    // the decode table and the partials
    for (int i = tid; i < (KIND == kKindNf4 ? 256 * kNf4LutCopies : 0); i += 64 * NW) {
        const int e = i / kNf4LutCopies;
        const float v0 = kNf4Values[e & 15], v1 = kNf4Values[e >> 4];
        const _Float16 h0 = static_cast<_Float16>(v0), h1 = static_cast<_Float16>(v1);
        const _Float16 l0 = static_cast<_Float16>(v0 - static_cast<float>(h0));
        const _Float16 l1 = static_cast<_Float16>(v1 - static_cast<float>(h1));
        const half2_t hi = {h0, h1}, lo = {l0, l1};
        reinterpret_cast<uint2 *>(lds)[i] = make_uint2(as_u(hi), as_u(lo));
    }
    for (int i = tid; i < ntiles * NW * 16; i += 64 * NW) accs[i] = 0.0f;

    // x to f16, each chunk of 128 scaled by the power of two that brings its largest |x| into
    // [2^14, 2^15) (every finite bf16 is then exact in f16 down to 2^-38 of that value); 2^sh is
    // kept per chunk.  The 16 lanes of a DPP row hold one chunk.  NF4 keeps the natural order;
    // Q4_0 and INT4 take, per 8 values, the pairs (0, 4), (1, 5), (2, 6), (3, 7) of their decode.
    auto convert = [&](const uint4 &r, int xl) __attribute__((always_inline)) {
        const uint32_t wv[4] = {r.x, r.y, r.z, r.w};
        uint32_t emax = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            emax = max(emax, (wv[q] >> 7) & 0xFFu);
            emax = max(emax, (wv[q] >> 23) & 0xFFu);
        }
        {
            int e = static_cast<int>(emax);
            e = max(e, __builtin_amdgcn_mov_dpp(e, 0x128, 0xF, 0xF, false));  // row_ror:8
            e = max(e, __builtin_amdgcn_mov_dpp(e, 0x124, 0xF, 0xF, false));  // row_ror:4
            e = max(e, __builtin_amdgcn_mov_dpp(e, 0x4E, 0xF, 0xF, false));
            e = max(e, __builtin_amdgcn_mov_dpp(e, 0xB1, 0xF, 0xF, false));
            emax = static_cast<uint32_t>(e);
        }
        int sh = static_cast<int>(emax) - 127 - 14;
        sh = sh < -126 ? -126 : (sh > 126 ? 126 : sh);
        const float pre = __uint_as_float(static_cast<uint32_t>(127 - sh) << 23);
        constexpr int kPerm[8] = {0, 4, 1, 5, 2, 6, 3, 7};
        uint32_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int s0 = Q40 || I4 ? kPerm[2 * q] : 2 * q, s1 = Q40 || I4 ? kPerm[2 * q + 1] : 2 * q + 1;
            const float f0 = bf16_to_f32(static_cast<uint16_t>(wv[s0 >> 1] >> (16 * (s0 & 1)))) * pre;
            const float f1 = bf16_to_f32(static_cast<uint16_t>(wv[s1 >> 1] >> (16 * (s1 & 1)))) * pre;
            o[q] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f0))) |
                   (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f1))) << 16);
        }
        const int g = 4 * xl + part;
        if (xl < nxl && g < G) {
            *reinterpret_cast<uint4 *>(lds + xoff + static_cast<uint32_t>(g) * 256u + r16 * 16u) =
                make_uint4(o[0], o[1], o[2], o[3]);
            if (r16 == 0)
                reinterpret_cast<float *>(lds + soff)[g] = __uint_as_float(static_cast<uint32_t>(127 + sh) << 23);
        }
    };
    static_for<kXRegs>([&](auto ii) __attribute__((always_inline)) {
        constexpr int i = decltype(ii)::value;
        convert(xr[i], wave + i * NW);
    });
    for (int xl = wave + kXRegs * NW; xl < nxl; xl += NW) {  // K > 16384 only (waits for the ring too)
        const uint4 r = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, lane * 16u, static_cast<uint32_t>(xl) * 1024u, 0));
        convert(r, xl);
    }
    lds_barrier<63>();

    const uint32_t LO = vgpr_const(0x000F000Fu), HI = vgpr_const(0x00F000F0u), MG = vgpr_const(0x64006400u);
    const uint32_t lbase = static_cast<uint32_t>(lane & (kNf4LutCopies - 1)) * 8u;  // < 256
    // table entry of byte B of word v for this lane, at (byte * 32 + lane % 32) * 8: one byte
    // permute puts the byte at bits 8..15 and the lane's copy offset at bits 0..7
    auto entry = [&](uint32_t v, auto B) __attribute__((always_inline)) {
        constexpr uint32_t sel = 0x0C0C0000u | ((4u + decltype(B)::value) << 8);
        return *reinterpret_cast<const uint2 *>(lds + __builtin_amdgcn_perm(v, lbase, sel));
    };
    float acc = 0.0f;
    const int steps = npos > wave ? (npos - wave + NW - 1) / NW : 0;
    for (int k = 0; k < steps; k += D) {
        static_for<D>([&](auto ii) __attribute__((always_inline)) {
            constexpr int i = decltype(ii)::value;
            const bool live = pt < ntiles;
            const NStage &s = st[i];
            const int g = pg;
            // A fragment of MFMA q: x[128 g + 32 q + 8 p .. + 7] (INT4: x[128 g + 32 p + 8 q ..])
            const uint8_t *xa = lds + xoff + g * (kGroup * 2) + part * (I4 ? 64 : 16);
            constexpr int xq = I4 ? 16 : 64;
            const float post = reinterpret_cast<const float *>(lds + soff)[g];
            // one accumulation chain per block of the chunk (two for a single block, to halve the
            // MFMA dependency latency)
            constexpr int NC = NBPC == 1 ? 2 : NBPC;
            floatx4 c[NC];
#pragma unroll
            for (int j = 0; j < NC; ++j) c[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const half8_t a = *reinterpret_cast<const half8_t *>(xa + xq * q);
                const uint32_t wq = s.w[q];
                const int j = NBPC == 1 ? (q & 1) : q * NBPC / 4;
                if constexpr (Q40 || I4) {
                    // (1024 + q) - (1024 + z) and (1024 + 16 q) / 16 - (64 + z): the exact
                    // integers q - z (Q4_0: z = 8)
                    const uint32_t zi = I4 ? (s.am[1] >> (4 * (r16 & 7))) & 15u : 8u;
                    const half2_t zc1024 = as_h2((0xE400u + zi) * 0x00010001u);
                    const half2_t zc64 = as_h2((0xD400u + (zi << 4)) * 0x00010001u);
                    const half2_t sixteenth = {static_cast<_Float16>(0.0625f), static_cast<_Float16>(0.0625f)};
                    const uint32_t w8 = wq >> 8;
                    const half8_t bq = pack8(as_u(as_h2((wq & LO) | MG) + zc1024), as_u(as_h2((wq & HI) | MG) * sixteenth + zc64),
                                             as_u(as_h2((w8 & LO) | MG) + zc1024), as_u(as_h2((w8 & HI) | MG) * sixteenth + zc64));
                    c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bq, c[j], 0, 0, 0);
                } else {
                    const uint2 e0 = entry(wq, std::integral_constant<uint32_t, 0>{});
                    const uint2 e1 = entry(wq, std::integral_constant<uint32_t, 1>{});
                    const uint2 e2 = entry(wq, std::integral_constant<uint32_t, 2>{});
                    const uint2 e3 = entry(wq, std::integral_constant<uint32_t, 3>{});
                    c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pack8(e0.x, e1.x, e2.x, e3.x), c[j], 0, 0, 0);
                    c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pack8(e0.y, e1.y, e2.y, e3.y), c[j], 0, 0, 0);
                }
            }
            float v;
            if constexpr (I4) {
                v = __fmul_rn(c[0][0] + c[1][0], f16_to_f32(static_cast<uint16_t>(s.am[0])) * post);
            } else if constexpr (Q40) {
                float t = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    t = __fadd_rn(t, __fmul_rn(c[j][0], f16_to_f32(static_cast<uint16_t>(s.am[j >> 1] >> (16 * (j & 1))))));
                v = __fmul_rn(t, post);
            } else if constexpr (NBPC == 1) {
                v = __fmul_rn(__fmul_rn(c[0][0] + c[1][0], __uint_as_float(s.am[0])), post);
            } else {
                float t = 0.0f;
#pragma unroll
                for (int j = 0; j < NBPC; ++j) t = __fadd_rn(t, __fmul_rn(c[j][0], __uint_as_float(s.am[j])));
                v = __fmul_rn(t, post);
            }
            asm volatile("" : "+v"(v));  // the product rounds on its own: no fused multiply-add into acc
            acc = __fadd_rn(acc, v);
            const int tile = pt;
            pg += NW;
            while (pg >= G) {
                pg -= G;
                ++pt;
            }
            if (live && pt != tile) {
                if (lane < 16) accs[(tile * NW + wave) * 16 + lane] = acc;
                acc = 0.0f;
            }
            load(st[i]);
            __builtin_amdgcn_sched_barrier(0);
        });
    }
    lds_barrier<63>();

    for (int i = tid; i < ntiles * 16; i += 64 * NW) {
        const int row = (t0 + (i >> 4)) * 16 + (i & 15);
        if (row >= rlo && row < rhi) {
            const float *pa = accs + (i >> 4) * NW * 16 + (i & 15);
            float v = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) v += pa[w2 * 16];
            if (b.y_bf16) static_cast<uint16_t *>(P.y)[row] = f32_to_bf16_rne(v);
            else static_cast<float *>(P.y)[row] = v;
        }
    }
}

// ---- M = 1, INT4 g128 GEMV planes on the integer MFMA ------------------------------------------
// planes_i8_kernel: the M = 1 INT4 GEMV over the same GEMV planes, work split, ring and
// per-(tile, wave) partials as planes_m1_kernel, with the products formed exactly in integers:
//   * x: each chunk of 128 (one group) is scaled by 2^(147 - e), e the biased exponent of its
//     largest |x| (1 for zero and subnormal chunks): t = x * 2^(147 - e), |t| < 2^21.  Its nearest
//     integer X = p0 + 256 p1 + 65536 p2 (signed bytes p0, p1 in [-128, 127], p2 in [-32, 31])
//     comes from t + (2^23 + 0x408080), a float in [2^23, 2^24) whose low 23 bits are
//     X + 0x408080 (one xor and add give the three bytes); the residual t - X, |t - X| <= 1/2,
//     is the fourth piece p3 = RN(128 (t - X)).  So t = X + p3 / 128 exactly for every element
//     within 2^-20 of the chunk's largest, and to within 2^-28 of the largest for the others.  The
//     pieces are rows 0..3 of the MFMA's A operand (rows 4..15 repeat row 3; their results are
//     not used).
//   * codes: nibble q of the planes becomes the signed byte 16 (q - 8) = (q ^ 8) << 4: the high
//     nibbles of a word by one and-xor, the low ones after a 4-bit rotation.  Even elements of a
//     lane's 32 take one v_mfma_i32_16x16x64_i8, odd ones a second, into one i32 accumulator:
//     c_i = sum over the group of p_i 16 (q - 8), exact.
//   * the zero point: D_i = c_i + 16 (8 - z) S_i = 16 sum p_i (q - z) exactly, S_i = sum of p_i
//     over the chunk (kept per chunk in LDS, |D_i| < 2^22), and 16 sum t (q - z) =
//     L + D_3 / 128 + 65536 D_2 with L = D_0 + 256 D_1 (exact in i32), made f32 by two fmas,
//     smallest term first.  The chunk's f32 partial is ((that * s) * 2^a) * 2^b with
//     2^(a + b) = 2^(e - 151), so y(2^k x) = 2^k y(x) bit for bit while no partial leaves the
//     f32 range.  A chunk holding inf or NaN gives NaN partials.
//   * per chunk: 12 VALU for the decode, 2 MFMAs and 3 LDS reads, against 36 VALU, 4 MFMAs and
//     4 LDS reads of the f16 form.
// LDS: [x pieces: per chunk 4 parts x (4 pieces x (16 B even, 16 B odd)) = 512 B][per chunk
// S0 | S1 << 16, S2 | S3 << 16, 2^a, 2^b: 16 B][partials: tiles x NW x 16 f32]
typedef int int32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kI8ChunkX = 512;
constexpr uint32_t kI8ChunkRec = 16;
// positions a wave loads into registers of their own ahead of the ring.  The E + D positions
// are issued right behind the wave's x loads, before x is awaited (19.87 against 20.00 us with
// x awaited first).  E = 1 / 2 / 3 over D = 2 that way: 19.85 / 19.72 / 19.97 us (with x
// awaited first, E = 1 / 4 / 6 / 8: 20.22 / 20.46 / 20.85 / 21.18 us); D = 3: 20.48 us.
constexpr int kI8Pre = 2;

template <int NW, int D>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW / 4)))
void planes_i8_kernel(NBatch b) {
    constexpr int E = kI8Pre;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = uni(tid >> 6);
    const int w = blockIdx.x;
    const int r16 = lane & 15, part = lane >> 4;

    int pi = 0;
#pragma unroll
    for (int i = 1; i < CFH_MAX_BATCH; ++i)
        if (i < b.count && w >= b.p[i].wg0) pi = i;
    const NProblem &P = b.p[pi];
    const int G = P.G, local = w - P.wg0;
    const int u0 = static_cast<int>(static_cast<uint32_t>(local * P.units) / static_cast<uint32_t>(P.wgs));
    const int u1 = static_cast<int>(static_cast<uint32_t>((local + 1) * P.units) / static_cast<uint32_t>(P.wgs));
    const int r0 = u0 << (3 + P.ush), r1 = u1 << (3 + P.ush);
    const int rlo = r0, rhi = min(r1, P.n);
    const int t0 = r0 >> 4, t1 = u1 > u0 ? (r1 + 15) >> 4 : t0;
    const int ntiles = t1 - t0, npos = ntiles * G;
    const uint32_t rowb = static_cast<uint32_t>(G) * (kGroup * 2);
    const uint32_t soff = static_cast<uint32_t>(G) * kI8ChunkX;
    const uint32_t aoff = soff + static_cast<uint32_t>(G) * kI8ChunkRec;
    float *const accs = reinterpret_cast<float *>(lds + aoff);

    // x first (straight into registers, 16 bytes a lane: wave load i holds chunks 4 i .. 4 i + 3,
    // lane (c4, j) elements 8 j .. 8 j + 7 of chunk 4 i + c4), then the weight ring
    const int nxl = (G + 3) >> 2;
    const rsrc_t rx = make_rsrc(P.x, rowb);
    uint4 xr[kXRegs];
    static_for<kXRegs>([&](auto ii) __attribute__((always_inline)) {
        constexpr int i = decltype(ii)::value;
        const int xl = wave + i * NW;
        xr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rx, (xl < nxl ? 0u : kOob) | (lane * 16u), static_cast<uint32_t>(xl) * 1024u, 0));
    });

    const uint32_t chunks = static_cast<uint32_t>(((P.n + 15) >> 4) * G);
    const rsrc_t rcode = make_rsrc(P.codes, chunks * 1024u);
    const rsrc_t rscale = make_rsrc(P.absmax, chunks * 32u);
    const rsrc_t rzero = make_rsrc(P.zeros, chunks * 8u);
    int lt = 0, lg = wave;
    while (lg >= G) {
        lg -= G;
        ++lt;
    }
    int pt = lt, pg = lg;
    // per-lane offsets, pushed out of range (OR kOob) for rows outside [rlo, rhi) and past the
    // workgroup's tiles: the f16 scale on lanes 0..15 (whose rows the MFMA result holds), the
    // zero-point dword with rows 8 (r / 8) .. + 7 on every lane.  A position past the tiles reads
    // scale 0 and is never stored.
    uint32_t vcode, vsc, vzero;
    auto lane_offsets = [&]() __attribute__((always_inline)) {
        const int row = (t0 + lt) * 16 + r16;
        const bool ok = lt < ntiles && row >= rlo && row < rhi;
        const uint32_t m = ok ? 0u : kOob;
        vcode = (static_cast<uint32_t>(lane) * 16u) | m;
        vsc = (static_cast<uint32_t>(r16) * 2u) | (lane < 16 ? m : kOob);
        vzero = static_cast<uint32_t>((r16 >> 3) * 4) | m;
    };
    lane_offsets();
    auto load = [&](NStage &st) __attribute__((always_inline)) {
        const uint32_t chunk = static_cast<uint32_t>((t0 + lt) * G + lg);
        const uint4 v = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rcode, vcode, chunk * 1024u, CFH_PLANES_CPOL));
        st.w[0] = v.x;
        st.w[1] = v.y;
        st.w[2] = v.z;
        st.w[3] = v.w;
        st.am[0] = __builtin_amdgcn_raw_buffer_load_b16(rscale, vsc, chunk * 32u, 0);
        st.am[1] = __builtin_amdgcn_raw_buffer_load_b32(rzero, vzero, chunk * 8u, 0);
        lg += NW;
        if (lg >= G) {
            do {
                lg -= G;
                ++lt;
            } while (lg >= G);
            lane_offsets();
        }
    };
    // the wave's first E positions go into registers of their own, then the ring's D: E + D
    // positions in flight while x is converted
    NStage pre[E], st[D];
    static_for<E>([&](auto i) __attribute__((always_inline)) {
        load(pre[i]);
        __builtin_amdgcn_sched_barrier(0);
    });
    static_for<D>([&](auto i) __attribute__((always_inline)) {
        load(st[i]);
        __builtin_amdgcn_sched_barrier(0);
    });

    for (int i = tid; i < ntiles * NW * 16; i += 64 * NW) accs[i] = 0.0f;

    // x to pieces.  The 16 lanes of a DPP row hold one chunk; lane j's 8 elements are the even
    // and odd elements 4 (j % 4) .. + 3 of part j / 4, i.e. dword j % 4 of each 16-byte block.
    auto convert = [&](const uint4 &r, int xl) __attribute__((always_inline)) {
        const uint32_t wv[4] = {r.x, r.y, r.z, r.w};  // element 2 q: low half of wv[q], 2 q + 1: high half
        int e = 1;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            e = max(e, static_cast<int>((wv[q] >> 7) & 0xFFu));
            e = max(e, static_cast<int>((wv[q] >> 23) & 0xFFu));
        }
        e = max(e, __builtin_amdgcn_mov_dpp(e, 0x128, 0xF, 0xF, false));  // row_ror:8
        e = max(e, __builtin_amdgcn_mov_dpp(e, 0x124, 0xF, 0xF, false));  // row_ror:4
        e = max(e, __builtin_amdgcn_mov_dpp(e, 0x4E, 0xF, 0xF, false));
        e = max(e, __builtin_amdgcn_mov_dpp(e, 0xB1, 0xF, 0xF, false));
        const int kx = 147 - e;
        // bytes 0..2 of pc[k] are the pieces p0, p1, p2 of element k, byte 0 of rc[k] is p3
        uint32_t pc[8], rc[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t h = wv[k >> 1];
            const float xf = __uint_as_float((k & 1) ? (h & 0xFFFF0000u) : (h << 16));
            const float t = __builtin_amdgcn_ldexpf(xf, kx);
            const float rf = t + 12615808.0f;  // 2^23 + 0x408080: rounds t to an integer
            const float res = t - (rf - 12615808.0f);  // both steps exact
            pc[k] = (__float_as_uint(rf) ^ 0x8080u) + 0xC00000u;
            rc[k] = __float_as_uint(__builtin_fmaf(res, 128.0f, 12582912.0f));  // 1.5 * 2^23 + p3
        }
        // gather: piece i of elements 0, 2, 4, 6 (even) and 1, 3, 5, 7 (odd), one byte each
        uint32_t ev[4], od[4];
        auto gather = [&](int k0, uint32_t *out) __attribute__((always_inline)) {
            const uint32_t a01 = __builtin_amdgcn_perm(pc[k0 + 2], pc[k0], 0x05010400u);  // p0[0] p0[2] p1[0] p1[2]
            const uint32_t a45 = __builtin_amdgcn_perm(pc[k0 + 6], pc[k0 + 4], 0x05010400u);
            const uint32_t b01 = __builtin_amdgcn_perm(pc[k0 + 2], pc[k0], 0x0C0C0602u);  // p2[0] p2[2]
            const uint32_t b45 = __builtin_amdgcn_perm(pc[k0 + 6], pc[k0 + 4], 0x0C0C0602u);
            const uint32_t c01 = __builtin_amdgcn_perm(rc[k0 + 2], rc[k0], 0x0C0C0400u);  // p3[0] p3[2]
            const uint32_t c45 = __builtin_amdgcn_perm(rc[k0 + 6], rc[k0 + 4], 0x0C0C0400u);
            out[0] = __builtin_amdgcn_perm(a45, a01, 0x05040100u);
            out[1] = __builtin_amdgcn_perm(a45, a01, 0x07060302u);
            out[2] = __builtin_amdgcn_perm(b45, b01, 0x05040100u);
            out[3] = __builtin_amdgcn_perm(c45, c01, 0x05040100u);
        };
        gather(0, ev);
        gather(1, od);
        // S_i over the chunk: this lane's 8 bytes, then the 16 lanes of the row
        int s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s[i] = __builtin_amdgcn_sdot4(static_cast<int>(ev[i]), 0x01010101, 0, false);
            s[i] = __builtin_amdgcn_sdot4(static_cast<int>(od[i]), 0x01010101, s[i], false);
            s[i] += __builtin_amdgcn_mov_dpp(s[i], 0x128, 0xF, 0xF, false);
            s[i] += __builtin_amdgcn_mov_dpp(s[i], 0x124, 0xF, 0xF, false);
            s[i] += __builtin_amdgcn_mov_dpp(s[i], 0x4E, 0xF, 0xF, false);
            s[i] += __builtin_amdgcn_mov_dpp(s[i], 0xB1, 0xF, 0xF, false);
        }
        const int g = 4 * xl + part;
        if (xl < nxl && g < G) {
            uint8_t *const px = lds + static_cast<uint32_t>(g) * kI8ChunkX + (r16 >> 2) * 128u + (r16 & 3) * 4u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                *reinterpret_cast<uint32_t *>(px + i * 32) = ev[i];
                *reinterpret_cast<uint32_t *>(px + i * 32 + 16) = od[i];
            }
            if (r16 == 0) {
                // 2^(e - 151) as 2^a * 2^b, both normal: a = max(e - 151, -126)
                const int a = max(e - 151, -126), bx = e - 151 - a;
                const float pa = e == 255 ? __uint_as_float(0x7FC00000u) : __uint_as_float(static_cast<uint32_t>(127 + a) << 23);
                const float pb = __uint_as_float(static_cast<uint32_t>(127 + bx) << 23);
                *reinterpret_cast<uint4 *>(lds + soff + static_cast<uint32_t>(g) * kI8ChunkRec) =
                    make_uint4((static_cast<uint32_t>(s[0]) & 0xFFFFu) | (static_cast<uint32_t>(s[1]) << 16),
                               (static_cast<uint32_t>(s[2]) & 0xFFFFu) | (static_cast<uint32_t>(s[3]) << 16),
                               __float_as_uint(pa), __float_as_uint(pb));
            }
        }
    };
    static_for<kXRegs>([&](auto ii) __attribute__((always_inline)) {
        constexpr int i = decltype(ii)::value;
        convert(xr[i], wave + i * NW);
    });
    for (int xl = wave + kXRegs * NW; xl < nxl; xl += NW) {  // K > 16384 only (waits for the ring too)
        const uint4 r = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, lane * 16u, static_cast<uint32_t>(xl) * 1024u, 0));
        convert(r, xl);
    }
    lds_barrier<63>();

    // A operand of lane (i, p): piece min(i, 3) of part p, the even block (+16: the odd block)
    const uint32_t xlane = static_cast<uint32_t>(part) * 128u + static_cast<uint32_t>(min(r16, 3)) * 32u;
    float acc = 0.0f;
    const int steps = npos > wave ? (npos - wave + NW - 1) / NW : 0;
    auto consume = [&](const NStage &s) __attribute__((always_inline)) {
        const bool live = pt < ntiles;
        const int g = pg;
        const uint8_t *xa = lds + static_cast<uint32_t>(g) * kI8ChunkX + xlane;
        const int32x4 a1 = *reinterpret_cast<const int32x4 *>(xa);
        const int32x4 a2 = *reinterpret_cast<const int32x4 *>(xa + 16);
        const uint4 rec = *reinterpret_cast<const uint4 *>(lds + soff + static_cast<uint32_t>(g) * kI8ChunkRec);
        int32x4 blo, bhi;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            blo[q] = static_cast<int>((__builtin_rotateleft32(s.w[q], 4) ^ 0x88888888u) & 0xF0F0F0F0u);
            bhi[q] = static_cast<int>((s.w[q] ^ 0x88888888u) & 0xF0F0F0F0u);
        }
        int32x4 c = {0, 0, 0, 0};
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, blo, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, bhi, c, 0, 0, 0);
        const int zc = 128 - static_cast<int>(((s.am[1] >> (4 * (r16 & 7))) & 15u) << 4);  // 16 (8 - z)
        const int d0 = c[0] + zc * (static_cast<int>(rec.x << 16) >> 16);
        const int d1 = c[1] + zc * (static_cast<int>(rec.x) >> 16);
        const int d2 = c[2] + zc * (static_cast<int>(rec.y << 16) >> 16);
        const int d3 = c[3] + zc * (static_cast<int>(rec.y) >> 16);
        const int lo = d0 + (d1 << 8);
        const float f = __builtin_fmaf(static_cast<float>(d2), 65536.0f,
                                       __builtin_fmaf(static_cast<float>(d3), 0.0078125f, static_cast<float>(lo)));
        float v = __fmul_rn(f, f16_to_f32(static_cast<uint16_t>(s.am[0])));
        v = __fmul_rn(__fmul_rn(v, __uint_as_float(rec.z)), __uint_as_float(rec.w));
        asm volatile("" : "+v"(v));  // the product rounds on its own: no fused multiply-add into acc
        acc = __fadd_rn(acc, v);
        const int tile = pt;
        pg += NW;
        while (pg >= G) {
            pg -= G;
            ++pt;
        }
        if (live && pt != tile) {
            if (lane < 16) accs[(tile * NW + wave) * 16 + lane] = acc;
            acc = 0.0f;
        }
    };
    static_for<E>([&](auto i) __attribute__((always_inline)) {
        if (decltype(i)::value < steps) consume(pre[decltype(i)::value]);
        __builtin_amdgcn_sched_barrier(0);
    });
    for (int k = E; k < steps; k += D) {
        static_for<D>([&](auto ii) __attribute__((always_inline)) {
            constexpr int i = decltype(ii)::value;
            consume(st[i]);
            load(st[i]);
            __builtin_amdgcn_sched_barrier(0);
        });
    }
    lds_barrier<63>();

    for (int i = tid; i < ntiles * 16; i += 64 * NW) {
        const int row = (t0 + (i >> 4)) * 16 + (i & 15);
        if (row >= rlo && row < rhi) {
            const float *pa = accs + (i >> 4) * NW * 16 + (i & 15);
            float v = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < NW; ++w2) v += pa[w2 * 16];
            if (b.y_bf16) static_cast<uint16_t *>(P.y)[row] = f32_to_bf16_rne(v);
            else static_cast<float *>(P.y)[row] = v;
        }
    }
}

// ---- canonical <-> planes ------------------------------------------------------------------
// One thread per 16-byte unit of the codes planes / per (tile, group, row) of the metadata.
__global__ void to_planes_kernel(const uint32_t *codes, const uint16_t *scales, const uint32_t *zeros, int64_t n,
                                 int64_t k, uint8_t *pc, uint16_t *ps, uint8_t *pz) {
    const int64_t G = k / kGroup, GP = (G + 7) / 8 * 8, ZW = (G + 7) / 8, T = (n + 15) / 16;
    const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (u >= T * G * 64) return;
    const int64_t chunk = u >> 6, l = u & 63;
    const int64_t t = chunk / G, g = chunk % G, p = l >> 4, r = l & 15, row = t * 16 + r;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < n) v = *reinterpret_cast<const uint4 *>(codes + row * (k / 8) + 16 * g + 4 * p);
    *reinterpret_cast<uint4 *>(pc + u * 16) = v;
    if (p == 0) {
        ps[chunk * 16 + r] = row < n ? scales[row * GP + g] : 0;
        if ((r & 1) == 0) {
            uint32_t z0 = row < n ? (zeros[row * ZW + g / 8] >> (4 * (g & 7))) & 15u : 0u;
            uint32_t z1 = row + 1 < n ? (zeros[(row + 1) * ZW + g / 8] >> (4 * (g & 7))) & 15u : 0u;
            pz[chunk * 8 + (r >> 1)] = static_cast<uint8_t>(z0 | (z1 << 4));
        }
    }
}

// One thread per 16-byte unit of the canonical codes; the thread holding a row's first unit
// of a group-of-8 also writes that row's scale slots (pad slots 0) and zero word.
__global__ void from_planes_kernel(const uint8_t *pc, const uint16_t *ps, const uint8_t *pz, int64_t n, int64_t k,
                                   uint32_t *codes, uint16_t *scales, uint32_t *zeros) {
    const int64_t G = k / kGroup, GP = (G + 7) / 8 * 8, ZW = (G + 7) / 8;
    const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // over n * (k / 32)
    const int64_t units = k / 32;
    if (u >= n * units) return;
    const int64_t row = u / units, c = u % units, g = c / 4, p = c % 4, t = row / 16, r = row % 16;
    const int64_t chunk = t * G + g;
    *reinterpret_cast<uint4 *>(codes + row * (k / 8) + 4 * c) =
        *reinterpret_cast<const uint4 *>(pc + (chunk * 64 + p * 16 + r) * 16);
    if (p == 0 && (g & 7) == 0) {
        uint32_t zw = 0;
        for (int64_t j = 0; j < 8; ++j) {
            const int64_t gg = g + j;
            uint16_t sv = 0;
            if (gg < G) {
                const int64_t ch = t * G + gg;
                sv = ps[ch * 16 + r];
                zw |= ((static_cast<uint32_t>(pz[ch * 8 + (r >> 1)]) >> (4 * (r & 1))) & 15u) << (4 * j);
            }
            scales[row * GP + gg] = sv;
        }
        zeros[row * ZW + g / 8] = zw;
    }
}

// NF4 canonical (codes u32 [N, K/8], absmax f32 [N, K/block]) <-> NF4 planes; nbpc =
// max(1, 128 / block) absmax values per chunk and row.  One thread per 16-byte piece.
__global__ void nf4_to_planes_kernel(const uint32_t *codes, const float *absmax, int64_t n, int64_t k,
                                     int64_t block, uint8_t *pc, float *pa) {
    const int64_t G = k / kGroup, T = (n + 15) / 16, NB = (k + block - 1) / block;
    const int64_t nbpc = block >= kGroup ? 1 : kGroup / block;
    const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (u >= T * G * 64) return;
    const int64_t chunk = u >> 6, l = u & 63;
    const int64_t t = chunk / G, g = chunk % G, p = l >> 4, r = l & 15, row = t * 16 + r;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < n) {
        const uint32_t *src = codes + row * (k / 8) + 16 * g + p;
        v = make_uint4(src[0], src[4], src[8], src[12]);
    }
    *reinterpret_cast<uint4 *>(pc + u * 16) = v;
    if (p == 0) {
        for (int64_t j = 0; j < nbpc; ++j) {
            const int64_t blk = block >= kGroup ? (g * kGroup) / block : g * nbpc + j;
            pa[(chunk * 16 + r) * nbpc + j] = row < n ? absmax[row * NB + blk] : 0.0f;
        }
    }
}

__global__ void nf4_from_planes_kernel(const uint8_t *pc, const float *pa, int64_t n, int64_t k, int64_t block,
                                       uint32_t *codes, float *absmax) {
    const int64_t G = k / kGroup, NB = (k + block - 1) / block;
    const int64_t nbpc = block >= kGroup ? 1 : kGroup / block;
    const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // over n * G * 4
    if (u >= n * G * 4) return;
    const int64_t row = u / (G * 4), c = u % (G * 4), g = c / 4, p = c % 4, t = row / 16, r = row % 16;
    const int64_t chunk = t * G + g;
    const uint4 v = *reinterpret_cast<const uint4 *>(pc + (chunk * 64 + p * 16 + r) * 16);
    uint32_t *dst = codes + row * (k / 8) + 16 * g + p;
    dst[0] = v.x;
    dst[4] = v.y;
    dst[8] = v.z;
    dst[12] = v.w;
    if (p == 0) {
        for (int64_t j = 0; j < nbpc; ++j) {
            const int64_t blk = block >= kGroup ? (g * kGroup) / block : g * nbpc + j;
            // a block longer than a chunk is written by the thread of its first chunk
            if (block < kGroup || (g * kGroup) % block == 0) absmax[row * NB + blk] = pa[(chunk * 16 + r) * nbpc + j];
        }
    }
}

// GGUF Q4_0 planes (codes u8 [N, K/2], 64-byte chunks of four 16-byte parts; d f16 [N, GP])
// <-> Q4_0 GEMV planes: chunk (t, g) holds at byte 16 * (16 p + r) part p of chunk g of row
// 16 t + r, and d [T][G][16][4] the four blocks' d of row 16 t + r.  One thread per piece.
__global__ void q40_to_planes_kernel(const uint8_t *codes, const uint16_t *scales, int64_t n, int64_t k, uint8_t *pc,
                                     uint16_t *pd) {
    const int64_t G = k / kGroup, T = (n + 15) / 16, GP = (k / 32 + 7) / 8 * 8;
    const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (u >= T * G * 64) return;
    const int64_t chunk = u >> 6, l = u & 63;
    const int64_t t = chunk / G, g = chunk % G, p = l >> 4, r = l & 15, row = t * 16 + r;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < n) v = *reinterpret_cast<const uint4 *>(codes + row * (k / 2) + g * 64 + 16 * p);
    *reinterpret_cast<uint4 *>(pc + u * 16) = v;
    if (p == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) pd[(chunk * 16 + r) * 4 + j] = row < n ? scales[row * GP + 4 * g + j] : 0;
    }
}

__global__ void q40_from_planes_kernel(const uint8_t *pc, const uint16_t *pd, int64_t n, int64_t k, uint8_t *codes,
                                       uint16_t *scales) {
    const int64_t G = k / kGroup, GP = (k / 32 + 7) / 8 * 8;
    const int64_t u = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;  // over n * G * 4
    if (u >= n * G * 4) return;
    const int64_t row = u / (G * 4), c = u % (G * 4), g = c / 4, p = c % 4, t = row / 16, r = row % 16;
    const int64_t chunk = t * G + g;
    *reinterpret_cast<uint4 *>(codes + row * (k / 2) + g * 64 + 16 * p) =
        *reinterpret_cast<const uint4 *>(pc + (chunk * 64 + p * 16 + r) * 16);
    if (p == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) scales[row * GP + 4 * g + j] = pd[(chunk * 16 + r) * 4 + j];
        if (g == G - 1)
            for (int64_t j = 4 * G; j < GP; ++j) scales[row * GP + j] = 0;  // pad slots
    }
}

// ---- host ----------------------------------------------------------------------------------
int cu_count() {
    static std::mutex mu;
    static std::map<int, int> cache;
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> g(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 0;
    check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    cache[dev] = cus;
    return cus;
}

// Workgroups per problem in proportion to its code bytes (largest remainders; at least one per
// problem, at most one per 8-row unit): every CU then streams about the same number of bytes.
std::vector<int> workgroups_per_problem(const std::vector<int64_t> &bytes, const std::vector<int64_t> &units,
                                        int W) {
    const size_t n = bytes.size();
    std::vector<int> wgs(n, 1);
    int64_t total = 0;
    for (int64_t v : bytes) total += v;
    int used = 0;
    std::vector<std::pair<double, size_t>> rem;
    for (size_t i = 0; i < n; ++i) {
        const double share = static_cast<double>(W) * static_cast<double>(bytes[i]) / static_cast<double>(total);
        wgs[i] = std::max(1, static_cast<int>(share));
        wgs[i] = static_cast<int>(std::min<int64_t>(wgs[i], units[i]));
        used += wgs[i];
        rem.push_back({share - static_cast<double>(wgs[i]), i});
    }
    std::sort(rem.begin(), rem.end(), [](const auto &a, const auto &c) { return a.first > c.first; });
    for (size_t j = 0; used < W && j < rem.size(); ++j) {
        const size_t i = rem[j].second;
        if (wgs[i] < units[i]) {
            ++wgs[i];
            ++used;
        }
    }
    return wgs;
}

template <int NW, int D, int MR>
void launch_planes(const PBatch<CFH_MAX_BATCH> &b, int64_t grid, int64_t lds, hipStream_t st) {
    static std::mutex mu;
    static std::map<int, bool> attr_set;  // per device
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    {
        std::lock_guard<std::mutex> g(mu);
        if (!attr_set[dev]) {
            check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(&planes_kernel<NW, D, MR>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax),
                      "hipFuncSetAttribute");
            attr_set[dev] = true;
        }
    }
    planes_kernel<NW, D, MR>
        <<<dim3(static_cast<unsigned>(grid)), dim3(64 * NW), static_cast<size_t>(lds), st>>>(b);
    check_launch("planes_kernel");
}


template <int NW, int D, int MR>
void launch_planes_xr(const PBatch<CFH_MAX_BATCH> &b, int64_t grid, int64_t lds, hipStream_t st) {
    static std::mutex mu;
    static std::map<int, bool> attr_set;  // per device
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    {
        std::lock_guard<std::mutex> g(mu);
        if (!attr_set[dev]) {
            check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(&planes_xr_kernel<NW, D, MR>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax),
                      "hipFuncSetAttribute");
            attr_set[dev] = true;
        }
    }
    planes_xr_kernel<NW, D, MR>
        <<<dim3(static_cast<unsigned>(grid)), dim3(64 * NW), static_cast<size_t>(lds), st>>>(b);
    check_launch("planes_xr_kernel");
}

// workgroups per problem such that bytes[i] / wgs[i] + fixed[i] is about equal over the problems
// (fixed: work every workgroup of problem i does whatever its share), at least lo[i] (>= 1) and
// at most units[i] each and W in total: the level T solves sum max(lo[i], bytes[i] / (T -
// fixed[i])) = W, the shares are rounded by largest remainder.  All fixed equal to 0 and lo to 1
// is workgroups_per_problem's split.
std::vector<int> workgroups_balanced(const std::vector<int64_t> &bytes, const std::vector<int64_t> &fixed,
                                     const std::vector<int64_t> &lo_wgs, const std::vector<int64_t> &units, int W) {
    const size_t n = bytes.size();
    double fmax = 0.0;
    for (int64_t f : fixed) fmax = std::max(fmax, static_cast<double>(f));
    auto share = [&](size_t i, double T) {
        return std::max(static_cast<double>(lo_wgs[i]), static_cast<double>(bytes[i]) / (T - static_cast<double>(fixed[i])));
    };
    auto total = [&](double T) {
        double t = 0.0;
        for (size_t i = 0; i < n; ++i) t += share(i, T);
        return t;
    };
    double lo = fmax, hi = fmax + 1.0;
    for (int it = 0; it < 200 && total(hi) > W; ++it) hi = fmax + 2.0 * (hi - fmax);
    for (int it = 0; it < 100; ++it) {
        const double mid = 0.5 * (lo + hi);
        if (mid <= fmax || total(mid) > W) lo = mid;
        else hi = mid;
    }
    std::vector<int> wgs(n, 1);
    int used = 0;
    std::vector<std::pair<double, size_t>> rem;
    for (size_t i = 0; i < n; ++i) {
        const double sh = share(i, hi);
        wgs[i] = static_cast<int>(std::min<int64_t>(std::max<int64_t>(lo_wgs[i], static_cast<int64_t>(sh)), units[i]));
        used += wgs[i];
        rem.push_back({sh - static_cast<double>(wgs[i]), i});
    }
    std::sort(rem.begin(), rem.end(), [](const auto &a, const auto &c) { return a.first > c.first; });
    for (size_t j = 0; used < W && j < rem.size(); ++j) {
        const size_t i = rem[j].second;
        if (wgs[i] < units[i]) {
            ++wgs[i];
            ++used;
        }
    }
    return wgs;
}

// Whole tiles per workgroup, the largest number of 1 KB positions a workgroup streams made as
// small as W workgroups allow: the least L with sum ceil(tiles[i] / floor(L / groups[i])) <= W,
// then the remaining workgroups one at a time to the problem whose workgroups stream most.  (A
// workgroup's time follows the positions it touches, and a tile split between two workgroups
// costs each of them a full position per chunk.)
std::vector<int> workgroups_whole_tiles(const std::vector<int64_t> &tiles, const std::vector<int64_t> &groups, int W) {
    const size_t n = tiles.size();
    auto need = [&](int64_t L) {
        int64_t t = 0;
        for (size_t i = 0; i < n; ++i) {
            const int64_t per = L / groups[i];
            if (per < 1) return int64_t(W) + 1;
            t += (tiles[i] + per - 1) / per;
        }
        return t;
    };
    int64_t lo = 1, hi = 1;
    for (size_t i = 0; i < n; ++i) hi = std::max(hi, tiles[i] * groups[i]);
    while (lo < hi) {  // least L with need(L) <= W (need(hi) = count <= W)
        const int64_t mid = (lo + hi) / 2;
        if (need(mid) <= W) hi = mid;
        else lo = mid + 1;
    }
    std::vector<int> wgs(n);
    int used = 0;
    for (size_t i = 0; i < n; ++i) {
        const int64_t per = lo / groups[i];
        wgs[i] = static_cast<int>((tiles[i] + per - 1) / per);
        used += wgs[i];
    }
    while (used < W) {
        size_t best = n;
        int64_t most = -1;
        for (size_t i = 0; i < n; ++i) {
            if (wgs[i] >= tiles[i]) continue;
            const int64_t pos = (tiles[i] + wgs[i] - 1) / wgs[i] * groups[i];
            if (pos > most) {
                most = pos;
                best = i;
            }
        }
        if (best == n) break;
        ++wgs[best];
        ++used;
    }
    return wgs;
}

// tiles one workgroup of a problem spans at most, for `units` 8-row units over `wgs` workgroups:
// U = ceil(units / wgs) units starting at an odd unit touch floor(U / 2) + 1 tiles
int64_t planes_tiles(int64_t units, int64_t wgs) { return (units + wgs - 1) / wgs / 2 + 1; }

// M = 2..16 on planes_xr_kernel: every problem's planes streamed once, each problem's share of
// the CUs by its bytes; a problem whose workgroups would span more tiles than their slots fit in
// LDS gets more workgroups.
template <int NW, int D, int MR>
void planes_xr_launch(const cfh_w4a16_problem_t *problems, int32_t count, int64_t m, int32_t y_dtype,
                      hipStream_t st) {
    const int64_t slot_bytes = int64_t(NW) * 64 * MR;          // one tile's slots
    const int64_t x_bytes = int64_t(NW) * (int64_t(MR) * 256 + 64);  // the waves' x areas
    const int64_t max_tiles = (kLdsMax / kWgPerCu - x_bytes) / slot_bytes;
    static_assert((kLdsMax / kWgPerCu - NW * (MR * 256 + 64)) / (NW * 64 * MR) >= 2, "room for two tiles' slots");
    std::vector<int64_t> bytes, units;
    for (int i = 0; i < count; ++i) {
        const cfh_w4a16_problem_t &q = problems[i];
        require(m * q.k * 2 < (int64_t(1) << 31), "x of one problem must stay below 2 GiB");
        bytes.push_back(((q.n + 15) / 16) * (q.k / kGroup) * 1024);
        units.push_back((q.n + 7) / 8);
    }
    // every workgroup converts its problem's whole x (M x K values) besides streaming its share of
    // the planes: the split equalises bytes / wgs + c M K over the problems (c: the cost of
    // converting one value in bytes streamed), each problem taking at least the workgroups that
    // keep its tiles' slots within LDS
    std::vector<int64_t> xcost, lo_wgs;
    const double c = MR == 16 ? CFH_PLANES_XR_XCOST16 : CFH_PLANES_XR_XCOST;
    for (int i = 0; i < count; ++i) {
        xcost.push_back(static_cast<int64_t>(c * static_cast<double>(m * problems[i].k)));
        lo_wgs.push_back(std::max<int64_t>(1, (units[static_cast<size_t>(i)] + 2 * (max_tiles - 1) - 1) / (2 * (max_tiles - 1))));
    }
    std::vector<int> wgs = workgroups_balanced(bytes, xcost, lo_wgs, units, cu_count() * kWgPerCu);
    PBatch<CFH_MAX_BATCH> b{};
    int64_t lds = 0, grid = 0;
    for (int j = 0; j < count; ++j) {
        const cfh_w4a16_problem_t &q = problems[j];
        int64_t wj = wgs[static_cast<size_t>(j)];
        const int64_t u = units[static_cast<size_t>(j)];
        if (planes_tiles(u, wj) > max_tiles) wj = std::min<int64_t>(u, (u + 2 * (max_tiles - 1) - 1) / (2 * (max_tiles - 1)));
        require(planes_tiles(u, wj) <= max_tiles, "a problem's rows exceed the GEMV planes kernel's LDS");
        PProblem &P = b.p[j];
        P.codes = reinterpret_cast<const uint8_t *>(q.codes);
        P.scales = q.scales_f16;
        P.zeros = reinterpret_cast<const uint8_t *>(q.zeros);
        P.x = q.x;
        P.y = q.y;
        P.n = static_cast<int32_t>(q.n);
        P.G = static_cast<int32_t>(q.k / kGroup);
        P.units = static_cast<int32_t>(u);
        P.wg0 = static_cast<int32_t>(grid);
        P.wgs = static_cast<int32_t>(wj);
        P.m = static_cast<int32_t>(m);
        require(wj * u < (int64_t(1) << 31), "too many rows for one launch");
        grid += wj;
        lds = std::max<int64_t>(lds, planes_tiles(u, wj) * slot_bytes + x_bytes);
    }
    b.count = count;
    b.y_bf16 = y_dtype == CFH_DTYPE_BF16;
    launch_planes_xr<NW, D, MR>(b, grid, std::max<int64_t>(lds, kLdsFloor), st);
}

void planes_xr_batched(const cfh_w4a16_problem_t *problems, int32_t count, int64_t m, int32_t y_dtype,
                       hipStream_t st) {
    if (m <= 4) planes_xr_launch<CFH_PLANES_XR_WAVES, CFH_PLANES_XR_DEPTH, 4>(problems, count, m, y_dtype, st);
    else if (m <= 8) planes_xr_launch<CFH_PLANES_XR_WAVES, CFH_PLANES_XR_DEPTH, 8>(problems, count, m, y_dtype, st);
    else planes_xr_launch<CFH_PLANES_XR_WAVES16, CFH_PLANES_XR_DEPTH16, 16>(problems, count, m, y_dtype, st);
}

// LDS bytes of one problem: its x rows, their post factors and the partials of the tiles one
// of its workgroups spans (at most ceil(units / wgs) / 2 + 2)
int64_t planes_lds(int mr, int nw, const PProblem &P) {
    const int64_t tiles = (P.units + P.wgs - 1) / P.wgs / 2 + 2;
    const int64_t rs = mr == 1 ? x_row_stride<1>(static_cast<uint32_t>(P.G)) : x_row_stride<4>(static_cast<uint32_t>(P.G));
    return (rs * P.m + 15) / 16 * 16 + (P.G * mr * 4 + 15) / 16 * 16 + tiles * nw * 64 * mr;
}

template <int NBPC, int KIND = kKindNf4>
void launch_planes_m1(const NBatch &b, int64_t grid, int64_t lds, hipStream_t st);
void launch_planes_i8(const NBatch &b, int64_t grid, int64_t lds, hipStream_t st);

// M = 1: one row of x per problem (planes_i8_kernel, planes_m1_kernel); M = 2..4: up to 4 rows
// staged in LDS (planes_kernel, 16 waves), measured faster there than planes_xr_kernel, which
// serves M = 5..16 and every batch whose x does not fit LDS.
void planes_batched(const cfh_w4a16_problem_t *problems, int32_t count, int64_t m, int32_t y_dtype,
                    hipStream_t st) {
    require(count >= 1 && count <= CFH_MAX_BATCH, "count must be in 1..8");
    require(problems != nullptr, "problems must not be NULL");
    require(m >= 1 && m <= 16, "the GEMV planes kernels take M = 1..16");
    require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
    const int mr = m == 1 ? 1 : 4;
    const int W = cu_count() * kWgPerCu;
    for (int i = 0; i < count; ++i) {
        const cfh_w4a16_problem_t &q = problems[i];
        require(q.group == kGroup, "GEMV planes hold INT4 groups of 128");
        require(q.n >= 1 && q.k >= kGroup && q.k % kGroup == 0, "GEMV planes need n >= 1 and k % 128 == 0");
        require(q.x && q.codes && q.scales_f16 && q.zeros && q.y, "x, planes and y must not be NULL");
        require(aligned(q.x, 16) && aligned(q.codes, 16) && aligned(q.scales_f16, 4) && aligned(q.y, 4),
                "x and codes planes must be 16-byte aligned, scales and y 4-byte aligned");
        require(((q.n + 15) / 16) * (q.k / kGroup) * 1024 < (int64_t(1) << 31),
                "GEMV planes of one matrix must stay below 2 GiB");
    }
    if (m > CFH_PLANES_XR_FROM - 1) {
        planes_xr_batched(problems, count, m, y_dtype, st);
        return;
    }
    if (m == 1 && CFH_PLANES_M1_GENERIC) {
        std::vector<int64_t> bytes, units, tiles, groups;
        for (int i = 0; i < count; ++i) {
            bytes.push_back(((problems[i].n + 15) / 16) * (problems[i].k / kGroup) * 1024);
            units.push_back((problems[i].n + 7) / 8);
            tiles.push_back((problems[i].n + 15) / 16);
            groups.push_back(problems[i].k / kGroup);
        }
        std::vector<int> wgs;
        std::vector<int> ush(static_cast<size_t>(count), 0);
        if (CFH_PLANES_M1_SPLIT == 1) {
            wgs = workgroups_whole_tiles(tiles, groups, W);
            for (int i = 0; i < count; ++i) {
                units[static_cast<size_t>(i)] = tiles[static_cast<size_t>(i)];
                ush[static_cast<size_t>(i)] = 1;
            }
        } else {
            wgs = workgroups_per_problem(bytes, units, W);
        }
        NBatch nb{};
        int64_t need_max = 0, need_i8 = 0, ngrid = 0;
        for (int j = 0; j < count; ++j) {
            const cfh_w4a16_problem_t &q = problems[j];
            NProblem &P = nb.p[j];
            P.codes = reinterpret_cast<const uint8_t *>(q.codes);
            P.absmax = reinterpret_cast<const float *>(q.scales_f16);  // f16 scale planes
            P.zeros = reinterpret_cast<const uint8_t *>(q.zeros);
            P.x = q.x;
            P.y = q.y;
            P.n = static_cast<int32_t>(q.n);
            P.G = static_cast<int32_t>(q.k / kGroup);
            P.units = static_cast<int32_t>(units[static_cast<size_t>(j)]);
            P.wg0 = static_cast<int32_t>(ngrid);
            P.wgs = wgs[static_cast<size_t>(j)];
            P.ush = ush[static_cast<size_t>(j)];
            require(static_cast<int64_t>(P.wgs) * P.units < (int64_t(1) << 31), "too many rows for one launch");
            ngrid += P.wgs;
            const int64_t tiles = (P.units + P.wgs - 1) / P.wgs / (2 - P.ush) + 2;
            need_max = std::max<int64_t>(need_max, int64_t(P.G) * 256 + (int64_t(P.G) * 4 + 15) / 16 * 16 +
                                                       tiles * kWaves * 64);
            need_i8 = std::max<int64_t>(need_i8, int64_t(P.G) * (kI8ChunkX + kI8ChunkRec) + tiles * kWaves * 64);
        }
        nb.count = count;
        nb.y_bf16 = y_dtype == CFH_DTYPE_BF16;
        if (need_i8 <= kLdsMax / kWgPerCu) {  // the integer form wherever its x pieces fit LDS
            launch_planes_i8(nb, ngrid, std::max<int64_t>(need_i8, kLdsFloor), st);
            return;
        }
        require(need_max <= kLdsMax / kWgPerCu, "a problem of the batch exceeds the GEMV planes kernel's LDS (m * k too "
                                                "large or too many rows per workgroup)");
        launch_planes_m1<1, kKindInt4>(nb, ngrid, std::max<int64_t>(need_max, kLdsFloor), st);
        return;
    }
    // M = 1 (the generic build) and M = 2..4: x of every problem staged in LDS, one problem per
    // matrix; M = 2..4 takes planes_xr_kernel where x does not fit
    PBatch<CFH_MAX_BATCH> b{};
    int64_t lds_max = 0, grid = 0;
    std::vector<int64_t> bytes, units;
    for (int i = 0; i < count; ++i) {
        bytes.push_back(((problems[i].n + 15) / 16) * (problems[i].k / kGroup) * 1024);
        units.push_back((problems[i].n + 7) / 8);
    }
    const std::vector<int> wgs = workgroups_per_problem(bytes, units, W);
    for (int j = 0; j < count; ++j) {
        const cfh_w4a16_problem_t &q = problems[j];
        PProblem &P = b.p[j];
        P.codes = reinterpret_cast<const uint8_t *>(q.codes);
        P.scales = q.scales_f16;
        P.zeros = reinterpret_cast<const uint8_t *>(q.zeros);
        P.x = q.x;
        P.y = q.y;
        P.n = static_cast<int32_t>(q.n);
        P.G = static_cast<int32_t>(q.k / kGroup);
        P.units = static_cast<int32_t>(units[static_cast<size_t>(j)]);
        P.wg0 = static_cast<int32_t>(grid);
        P.wgs = wgs[static_cast<size_t>(j)];
        P.m = static_cast<int32_t>(m);
        require(static_cast<int64_t>(P.wgs) * P.units < (int64_t(1) << 31), "too many rows for one launch");
        grid += P.wgs;
        lds_max = std::max<int64_t>(lds_max, planes_lds(mr, kWaves, P));
    }
    b.count = count;
    b.y_bf16 = y_dtype == CFH_DTYPE_BF16;
    if (lds_max > kLdsMax / kWgPerCu && m >= 2) {
        planes_xr_batched(problems, count, m, y_dtype, st);
        return;
    }
    require(lds_max <= kLdsMax / kWgPerCu, "a problem of the batch exceeds the GEMV planes kernel's LDS (m * k too large "
                                "or too many rows per workgroup)");
    const int64_t req = std::max<int64_t>(lds_max, kLdsFloor);
    if (mr == 1) launch_planes<kWaves, kDepth, 1>(b, grid, req, st);
    else launch_planes<kWaves, kDepth, 4>(b, grid, req, st);
}

template <int NBPC, int KIND>
void launch_planes_m1(const NBatch &b, int64_t grid, int64_t lds, hipStream_t st) {
    constexpr int D = KIND == kKindInt4 ? kI4Depth : kNf4Depth;
    static std::mutex mu;
    static std::map<int, bool> attr_set;  // per device
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    {
        std::lock_guard<std::mutex> g(mu);
        if (!attr_set[dev]) {
            check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(&planes_m1_kernel<kWaves, D, NBPC, KIND>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax),
                      "hipFuncSetAttribute");
            attr_set[dev] = true;
        }
    }
    planes_m1_kernel<kWaves, D, NBPC, KIND>
        <<<dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), static_cast<size_t>(lds), st>>>(b);
    check_launch("planes_m1_kernel");
}

void launch_planes_i8(const NBatch &b, int64_t grid, int64_t lds, hipStream_t st) {
    static std::mutex mu;
    static std::map<int, bool> attr_set;  // per device
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    {
        std::lock_guard<std::mutex> g(mu);
        if (!attr_set[dev]) {
            check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(&planes_i8_kernel<kWaves, kI4Depth>),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax),
                      "hipFuncSetAttribute");
            attr_set[dev] = true;
        }
    }
    planes_i8_kernel<kWaves, kI4Depth>
        <<<dim3(static_cast<unsigned>(grid)), dim3(64 * kWaves), static_cast<size_t>(lds), st>>>(b);
    check_launch("planes_i8_kernel");
}

bool nf4_block_ok(int64_t block) { return block >= 32 && block <= (int64_t(1) << 20) && (block & (block - 1)) == 0; }

// NF4 decode GEMV (M = 1) over NF4 planes: one workgroup of 16 waves per CU, problems sharing
// the CUs in proportion to their bytes (as the INT4 planes kernel).
void nf4_planes_batched(const cfh_nf4_problem_t *problems, int32_t count, int64_t m, int32_t y_dtype,
                        hipStream_t st) {
    require(count >= 1 && count <= CFH_MAX_BATCH, "count must be in 1..8");
    require(problems != nullptr, "problems must not be NULL");
    require(m == 1, "the NF4 planes kernel takes M = 1");
    require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
    const int64_t block = problems[0].block;
    require(nf4_block_ok(block), "NF4 block must be a power of two >= 32");
    const int64_t nbpc = block >= kGroup ? 1 : kGroup / block;
    const int W = cu_count();
    std::vector<int64_t> bytes, units;
    for (int i = 0; i < count; ++i) {
        const cfh_nf4_problem_t &q = problems[i];
        require(q.block == block, "every problem of a batch must have the same NF4 block");
        require(q.n >= 1 && q.k >= kGroup && q.k % kGroup == 0, "NF4 planes need n >= 1 and k % 128 == 0");
        require(q.x && q.codes && q.absmax && q.y, "x, planes and y must not be NULL");
        require(aligned(q.x, 16) && aligned(q.codes, 16) && aligned(q.absmax, 4 * nbpc) && aligned(q.y, 4),
                "x and codes planes must be 16-byte aligned, absmax planes aligned to their per-row values, "
                "y 4-byte aligned");
        require(((q.n + 15) / 16) * (q.k / kGroup) * 1024 < (int64_t(1) << 31),
                "NF4 planes of one matrix must stay below 2 GiB");
        bytes.push_back(((q.n + 15) / 16) * (q.k / kGroup) * (1024 + 64 * nbpc));
        units.push_back((q.n + 7) / 8);
    }
    const std::vector<int> wgs = workgroups_per_problem(bytes, units, W);
    NBatch b{};
    int64_t lds_max = 0, grid = 0;
    for (int j = 0; j < count; ++j) {
        const cfh_nf4_problem_t &q = problems[j];
        NProblem &P = b.p[j];
        P.codes = reinterpret_cast<const uint8_t *>(q.codes);
        P.absmax = q.absmax;
        P.x = q.x;
        P.y = q.y;
        P.n = static_cast<int32_t>(q.n);
        P.G = static_cast<int32_t>(q.k / kGroup);
        P.units = static_cast<int32_t>(units[j]);
        P.wg0 = static_cast<int32_t>(grid);
        P.wgs = wgs[j];
        require(static_cast<int64_t>(P.wgs) * P.units < (int64_t(1) << 31), "too many rows for one launch");
        grid += P.wgs;
        const int64_t tiles = (P.units + P.wgs - 1) / P.wgs / 2 + 2;
        const int64_t need = kNf4LutBytes + int64_t(P.G) * 256 + (int64_t(P.G) * 4 + 15) / 16 * 16 + tiles * kWaves * 64;
        lds_max = std::max<int64_t>(lds_max, need);
    }
    b.count = count;
    b.y_bf16 = y_dtype == CFH_DTYPE_BF16;
    require(lds_max <= kLdsMax, "a problem of the batch exceeds the NF4 planes kernel's LDS (k too large)");
    // at least kLdsFloor, so that one workgroup per CU holds for small k too
    const int64_t req = std::max<int64_t>(lds_max, kLdsFloor);
    if (nbpc == 1) launch_planes_m1<1>(b, grid, req, st);
    else if (nbpc == 2) launch_planes_m1<2>(b, grid, req, st);
    else launch_planes_m1<4>(b, grid, req, st);
}

// GGUF Q4_0 decode GEMV (M = 1) over Q4_0 GEMV planes: the NF4 planes kernel with the exact
// (q - 8) decode and one f16 d per block of 32.
void q40_planes_batched(const cfh_gguf_problem_t *problems, int32_t count, int64_t m, int32_t y_dtype,
                        hipStream_t st) {
    require(count >= 1 && count <= CFH_MAX_BATCH, "count must be in 1..8");
    require(problems != nullptr, "problems must not be NULL");
    require(m == 1, "the Q4_0 planes kernel takes M = 1");
    require(y_dtype == CFH_DTYPE_F32 || y_dtype == CFH_DTYPE_BF16, "y_dtype must be F32 or BF16");
    const int W = cu_count();
    std::vector<int64_t> bytes, units;
    for (int i = 0; i < count; ++i) {
        const cfh_gguf_problem_t &q = problems[i];
        require(q.n >= 1 && q.k >= kGroup && q.k % kGroup == 0, "Q4_0 planes need n >= 1 and k % 128 == 0");
        require(q.x && q.codes && q.scales_f16 && q.y, "x, planes and y must not be NULL");
        require(aligned(q.x, 16) && aligned(q.codes, 16) && aligned(q.scales_f16, 8) && aligned(q.y, 4),
                "x and codes planes must be 16-byte aligned, d planes 8-byte aligned, y 4-byte aligned");
        require(((q.n + 15) / 16) * (q.k / kGroup) * 1024 < (int64_t(1) << 31),
                "Q4_0 planes of one matrix must stay below 2 GiB");
        bytes.push_back(((q.n + 15) / 16) * (q.k / kGroup) * (1024 + 128));
        units.push_back((q.n + 7) / 8);
    }
    const std::vector<int> wgs = workgroups_per_problem(bytes, units, W);
    NBatch b{};
    int64_t lds_max = 0, grid = 0;
    for (int j = 0; j < count; ++j) {
        const cfh_gguf_problem_t &q = problems[j];
        NProblem &P = b.p[j];
        P.codes = reinterpret_cast<const uint8_t *>(q.codes);
        P.absmax = reinterpret_cast<const float *>(q.scales_f16);  // the d planes (8 bytes per row and chunk)
        P.x = q.x;
        P.y = q.y;
        P.n = static_cast<int32_t>(q.n);
        P.G = static_cast<int32_t>(q.k / kGroup);
        P.units = static_cast<int32_t>(units[j]);
        P.wg0 = static_cast<int32_t>(grid);
        P.wgs = wgs[j];
        require(static_cast<int64_t>(P.wgs) * P.units < (int64_t(1) << 31), "too many rows for one launch");
        grid += P.wgs;
        const int64_t tiles = (P.units + P.wgs - 1) / P.wgs / 2 + 2;
        const int64_t need = int64_t(P.G) * 256 + (int64_t(P.G) * 4 + 15) / 16 * 16 + tiles * kWaves * 64;
        lds_max = std::max<int64_t>(lds_max, need);
    }
    b.count = count;
    b.y_bf16 = y_dtype == CFH_DTYPE_BF16;
    require(lds_max <= kLdsMax, "a problem of the batch exceeds the Q4_0 planes kernel's LDS (k too large)");
    launch_planes_m1<4, kKindQ40>(b, grid, std::max<int64_t>(lds_max, kLdsFloor), st);
}

void q40_planes_checks(const void *codes, const void *scales, int64_t rows, int64_t k, const void *pc, const void *pd) {
    require(rows >= 0 && k >= 0 && k % kGroup == 0, "rows >= 0 and k % 128 == 0 are required");
    if (rows > 0 && k > 0) {
        require(codes && scales && pc && pd, "buffers must not be NULL");
        require(aligned(codes, 16) && aligned(pc, 16), "codes and codes planes must be 16-byte aligned");
        require(aligned(scales, 2) && aligned(pd, 8), "d must be 2-byte and d planes 8-byte aligned");
        require(((rows + 15) / 16) * (k / kGroup) * 1024 < (int64_t(1) << 31), "planes must stay below 2 GiB");
    }
}

void nf4_planes_checks(const void *codes, const void *absmax, int64_t rows, int64_t k, int64_t block, const void *pc,
                       const void *pa) {
    require(nf4_block_ok(block), "NF4 block must be a power of two >= 32");
    require(rows >= 0 && k >= 0 && k % kGroup == 0, "rows >= 0 and k % 128 == 0 are required");
    if (rows > 0 && k > 0) {
        require(codes && absmax && pc && pa, "buffers must not be NULL");
        require(aligned(codes, 4) && aligned(pc, 16), "codes must be 4-byte and codes planes 16-byte aligned");
        require(aligned(absmax, 4) && aligned(pa, 4), "absmax arrays must be 4-byte aligned");
        require(((rows + 15) / 16) * (k / kGroup) * 1024 < (int64_t(1) << 31), "planes must stay below 2 GiB");
    }
}

void planes_checks(const void *codes, const void *scales, const void *zeros, int64_t rows, int64_t k,
                   int64_t group, const void *pc, const void *ps, const void *pz) {
    require(group == kGroup, "GEMV planes hold INT4 groups of 128");
    require(rows >= 0 && k >= 0 && k % kGroup == 0, "rows >= 0 and k % 128 == 0 are required");
    if (rows > 0 && k > 0) {
        require(codes && scales && zeros && pc && ps && pz, "buffers must not be NULL");
        require(aligned(codes, 16) && aligned(pc, 16), "codes and codes planes must be 16-byte aligned");
        require(aligned(scales, 2) && aligned(ps, 2) && aligned(zeros, 4), "scales and zeros must be aligned");
        require(((rows + 15) / 16) * (k / kGroup) * 1024 < (int64_t(1) << 31), "planes must stay below 2 GiB");
    }
}

}  // namespace
}  // namespace cfh

using namespace cfh;

extern "C" {

int32_t castforge_hip_int4g_to_planes(const uint32_t *codes, const uint16_t *scales_f16, const uint32_t *zeros,
                                      int64_t rows, int64_t k, int64_t group, void *planes_codes,
                                      uint16_t *planes_scales, uint8_t *planes_zeros, void *stream,
                                      char **out_error) {
    return guarded(out_error, [&] {
        planes_checks(codes, scales_f16, zeros, rows, k, group, planes_codes, planes_scales, planes_zeros);
        const int64_t units = ((rows + 15) / 16) * (k / kGroup) * 64;
        if (units == 0) return;
        to_planes_kernel<<<dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0,
                           static_cast<hipStream_t>(stream)>>>(codes, scales_f16, zeros, rows, k,
                                                               static_cast<uint8_t *>(planes_codes), planes_scales,
                                                               planes_zeros);
        check_launch("to_planes_kernel");
    });
}

int32_t castforge_hip_int4g_from_planes(const void *planes_codes, const uint16_t *planes_scales,
                                        const uint8_t *planes_zeros, int64_t rows, int64_t k, int64_t group,
                                        uint32_t *codes, uint16_t *scales_f16, uint32_t *zeros, void *stream,
                                        char **out_error) {
    return guarded(out_error, [&] {
        planes_checks(codes, scales_f16, zeros, rows, k, group, planes_codes, planes_scales, planes_zeros);
        const int64_t units = rows * (k / 32);
        if (units == 0) return;
        from_planes_kernel<<<dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0,
                             static_cast<hipStream_t>(stream)>>>(static_cast<const uint8_t *>(planes_codes),
                                                                 planes_scales, planes_zeros, rows, k, codes,
                                                                 scales_f16, zeros);
        check_launch("from_planes_kernel");
    });
}

int32_t castforge_hip_gemv_w4a16_planes_batched(const cfh_w4a16_problem_t *problems, int32_t count, int64_t m,
                                                int32_t y_dtype, void *stream, char **out_error) {
    return guarded(out_error, [&] { planes_batched(problems, count, m, y_dtype, static_cast<hipStream_t>(stream)); });
}

int32_t castforge_hip_nf4_to_planes(const uint32_t *codes, const float *absmax, int64_t rows, int64_t k,
                                    int64_t block, void *planes_codes, float *planes_absmax, void *stream,
                                    char **out_error) {
    return guarded(out_error, [&] {
        nf4_planes_checks(codes, absmax, rows, k, block, planes_codes, planes_absmax);
        const int64_t units = ((rows + 15) / 16) * (k / kGroup) * 64;
        if (units == 0) return;
        nf4_to_planes_kernel<<<dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0,
                               static_cast<hipStream_t>(stream)>>>(codes, absmax, rows, k, block,
                                                                   static_cast<uint8_t *>(planes_codes), planes_absmax);
        check_launch("nf4_to_planes_kernel");
    });
}

int32_t castforge_hip_nf4_from_planes(const void *planes_codes, const float *planes_absmax, int64_t rows, int64_t k,
                                      int64_t block, uint32_t *codes, float *absmax, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        nf4_planes_checks(codes, absmax, rows, k, block, planes_codes, planes_absmax);
        const int64_t units = rows * (k / kGroup) * 4;
        if (units == 0) return;
        nf4_from_planes_kernel<<<dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0,
                                 static_cast<hipStream_t>(stream)>>>(static_cast<const uint8_t *>(planes_codes),
                                                                     planes_absmax, rows, k, block, codes, absmax);
        check_launch("nf4_from_planes_kernel");
    });
}

int32_t castforge_hip_gemv_nf4_planes_batched(const cfh_nf4_problem_t *problems, int32_t count, int64_t m,
                                              int32_t y_dtype, void *stream, char **out_error) {
    return guarded(out_error, [&] { nf4_planes_batched(problems, count, m, y_dtype, static_cast<hipStream_t>(stream)); });
}

int32_t castforge_hip_gguf_q4_0_to_gemv_planes(const void *codes, const uint16_t *scales_f16, int64_t rows, int64_t k,
                                              void *planes_codes, uint16_t *planes_d, void *stream, char **out_error) {
    return guarded(out_error, [&] {
        q40_planes_checks(codes, scales_f16, rows, k, planes_codes, planes_d);
        const int64_t units = ((rows + 15) / 16) * (k / kGroup) * 64;
        if (units == 0) return;
        q40_to_planes_kernel<<<dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0,
                               static_cast<hipStream_t>(stream)>>>(static_cast<const uint8_t *>(codes), scales_f16, rows,
                                                                   k, static_cast<uint8_t *>(planes_codes), planes_d);
        check_launch("q40_to_planes_kernel");
    });
}

int32_t castforge_hip_gguf_q4_0_from_gemv_planes(const void *planes_codes, const uint16_t *planes_d, int64_t rows,
                                                int64_t k, void *codes, uint16_t *scales_f16, void *stream,
                                                char **out_error) {
    return guarded(out_error, [&] {
        q40_planes_checks(codes, scales_f16, rows, k, planes_codes, planes_d);
        const int64_t units = rows * (k / kGroup) * 4;
        if (units == 0) return;
        q40_from_planes_kernel<<<dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0,
                                 static_cast<hipStream_t>(stream)>>>(static_cast<const uint8_t *>(planes_codes), planes_d,
                                                                     rows, k, static_cast<uint8_t *>(codes), scales_f16);
        check_launch("q40_from_planes_kernel");
    });
}

int32_t castforge_hip_gemv_gguf_q4_0_planes_batched(const cfh_gguf_problem_t *problems, int32_t count, int64_t m,
                                                   int32_t y_dtype, void *stream, char **out_error) {
    return guarded(out_error, [&] { q40_planes_batched(problems, count, m, y_dtype, static_cast<hipStream_t>(stream)); });
}

}  // extern "C"
