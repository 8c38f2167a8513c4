// NF4 dequant-fused GEMM on one bf16 MFMA pair per product, for every M > 16 (gfx950).
//
// Y[m, n] = sum_k x[m, k] * f32(T[q[n, k]] * absmax[n, k / block]): the evaluation of
// `castforge.fused_qmatmul` over NF4 weights (codegen/eval.rs:1145-1179 with eval_matmul_2d,
// eval.rs:1465-1507; the NF4 table and dequant of schemes.rs), x bf16 [M, K], codes u32 [N, K/8]
// (8 nibbles per word, k = 8 w + j at bits 4 j), absmax f32 [N, K / block].
//
// Numerics.  The table value T[q] is fed to v_mfma_f32_32x32x16_bf16 as two bf16 terms,
// T_hi = RNE(T) and T_lo = RNE(T - T_hi), which carry 16 significant bits of the f32 table value
// (|T - T_hi - T_lo| <= 2^-17 |T|); x enters as the bf16 it is, so every product is exact.  Each
// 64-wide K chunk sums x * (T_hi + T_lo) into a fresh f32 partial, and one fma per accumulator
// adds absmax * partial to the total (the block a power of two >= 64: a chunk lies in one
// absmax block).  Against the evaluator's sum of x * RN(T absmax) each product differs by at
// most ~2^-16 of itself, so an output differs by at most ~2^-16 sum |x w| plus the summation
// order -- less than the evaluator's own worst-case f32 summation error (K 2^-24 sum |x w|) for
// K >= 256, and far inside the 1e-2 / 1e-3 bound on the BASELINE inputs and on cancelling rows.
//
// Design (one workgroup of 8 waves per CU):
//   * the workgroup owns one tile of 32 J rows (m) and NB blocks of 32 columns (n) over the
//     whole K; its waves are NB n blocks x KP = 8 / NB parts of K (NB = 4 or 2, chosen per
//     problem so that every workgroup carries a similar number of weights: W_gate's 128 x 4096
//     and W_down's 64 x 11008); the parts' totals are added in part order at the end (LDS), so
//     results do not depend on timing;
//   * x goes global -> LDS once per workgroup: each K part streams its 32 J x 64 chunks through
//     a ring of three LDS stages (buffer loads to LDS, issued by the part's NB waves), read by
//     those NB waves; 16-byte pieces are XOR-swizzled by row so the fragment reads hit distinct
//     banks;
//   * W is the MFMA B operand (a lane's 16 accumulators share one n, so one absmax scales
//     them); per 64-wide chunk, lane (r = lane % 32, h = lane / 32) loads 16 code bytes of row r
//     (k = 64 c + 32 h .. + 31) into registers; MFMA step s takes code word s and the x piece of
//     k = 64 c + 32 h + 8 s .. + 7, so A and B agree on k;
//   * decode: a 64 KB LDS table maps a code byte (two k) to its T_hi pair and its T_lo pair, the
//     bf16 operand words themselves, read straight into the MFMA operand registers; 32 copies put
//     lane l's reads on bank l % 32 (+32 for the T_lo half), and one v_perm builds each address
//     (byte of the code word in address bits 8..15, the copy in bits 2..6): 4 VALU and 8 LDS
//     reads per 8 weights.
#include <algorithm>
#include <cstring>

#include "../../include/castforge_hip.h"
#include "cfh_common.hpp"

namespace cfh {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kCopies = 32;
constexpr int kLutBytes = 256 * kCopies * 8;  // 64 KB
constexpr int kMaxP = CFH_MAX_BATCH;
constexpr int kStages = 3;  // x ring per K part (L2-resident activations)
constexpr int kWDepth = 6;  // code / absmax register ring (HBM weights: the longer lead)
// LDS: the table, then KP rings of kStages stages of 32 J rows x 128 bytes
constexpr int lds_bytes(int J, int kp) { return kLutBytes + kp * kStages * 4 * J * 1024; }

// the NF4 table (QLoRA's 16 quantiles of N(0, 1), scaled to [-1, 1]), as the f32 values the
// evaluator uses; kNf4Tc is the same table for indices known at compile time
#define CFH_NF4_TABLE                                                                               \
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,                    \
        -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,                 \
        0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,   \
        0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f
__constant__ float kNf4T[16] = {CFH_NF4_TABLE};
constexpr float kNf4Tc[16] = {CFH_NF4_TABLE};

struct Nf4Prob {
    const uint16_t *x;
    const uint32_t *codes;
    const float *absmax;
    void *y;
    int n, k, block;
    int kparts;    // K parts (2 or 4); 8 / kparts blocks of 32 columns per workgroup
    int tiles_n;   // workgroups along n: ceil(n / (32 * 8 / kparts))
    int wg_begin;  // first workgroup of the problem
};

struct Nf4Batch {
    Nf4Prob p[kMaxP];
    int count, m, tiles_m, y_bf16;
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), 0x00020000);
}

template <int J>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void nf4_mfma_kernel(Nf4Batch b) {
    extern __shared__ __align__(16) uint8_t lds[];  // the decode table, the x rings; at the end the K-part totals
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = uni(tid >> 6);
    const int r = lane & 31, h = lane >> 5;

    int pi = 0;
#pragma unroll
    for (int i = 1; i < kMaxP; ++i)
        if (i < b.count && static_cast<int>(blockIdx.x) >= b.p[i].wg_begin) pi = i;
    const Nf4Prob &P = b.p[pi];
    const int N = P.n, K = P.k, M = b.m;
    const int kparts = P.kparts, nblk = kWaves / kparts;
    const int local = static_cast<int>(blockIdx.x) - P.wg_begin;
    const int tile_n = local % P.tiles_n, tile_m = local / P.tiles_n;
    const int nb = wave % nblk, kp = wave / nblk;
    const int n0 = (tile_n * nblk + nb) * 32;  // this wave's 32 columns
    const int m0 = tile_m * 32 * J;

    // decode table: row v (256 bytes) holds, for each copy c = 0..31, the bf16 pair
    // (T_hi[v & 15], T_hi[v >> 4]) at 4 c and (T_lo[v & 15], T_lo[v >> 4]) at 128 + 4 c.  Thread t
    // writes rows v = t / 32 + 16 i (i = 0..15), copy t % 32: v >> 4 = i is known at compile time
    // and v & 15 = t / 32 is one table load per thread.
    {
        const float t0 = kNf4T[tid >> 5];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float t1 = kNf4Tc[i];
            const uint32_t hi = f32x2_to_bf16x2_rne(t0, t1);
            const float h0 = __uint_as_float(hi << 16), h1 = __uint_as_float(hi & 0xffff0000u);
            const uint32_t lo = f32x2_to_bf16x2_rne(t0 - h0, t1 - h1);
            uint8_t *row = lds + ((tid >> 5) + 16 * i) * 256 + 4 * (tid & 31);
            *reinterpret_cast<uint32_t *>(row) = hi;
            *reinterpret_cast<uint32_t *>(row + 128) = lo;
        }
    }

    // sources: rows past N / M read zero (a zero code decodes to T[0] = -1, but such columns are
    // never stored, and their absmax reads 0)
    const int nvalid = uni(max(0, min(32, N - n0)));
    const int mvalid = uni(max(0, min(32 * J, M - m0)));
    const uint32_t row_bytes = static_cast<uint32_t>(K) / 2;
    const int NB = K / P.block;  // absmax blocks per row
    const rsrc_t rc = make_rsrc(reinterpret_cast<const uint8_t *>(P.codes) + static_cast<int64_t>(n0) * row_bytes,
                                static_cast<uint32_t>(nvalid) * row_bytes);
    const rsrc_t ra = make_rsrc(P.absmax + static_cast<int64_t>(n0) * NB, static_cast<uint32_t>(nvalid * NB) * 4);
    const rsrc_t rx = make_rsrc(P.x + static_cast<int64_t>(m0) * K, static_cast<uint32_t>(mvalid) * K * 2);
    const int chunks = K / 64;
    // every part gets the same number of chunks, +-1; parts with fewer run one empty step, so
    // all waves pass the same barriers
    const int c_lo = uni(kp * chunks / kparts), c_hi = uni((kp + 1) * chunks / kparts);
    const int steps = uni((chunks + kparts - 1) / kparts);
    const int cshift = __builtin_ctz(static_cast<uint32_t>(P.block / 64));  // chunk -> absmax block

    // this part's x ring: stage i at ring + i * kStage; row q, 16-byte piece p at 128 q + 16 (p ^ ((q >> 1) & 7))
    // A stage is 4 J loads of 1 KB (64 lanes x 16 bytes), issued by the part's nblk waves: 2 J each
    // with nblk = 2, J each with nblk = 4.  The loop below is instantiated for both counts (a
    // wave-uniform choice), so every load carries data and the steps have no branches.
    constexpr int kStage = 4 * J * 1024;
    uint8_t *const ring = lds + kLutBytes + kp * kStages * kStage;
    // a load t covers stage pieces 64 t .. 64 t + 63: lane -> row 8 t + lane / 8, physical piece lane % 8
    const int lrow = lane >> 3, lpiece = lane & 7;
    // the lane's offset does not depend on the chunk (the compiler keeps it out of the loop); the
    // chunk adds a wave-uniform byte offset (soffset)
    auto issue = [&](auto RC, uint8_t *__restrict__ dst, int c) __attribute__((always_inline)) {
        constexpr int R = decltype(RC)::value;
#pragma unroll
        for (int t0 = 0; t0 < R; ++t0) {
            const int t = nb * R + t0;
            const int row = 8 * t + lrow;
            const int q = lpiece ^ ((row >> 1) & 7);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rx, (__attribute__((address_space(3))) void *)(dst + t * 1024), 16,
                static_cast<uint32_t>((row * K + q * 8) * 2), c * 128, 0, 0);
        }
    };
    struct WRegs {
        uint4 w;
        float am;
    };
    const uint32_t w_off = static_cast<uint32_t>(r) * row_bytes + h * 16, a_off = static_cast<uint32_t>(r * NB) * 4;
    auto wload = [&](WRegs &R, int c) {
        R.w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rc, w_off, c * 32, 0));
        R.am = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ra, a_off, (c >> cshift) * 4, 0));
    };

    floatx16 tot[J];
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) tot[j][e] = 0.0f;
    const uint32_t c4 = static_cast<uint32_t>(r) << 2;

    // A chunk's B operands, decoded from its code words through the table (T_hi and T_lo words
    // for the 4 MFMA steps), and the absmax that scales its partial.
    struct Dec {
        uint4 hi[4], lo[4];
        float am;
    };
    auto decode = [&](const uint8_t *__restrict__ lut, const WRegs &R, float am, Dec &D) __attribute__((always_inline)) {
        const uint32_t wv[4] = {R.w.x, R.w.y, R.w.z, R.w.w};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // address 256 * byte q of the word + 4 * copy: byte 1 <- byte q of w, byte 0 <- c4
                const uint32_t a = __builtin_amdgcn_perm(wv[s], c4, 0x0c0c0000u | ((0x04u + q) << 8));
                hi[q] = *reinterpret_cast<const uint32_t *>(lut + a);
                lo[q] = *reinterpret_cast<const uint32_t *>(lut + a + 128);
            }
            D.hi[s] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            D.lo[s] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        }
        D.am = am;
    };
    // the chunk's MFMAs into a fresh partial
    auto mma = [&](const uint8_t *__restrict__ cur, const Dec &D, floatx16 (&part)[J]) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bf16x8_t bh = __builtin_bit_cast(bf16x8_t, D.hi[s]);
            const bf16x8_t bl = __builtin_bit_cast(bf16x8_t, D.lo[s]);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int row = 32 * j + r, piece = 4 * h + s;
                const bf16x8_t a = *reinterpret_cast<const bf16x8_t *>(cur + row * 128 + 16 * (piece ^ ((row >> 1) & 7)));
                if (s == 0) {
                    const floatx16 zero = {};
                    part[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bh, zero, 0, 0, 0);
                } else {
                    part[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bh, part[j], 0, 0, 0);
                }
                part[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bl, part[j], 0, 0, 0);
            }
        }
    };
    auto fold = [&](float am, const floatx16 (&part)[J]) {
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) tot[j][e] = __builtin_fmaf(am, part[j][e], tot[j][e]);
    };

    __syncthreads();  // decode table written (the rings are written only by LDS-DMA below)
    auto main_loop = [&](auto RC) __attribute__((always_inline)) {
        constexpr int kPer = decltype(RC)::value + 2;  // a wave's loads per chunk: its x loads, codes, absmax
        // Rings: step t consumes chunk c_lo + t, its x from stage t % kStages and its codes / absmax
        // from register slot t % kWDepth.  Step t issues the x of chunk t + kStages - 1 (L2) and then
        // the codes of chunk t + kWDepth - 1 (HBM: the deeper lead).  vmcnt counts in issue order, so
        // chunk t's x has landed once at most the 2 code loads issued right after it and step t - 1's
        // kPer loads are outstanding -- and chunk t's codes, issued kWDepth - 1 steps back, are in
        // too.  Step t: wait for that, barrier (every wave's x pieces of chunk t are in LDS, and no
        // wave still reads the stage of chunk t - 1), issue, consume.  Chunk indices past a part's end are clamped to
        // its last chunk (a reload that nothing consumes), so every step issues the same loads and
        // every wave passes the same barriers; a part with one chunk fewer skips its last consume.
        WRegs wr[kWDepth];
        auto chunk_of = [&](int t) { return min(c_lo + t, c_hi - 1); };
        // prologue, in the steady order: the codes of chunks 0 .. kWDepth - kStages - 1, then for the
        // pseudo-steps t = -(kStages - 1) .. -1 the x of chunk t + kStages - 1 and the codes of chunk
        // t + kWDepth - 1
        static_for<kWDepth - kStages>([&](auto I) { wload(wr[decltype(I)::value], chunk_of(decltype(I)::value)); });
        static_for<kStages - 1>([&](auto I) {
            constexpr int t = decltype(I)::value;
            issue(RC, ring + t * kStage, chunk_of(t));
            wload(wr[t + kWDepth - kStages], chunk_of(t + kWDepth - kStages));
        });
        // Step t runs chunk t's MFMAs from operands decoded in step t - 1 and, between them, folds
        // chunk t - 1's partial into the totals (VALU beside the MFMAs) and decodes chunk t + 1 (the
        // table and the code registers do not depend on the barrier).  A part with one chunk fewer
        // runs its last step on a repeat of its last chunk with absmax 0.
        Dec dec[2];
        floatx16 part[2][J];
    #pragma unroll
        for (int j = 0; j < J; ++j)
    #pragma unroll
            for (int e = 0; e < 16; ++e) part[1][j][e] = 0.0f;
        dec[1].am = 0.0f;  // step 0 folds this empty "chunk -1"
        auto am_of = [&](int t, const WRegs &R) { return c_lo + t < c_hi ? R.am : 0.0f; };
        // chunk 0's codes: issued before the two pseudo-steps' kPer + 2 loads each
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kPer + 4) & ~(15 << 8));
        decode(lds, wr[0], am_of(0, wr[0]), dec[0]);
        // One step's work.  The three LDS pointers are restrict-qualified parameters of this one
        // function: the compiler then knows that the table and fragment reads do not touch the
        // stage the step's buffer->LDS loads write, and need not wait for those loads.
        auto body = [&](const uint8_t *__restrict__ lut, const uint8_t *__restrict__ cur, uint8_t *__restrict__ nxt,
                        auto I, int t) __attribute__((always_inline)) {
            constexpr int i = decltype(I)::value;
            issue(RC, nxt, chunk_of(t + kStages - 1));
            wload(wr[(i + kWDepth - 1) % kWDepth], chunk_of(t + kWDepth - 1));
            mma(cur, dec[i & 1], part[i & 1]);
            fold(dec[(i + 1) & 1].am, part[(i + 1) & 1]);
            decode(lut, wr[(i + 1) % kWDepth], am_of(t + 1, wr[(i + 1) % kWDepth]), dec[(i + 1) & 1]);
        };
        auto step = [&](auto I, int t) {
            constexpr int i = decltype(I)::value;  // t modulo kWDepth (a multiple of kStages and of 2)
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(kPer + 2) & ~(15 << 8));
            // unconditional: the compiler's own wait tracking then sees every LDS read retired
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));
            __builtin_amdgcn_s_barrier();
            body(lds, ring + (i % kStages) * kStage, ring + ((i + kStages - 1) % kStages) * kStage, I, t);
        };
        static_assert(kWDepth % kStages == 0 && kWDepth % 2 == 0, "one unrolled group covers every ring");
        int t = 0;
        for (; t + kWDepth <= steps; t += kWDepth)
            static_for<kWDepth>([&](auto I) { step(I, t + decltype(I)::value); });
        static_for<kWDepth>([&](auto I) {
            if (t + decltype(I)::value < steps) step(I, t + decltype(I)::value);
        });
        // the last chunk's partial: part[(steps - 1) & 1], its absmax in dec[(steps - 1) & 1]
        if ((steps - 1) & 1) fold(dec[1].am, part[1]);
        else fold(dec[0].am, part[0]);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & ~(15 << 8));  // the trailing reloads
    };
    if (nblk == 2) main_loop(std::integral_constant<int, 2 * J>{});
    else main_loop(std::integral_constant<int, J>{});

    // K parts of one n block: parts 1.. write their totals over the table, part 0 adds them in
    // part order and stores
    __syncthreads();  // every wave is done with the table and the rings
    float *slot = reinterpret_cast<float *>(lds) + (wave * 64 + lane) * (16 * J);
    if (kp > 0) {
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) slot[j * 16 + e] = tot[j][e];
    }
    __syncthreads();
    if (kp != 0) return;
    for (int p = 1; p < kparts; ++p) {
        const float *o = reinterpret_cast<const float *>(lds) + ((wave + p * nblk) * 64 + lane) * (16 * J);
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) tot[j][e] += o[j * 16 + e];
    }
    const int n = n0 + r;
    if (n >= N) return;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int m = m0 + 32 * j + 8 * (e >> 2) + 4 * h + (e & 3);
            if (m < M) {
                const int64_t o = static_cast<int64_t>(m) * N + n;
                if (b.y_bf16) static_cast<uint16_t *>(P.y)[o] = f32_to_bf16_rne(tot[j][e]);
                else static_cast<float *>(P.y)[o] = tot[j][e];
            }
        }
}

template <int J>
void launch(const Nf4Batch &b, int grid, int lds, hipStream_t st) {
    static bool attr[64] = {};
    int dev = 0;
    require(hipGetDevice(&dev) == hipSuccess, "hipGetDevice failed");
    if (dev >= 0 && dev < 64 && !attr[dev]) {
        require(hipFuncSetAttribute(reinterpret_cast<const void *>(&nf4_mfma_kernel<J>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes(J, 4)) == hipSuccess,
                "hipFuncSetAttribute failed");
        attr[dev] = true;
    }
    nf4_mfma_kernel<J><<<grid, kThreads, lds, st>>>(b);
    check_launch("nf4_mfma");
}

}  // namespace

// True when a problem fits nf4_mfma_kernel: M >= 17, block a power of two >= 64 with k a
// multiple of block, 32-bit offsets over one workgroup's rows, 16-byte aligned x and codes.
bool nf4_mfma_ok(const uint16_t *x, int64_t m, int64_t n, int64_t k, int64_t block, const void *codes) {
    if (m < 17 || m > 0x7fffffff || n < 1 || n > 0x7fffffff) return false;
    if (block < 64 || (block & (block - 1)) != 0 || k < block || k % block != 0) return false;
    if (k < 4 * 64) return false;  // at least one 64-wide chunk per K part
    if (int64_t{64} * k * 2 >= (int64_t{1} << 31)) return false;
    return (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(codes) & 15) == 0;
}

// One launch over up to CFH_MAX_BATCH problems with the same M (each checked by nf4_mfma_ok).
void nf4_mfma_launch(const cfh_nf4_problem_t *ps, int count, int64_t m, int y_bf16, hipStream_t st) {
    require(count >= 1 && count <= kMaxP, "nf4_mfma_launch: 1..CFH_MAX_BATCH problems");
    const int J = m > 32 ? 2 : 1;
    Nf4Batch b{};
    b.m = static_cast<int>(m);
    b.tiles_m = static_cast<int>((m + 32 * J - 1) / (32 * J));
    b.y_bf16 = y_bf16;
    // longest K first: the workgroups that run longest are not left for the end
    int order[kMaxP];
    for (int i = 0; i < count; ++i) order[i] = i;
    std::stable_sort(order, order + count, [&](int a, int c) { return ps[a].k > ps[c].k; });
    int64_t wg = 0;
    for (int oi = 0; oi < count; ++oi) {
        const cfh_nf4_problem_t &q = ps[order[oi]];
        Nf4Prob &p = b.p[b.count++];
        p.x = q.x;
        p.codes = q.codes;
        p.absmax = q.absmax;
        p.y = q.y;
        p.n = static_cast<int>(q.n);
        p.k = static_cast<int>(q.k);
        p.block = static_cast<int>(q.block);
        // K parts: 2 (128 columns per workgroup) up to k = 6144, else 4 (64 columns): W_gate's
        // 128 x 4096 and W_down's 64 x 11008 workgroups then carry 0.5 M and 0.7 M weights
        const int kp = q.k > 6144 ? 4 : 2;
        p.kparts = kp;
        const int64_t cols = int64_t{32} * (kWaves / kp);
        p.tiles_n = static_cast<int>((q.n + cols - 1) / cols);
        p.wg_begin = static_cast<int>(wg);
        wg += int64_t{p.tiles_n} * b.tiles_m;
    }
    require(wg <= 0x7fffffff, "nf4_mfma_launch: too many workgroups");
    int kpmax = 2;
    for (int i = 0; i < b.count; ++i) kpmax = std::max(kpmax, b.p[i].kparts);
    if (J == 2) launch<2>(b, static_cast<int>(wg), lds_bytes(2, kpmax), st);
    else launch<1>(b, static_cast<int>(wg), lds_bytes(1, kpmax), st);
}

}  // namespace cfh
