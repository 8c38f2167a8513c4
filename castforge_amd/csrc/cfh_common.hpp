// Shared host/device helpers for the CastForge MI355X quantized-weight library.
//
// Host side: the C-ABI status convention of the reference FFI (ffi.rs:46-72, 198-215):
// return 0 on success, 1 on a reported error with a heap string in *out_error, 2 when an
// internal exception was caught; out-pointers are cleared on entry; no exception or abort
// ever crosses the ABI.
//
// Device side: exact scalar codecs (f16/bf16 RNE, OCP E4M3FN with the reference's quirk)
// and wave64 reductions used by every kernel.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>

#include <cstring>
#include <stdexcept>
#include <string>

namespace cfh {

// ----------------------------------------------------------------------------------------
// host: errors and status
// ----------------------------------------------------------------------------------------
struct UserError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

char *dup_string(const std::string &s);  // heap string freed by castforge_hip_free_string

inline void require(bool ok, const std::string &msg) {
    if (!ok) throw UserError(msg);
}

inline void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess)
        throw UserError(std::string(what) + ": " + hipGetErrorString(e));
}

// Launch-error check after every kernel launch (reports bad launch shapes, missing code
// objects, or an earlier asynchronous fault).
inline void check_launch(const char *kernel) { check_hip(hipGetLastError(), kernel); }

inline bool aligned(const void *p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Runs `body` and turns every outcome into the reference's status codes.
template <class F>
int32_t guarded(char **out_error, F &&body) {
    if (out_error) *out_error = nullptr;
    try {
        body();
        return 0;
    } catch (const UserError &e) {
        if (out_error) *out_error = dup_string(e.what());
        return 1;
    } catch (const std::exception &e) {
        if (out_error) *out_error = dup_string(std::string("internal error: ") + e.what());
        return 2;
    } catch (...) {
        if (out_error) *out_error = dup_string("internal error: unknown exception");
        return 2;
    }
}

// ----------------------------------------------------------------------------------------
// device: scalar codecs
// ----------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float v) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Two f32 -> packed bf16 (low half = a) with round-to-nearest-even: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_rne(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// IEEE RNE f32 -> f16 (hardware v_cvt_f16_f32 rounds to nearest even, keeps subnormals).
__device__ __forceinline__ uint16_t f32_to_f16_rne(float v) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// The value of lane (lane ^ D) of the wave.  D = 1, 2: DPP quad permutations; D = 4: DPP row
// shifts (lanes with bit 2 clear read lane + 4, the others lane - 4); D = 8: DPP row rotate by
// 8; D = 16, 32: ds_bpermute.  DPP moves run on the VALU, without the LDS permute unit.
template <int D>
__device__ __forceinline__ float lane_xor(float v) {
    const int x = __builtin_bit_cast(int, v);
    if constexpr (D == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));
    else if constexpr (D == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));
    else if constexpr (D == 4) {
        const int up = __builtin_amdgcn_mov_dpp(x, 0x104, 0xF, 0xF, false);  // row_shl:4, lane + 4
        const int dn = __builtin_amdgcn_mov_dpp(x, 0x114, 0xF, 0xF, false);  // row_shr:4, lane - 4
        return __builtin_bit_cast(float, (threadIdx.x & 4) ? dn : up);
    } else if constexpr (D == 8) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false));
    else return __shfl_xor(v, D);
}

// Sub-block that lane t holds when a Walsh-Hadamard block spans 2..16 lanes of sub-blocks:
// within each 16-lane DPP row, lane bits (l0, l1, l2, l3) hold sub-block bits
// (l0 ^ l2, l1 ^ l2, l2, l3).  The cross-lane stages pair sub-blocks that differ in bit 0, 1,
// 2, 3, and in this layout the partners are lane ^ 1, lane ^ 2 (quad permutations), lane ^ 7
// (the half-row mirror, DPP 0x141) and lane ^ 8 (row rotation by 8, DPP 0x128): one DPP read
// each.  An involution, the identity on bits above 3, and it maps aligned runs of 2, 4, 8 and
// 16 lanes onto aligned runs of sub-blocks.
__device__ __forceinline__ int hsub16(int t) { return t ^ (((t >> 2) & 1) * 3); }

// One cross-lane butterfly stage over N values per lane against lane ^ D: the lane with bit D
// clear holds position j and keeps x + y, its partner holds j + h and keeps x - y (x the lower
// lane's value, y the upper's), exactly the reference's buf[j] / buf[j + h] update.
template <int D, int N>
__device__ __forceinline__ void lane_butterfly(float (&v)[N]) {
    const bool lower = (threadIdx.x & D) == 0;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float p = lane_xor<D>(v[i]);
        v[i] = lower ? v[i] + p : p - v[i];
    }
}

// Cross-lane stages for partner distances 1, 2, 4, .. below `lanes` (lanes <= 64).
template <int N>
__device__ __forceinline__ void lane_butterflies(float (&v)[N], int lanes) {
    if (lanes > 1) lane_butterfly<1, N>(v);
    if (lanes > 2) lane_butterfly<2, N>(v);
    if (lanes > 4) lane_butterfly<4, N>(v);
    if (lanes > 8) lane_butterfly<8, N>(v);
    if (lanes > 16) lane_butterfly<16, N>(v);
    if (lanes > 32) lane_butterfly<32, N>(v);
}

// OCP E4M3FN encode, bit-exact with the reference codec (mutable_loads.rs:367-411):
// integer round-half-even with saturation to +-448 (0x7E/0xFE), NaN -> 0x7F, plus the 16
// inputs just below a power of two where the reference's floor(log2f(|v|)) rounds up and it
// returns code+1.  That set is the f32 exponent field e in [0x79, 0x86] with mantissa at or
// above a per-binade threshold.
__device__ __forceinline__ uint8_t f32_to_e4m3fn(float v) {
    uint32_t b = __float_as_uint(v);
    uint32_t s = (b >> 24) & 0x80u;
    uint32_t a = b & 0x7fffffffu;
    if (a > 0x7f800000u) return 0x7F;
    if (a >= 0x43e00000u) return static_cast<uint8_t>(s | 0x7Eu);
    uint32_t ef = a >> 23;
    uint32_t m = a & 0x7fffffu;
    uint32_t q;
    if (ef < 121u) {  // |v| < 2^-6: e4m3 subnormal, q = RNE(|v| * 2^9)
        uint32_t sig = ef ? (m | 0x800000u) : m;
        int32_t shift = 14 - (ef ? static_cast<int32_t>(ef) - 127 : -126);
        if (shift >= 32) return static_cast<uint8_t>(s);
        q = sig >> shift;
        uint32_t rem = sig & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return static_cast<uint8_t>(s | q);
    }
    q = m >> 20;
    uint32_t rem = m & 0xfffffu;
    uint32_t eb = ef - 120u;  // (ef - 127) + 7
    if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) {
        q++;
        if (q == 8u) { q = 0; eb++; }
    }
    if (eb > 15u || (eb == 15u && q >= 7u)) return static_cast<uint8_t>(s | 0x7Eu);
    uint32_t code = (eb << 3) | q;
    // reference log2 quirk: thresholds for ef = 0x79..0x86 (0 = none)
    if (ef >= 0x79u && ef <= 0x86u) {
        uint32_t i = ef - 0x79u;
        uint32_t thr = (i < 2u || (i >= 10u)) ? 0x7ffffeu : ((i < 4u || i == 8u || i == 9u) ? 0x7fffffu : 0u);
        if (thr != 0u && m >= thr) code += 1u;
    }
    return static_cast<uint8_t>(s | code);
}

__device__ __forceinline__ float e4m3fn_to_f32(uint8_t b) {
    uint32_t sgn = (b & 0x80u) ? 0x80000000u : 0u;
    uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
    if (e == 15u && m == 7u) return __uint_as_float(0x7fc00000u);
    if (e == 0u) return __uint_as_float(sgn) + (sgn ? -1.0f : 1.0f) * (static_cast<float>(m) * 0.001953125f);
    return __uint_as_float(sgn | ((e + 120u) << 23) | (m << 20));
}

// ----------------------------------------------------------------------------------------
// device: wave64 reductions (butterfly over xor lane masks, stays within `width` lanes)
// ----------------------------------------------------------------------------------------
template <int WIDTH>
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

template <int WIDTH>
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}

template <int WIDTH>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int WIDTH>
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v = max(v, static_cast<uint32_t>(__shfl_xor(v, o, 64)));
    return v;
}

template <int WIDTH>
__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
    return v;
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector-memory loads are
// outstanding and ignores the export and LDS/scalar counters.
constexpr int vmcnt_imm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Calls f(std::integral_constant<int, I>{}) for I = 0 .. N-1 with I a compile-time constant,
// so register arrays indexed by I never fall back to scratch memory.
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

}  // namespace cfh
