"""numpy front end of the CPU oracle (oracle/_build/libcf_oracle.so) — test infrastructure.

Builds the oracle with its Makefile when the library is missing (it is plain C, seconds).
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_float, c_int, c_int64, c_uint8, c_uint16, c_uint32, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "oracle" / "_build" / "libcf_oracle.so"

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-C", str(ROOT / "oracle"), "-s"], check=True)
        l = ctypes.CDLL(str(LIB))
        P, I64 = c_void_p, c_int64
        sig = {
            "orc_f32_to_bf16_trunc": (c_uint16, [c_float]),
            "orc_f32_to_f16_trunc": (c_uint16, [c_float]),
            "orc_f16_to_f32": (c_float, [c_uint16]),
            "orc_bf16_to_f32": (c_float, [c_uint16]),
            "orc_f32_to_bf16_rne": (c_uint16, [c_float]),
            "orc_f32_to_f16_rne": (c_uint16, [c_float]),
            "orc_f32_to_e4m3fn": (c_uint8, [c_float]),
            "orc_e4m3fn_to_f32": (c_float, [c_uint8]),
            "orc_f32_to_e4m3fn_int": (c_uint8, [c_float]),
            "orc_f32_to_e4m3fn_fast": (c_uint8, [c_float]),
            "orc_e4m3_crosscheck": (I64, [c_uint32, c_uint32, c_uint32, c_int, P]),
            "orc_int_bounds": (None, [c_int, P, P, P]),
            "orc_quantize_symmetric": (c_float, [P, I64, c_int, c_int, P]),
            "orc_scale_string": (None, [c_float, ctypes.c_char_p, c_int]),
            "orc_quantize_groupwise": (I64, [P, I64, c_int, I64, c_int, c_float, c_int, P, P, P]),
            "orc_quantize_fp8_grid": (None, [P, I64, c_int, c_int, I64, P]),
            "orc_quantize_int8_rows": (None, [P, I64, I64, c_int, c_int, P, P]),
            "orc_quantize_int4g": (None, [P, I64, I64, I64, P, P, P]),
            "orc_dequantize_int4g": (None, [P, P, P, I64, I64, I64, P]),
            "orc_nf4_code": (c_uint8, [c_float]),
            "orc_quantize_nf4": (None, [P, I64, I64, I64, P, P]),
            "orc_dequantize_nf4": (None, [P, P, I64, I64, I64, P]),
            "orc_quantize_fp8_rows": (None, [P, I64, I64, P, P]),
            "orc_quantize_fp8_rows_bf16": (None, [P, I64, I64, P, P]),
            "orc_matmul_2d": (None, [P, P, I64, I64, I64, c_int, P]),
            "orc_epilogue": (None, [P, I64, P, I64, P, I64, c_int]),
            "orc_gemm_w8a16": (None, [P, I64, I64, I64, P, P, P]),
            "orc_gemm_w4a16": (None, [P, I64, I64, I64, I64, P, P, P, P]),
            "orc_gemm_nf4": (None, [P, I64, I64, I64, I64, P, P, P]),
            "orc_gemm_fp8": (None, [P, P, I64, P, P, I64, I64, P]),
            "orc_now_seconds": (ctypes.c_double, []),
            "orc_mx_scale_exp_model": (c_int, [c_float]),
            "orc_quantize_int4g_awq": (None, [P, P, I64, I64, I64, P, P, P]),
            "orc_mx_scale_crosscheck": (I64, [c_uint32, c_uint32, P]),
            "orc_static_quantize": (None, [P, I64, c_float, c_int, P]),
            "orc_gguf_decode": (I64, [c_int, P, I64, P]),
            "orc_gguf_encode_q8_0": (I64, [P, I64, c_float, P]),
            "orc_rotate_hadamard": (I64, [P, I64, I64, I64]),
            "orc_smoothquant": (None, [P, I64, c_float, c_float, c_int, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def nf4_table() -> np.ndarray:
    return np.ctypeslib.as_array((ctypes.c_float * 16).in_dll(lib(), "ORC_NF4_TABLE")).copy()


# ------------------------------------------------------------------ quantizers ----
def quantize_symmetric(v: np.ndarray, bits: int = 8, round_mode: int = 0):
    v = np.ascontiguousarray(v, np.float32)
    q = np.zeros(v.shape, np.int8)
    s = lib().orc_quantize_symmetric(_p(v), v.size, bits, round_mode, _p(q))
    return q, np.float32(s)


def static_quantize(x: np.ndarray, scale: float, bits: int = 8) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().orc_static_quantize(_p(x), x.size, np.float32(scale), bits, _p(y))
    return y


def scale_string(scale: float) -> str:
    buf = ctypes.create_string_buffer(64)
    lib().orc_scale_string(scale, buf, 64)
    return buf.value.decode()


def quantize_int8_rows(w: np.ndarray, bits: int = 8, round_mode: int = 1):
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    q = np.zeros((n, k), np.int8)
    s = np.zeros(n, np.float32)
    lib().orc_quantize_int8_rows(_p(w), n, k, bits, round_mode, _p(q), _p(s))
    return q, s


def quantize_int4g(w: np.ndarray, group: int = 128):
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    g = (k + group - 1) // group
    codes = np.zeros((n, k // 8), np.uint32)
    scales = np.zeros((n, (g + 7) // 8 * 8), np.uint16)
    zeros = np.zeros((n, (g + 7) // 8), np.uint32)
    lib().orc_quantize_int4g(_p(w), n, k, group, _p(codes), _p(scales), _p(zeros))
    return codes, scales, zeros


def quantize_int4g_awq(w: np.ndarray, s: np.ndarray, group: int = 128):
    w = np.ascontiguousarray(w, np.float32)
    s = np.ascontiguousarray(s, np.float32)
    n, k = w.shape
    g = (k + group - 1) // group
    zw = (g + 7) // 8
    codes = np.zeros((n, k // 8), np.uint32)
    scales = np.zeros((n, zw * 8), np.uint16)
    zeros = np.zeros((n, zw), np.uint32)
    lib().orc_quantize_int4g_awq(_p(w), _p(s), n, k, group, _p(codes), _p(scales), _p(zeros))
    return codes, scales, zeros


def dequantize_int4g(codes, scales, zeros, n, k, group):
    out = np.zeros((n, k), np.float32)
    lib().orc_dequantize_int4g(_p(codes), _p(scales), _p(zeros), n, k, group, _p(out))
    return out


def quantize_nf4(w: np.ndarray, block: int = 64):
    w = np.ascontiguousarray(w, np.float32)
    n, k = w.shape
    nb = (k + block - 1) // block
    codes = np.zeros((n, k // 8), np.uint32)
    absmax = np.zeros((n, nb), np.float32)
    lib().orc_quantize_nf4(_p(w), n, k, block, _p(codes), _p(absmax))
    return codes, absmax


def dequantize_nf4(codes, absmax, n, k, block):
    out = np.zeros((n, k), np.float32)
    lib().orc_dequantize_nf4(_p(codes), _p(absmax), n, k, block, _p(out))
    return out


def quantize_fp8_rows(v: np.ndarray):
    """v float32 [R, C] or bfloat16 bits (uint16) [R, C]."""
    v = np.ascontiguousarray(v)
    r, c = v.shape
    codes = np.zeros((r, c), np.uint8)
    scales = np.zeros(r, np.float32)
    if v.dtype == np.uint16:
        lib().orc_quantize_fp8_rows_bf16(_p(v), r, c, _p(codes), _p(scales))
    else:
        v = np.ascontiguousarray(v, np.float32)
        lib().orc_quantize_fp8_rows(_p(v), r, c, _p(codes), _p(scales))
    return codes, scales


def quantize_groupwise(v: np.ndarray, bits=4, group_size=32, awq_salient=True, salient_ratio=0.01,
                       round_mode=0):
    v = np.ascontiguousarray(v, np.float32).ravel()
    deq = np.zeros_like(v)
    gs = max(group_size, 2)
    scales = np.zeros((v.size + gs - 1) // gs, np.float32)
    thr = np.zeros(1, np.float32)
    cnt = lib().orc_quantize_groupwise(_p(v), v.size, bits, group_size, int(awq_salient),
                                       salient_ratio, round_mode, _p(deq), _p(scales), _p(thr))
    return deq, scales, int(cnt), float(thr[0])


def quantize_fp8_grid(v: np.ndarray, e5m2=False, mxfp8=True, block_size=32):
    v = np.ascontiguousarray(v, np.float32).ravel()
    deq = np.zeros_like(v)
    lib().orc_quantize_fp8_grid(_p(v), v.size, int(e5m2), int(mxfp8), block_size, _p(deq))
    return deq


# ---------------------------------------------------------------------- GGUF ----
GGML = {"F32": 0, "F16": 1, "Q4_0": 2, "Q8_0": 8, "BF16": 30}


def gguf_decode(ggml_type: int, raw: np.ndarray, num_elems: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.zeros(max(num_elems, 1), np.float32)
    used = lib().orc_gguf_decode(ggml_type, _p(raw), num_elems, _p(out))
    assert 0 <= used <= raw.size, (used, raw.size)
    return out[:num_elems]


def gguf_encode_q8_0(codes: np.ndarray, scale: float) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.int8).reshape(-1)
    out = np.zeros((max(codes.size, 1) + 31) // 32 * 34, np.uint8)
    n = lib().orc_gguf_encode_q8_0(_p(codes) if codes.size else 0, codes.size, np.float32(scale), _p(out))
    assert n == out.size
    return out


# ------------------------------------------------------------ outlier suppression ----
def rotate_hadamard(w: np.ndarray, block_size: int):
    """(rotated copy of a [k, n] array, the resolved block b or -1)."""
    w = np.array(w, np.float32, order="C", copy=True)
    k, n = w.shape
    b = lib().orc_rotate_hadamard(_p(w), k, n, block_size)
    return w, b


def smoothquant(w: np.ndarray, act_max: float, alpha: float = 0.5, bits: int = 8):
    """(fake-quantized copy, smoothing scale s, quantizer step e)."""
    w = np.array(w, np.float32, order="C", copy=True)
    sc = np.zeros(2, np.float32)
    lib().orc_smoothquant(_p(w), w.size, np.float32(act_max), np.float32(alpha), bits, _p(sc))
    return w, sc[0], sc[1]


# ---------------------------------------------------------------------- GEMMs ----
def matmul_2d(a: np.ndarray, b: np.ndarray, packed_rhs: bool) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    n = b.shape[0] if packed_rhs else b.shape[1]
    out = np.zeros((m, n), np.float32)
    lib().orc_matmul_2d(_p(a), _p(b), m, n, k, int(packed_rhs), _p(out))
    return out


def dot_general_flat(a: np.ndarray, b: np.ndarray, batch: int, k: int, rhs_contract_last: bool) -> np.ndarray:
    """eval_dot_general (eval.rs:1509-1604) past its 2-D case: both operands read flat, m and n
    from their element counts, lhs as [batch, m, k], rhs as [batch, n, k] (rhs_contract_last)
    or [batch, k, n]; each batch is eval_matmul_2d's loop (orc_matmul_2d).  Operands that do not
    factor that way are refused here (the reference reads zeros past them)."""
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    m, n = a.size // (batch * k), b.size // (batch * k)
    if a.size != batch * m * k or b.size != batch * k * n:
        raise ValueError("operands do not factor as [batch, m, k] x [batch, k, n]")
    a3 = a.reshape(batch, m, k)
    b3 = b.reshape((batch, n, k) if rhs_contract_last else (batch, k, n))
    return np.stack([matmul_2d(a3[i], b3[i], rhs_contract_last) for i in range(batch)])


def gemm_w8a16(x_bf16: np.ndarray, codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    m, k = x_bf16.shape
    n = codes.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().orc_gemm_w8a16(_p(x_bf16), m, n, k, _p(codes), _p(np.ascontiguousarray(scales, np.float32)), _p(out))
    return out


def gemm_w4a16(x_bf16, codes, scales, zeros, n, k, group) -> np.ndarray:
    m = x_bf16.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().orc_gemm_w4a16(_p(x_bf16), m, n, k, group, _p(codes), _p(scales), _p(zeros), _p(out))
    return out


def gemm_nf4(x_bf16, codes, absmax, n, k, block) -> np.ndarray:
    m = x_bf16.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().orc_gemm_nf4(_p(x_bf16), m, n, k, block, _p(codes), _p(absmax), _p(out))
    return out


def gemm_fp8(qa, sa, qw, sw) -> np.ndarray:
    m, k = qa.shape
    n = qw.shape[0]
    out = np.zeros((m, n), np.float32)
    lib().orc_gemm_fp8(_p(qa), _p(sa), m, _p(qw), _p(sw), n, k, _p(out))
    return out


# ------------------------------------------------------------------- helpers ----
def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (numpy)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)
