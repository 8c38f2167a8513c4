"""ctypes binding of include/castforge_hip.h (libcastforge_hip.so).

Modelled on the reference's Python SDK (bindings/python/castforge.py:22-41, 91-133): load the
shared library, declare argument/return types, turn non-zero status codes into exceptions and
free error strings with the library's own free function.  There is no fallback: if the
library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os
import re
from ctypes import POINTER, c_char_p, c_int32, c_int64, c_uint16, c_uint32, c_uint8, c_void_p
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("CASTFORGE_HIP_LIB", PKG / "libcastforge_hip.so"))
HEADER = PKG.parent / "include" / "castforge_hip.h"

ROUND_HALF_AWAY, ROUND_HALF_EVEN = 0, 1
GRAN_TENSOR, GRAN_CHANNEL = 0, 1
DTYPE_F32, DTYPE_BF16 = 0, 1
MAX_BATCH = 8
GROUPWISE_WORKSPACE_BYTES = 2048
EPI_BIAS, EPI_RELU, EPI_TANH, EPI_SILU, EPI_GELU, EPI_SCALE = range(6)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_BF16 = 0, 1, 2, 8, 30


class CastForgeHipError(RuntimeError):
    """A non-zero status from the C ABI (1 = reported error, 2 = internal exception)."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} failed (status {code}): {message}")
        self.code = code
        self.message = message


class QuantProblem(ctypes.Structure):
    _fields_ = [
        ("src", c_void_p),
        ("rows", c_int64),
        ("cols", c_int64),
        ("codes", c_void_p),
        ("scales", c_void_p),
        ("zeros", c_void_p),
    ]


class W8A16Problem(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p),
        ("codes", c_void_p),
        ("scales", c_void_p),
        ("y", c_void_p),
        ("n", c_int64),
        ("k", c_int64),
        ("granularity", c_int32),
    ]


class Nf4Problem(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p),
        ("codes", c_void_p),
        ("absmax", c_void_p),
        ("y", c_void_p),
        ("n", c_int64),
        ("k", c_int64),
        ("block", c_int64),
    ]


class W4A16Problem(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p),
        ("codes", c_void_p),
        ("scales_f16", c_void_p),
        ("zeros", c_void_p),
        ("y", c_void_p),
        ("n", c_int64),
        ("k", c_int64),
        ("group", c_int64),
    ]


class GgufProblem(ctypes.Structure):
    _fields_ = [
        ("x", c_void_p),
        ("codes", c_void_p),
        ("scales_f16", c_void_p),
        ("y", c_void_p),
        ("n", c_int64),
        ("k", c_int64),
    ]


_P = c_void_p
_E = POINTER(c_char_p)
# name -> (restype, argtypes) for every entry point of the header
SIGNATURES = {
    "castforge_hip_version": (c_char_p, []),
    "castforge_hip_free_string": (None, [c_void_p]),
    "castforge_hip_device_info": (c_int32, [POINTER(c_void_p), _E]),
    "castforge_hip_quantize_int8": (c_int32, [_P, c_int64, c_int64, c_int32, c_int32, c_int32, _P, _P, _P, _E]),
    "castforge_hip_dequantize_int8": (c_int32, [_P, _P, c_int64, c_int64, c_int32, _P, _P, _E]),
    "castforge_hip_quantize_int4g": (c_int32, [_P, c_int64, c_int64, c_int64, _P, _P, _P, _P, _E]),
    "castforge_hip_quantize_int4g_awq": (c_int32, [_P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _P, _E]),
    "castforge_hip_dequantize_int4g": (c_int32, [_P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _E]),
    "castforge_hip_quantize_nf4": (c_int32, [_P, c_int64, c_int64, c_int64, _P, _P, _P, _E]),
    "castforge_hip_dequantize_nf4": (c_int32, [_P, _P, c_int64, c_int64, c_int64, _P, _P, _E]),
    "castforge_hip_quantize_fp8": (c_int32, [_P, c_int32, c_int64, c_int64, _P, _P, _P, _E]),
    "castforge_hip_dequantize_fp8": (c_int32, [_P, _P, c_int64, c_int64, _P, _P, _E]),
    "castforge_hip_gemv_w4a16": (c_int32, [_P, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, _P, c_int32, _P, _E]),
    "castforge_hip_gemv_w8a16": (c_int32, [_P, c_int64, c_int64, c_int64, _P, _P, c_int32, _P, c_int32, _P, _E]),
    "castforge_hip_gemv_nf4": (c_int32, [_P, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, c_int32, _P, _E]),
    "castforge_hip_gemv_w4a16_batched": (c_int32, [POINTER(W4A16Problem), c_int32, c_int64, c_int32, _P, _E]),
    "castforge_hip_gemv_w8a16_batched": (c_int32, [POINTER(W8A16Problem), c_int32, c_int64, c_int32, _P, _E]),
    "castforge_hip_int4g_to_planes": (c_int32, [_P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _P, _E]),
    "castforge_hip_int4g_from_planes": (c_int32, [_P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _P, _E]),
    "castforge_hip_gemv_w4a16_planes_batched": (c_int32, [POINTER(W4A16Problem), c_int32, c_int64, c_int32, _P, _E]),
    "castforge_hip_gemv_nf4_batched": (c_int32, [POINTER(Nf4Problem), c_int32, c_int64, c_int32, _P, _E]),
    "castforge_hip_nf4_to_planes": (c_int32, [_P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _E]),
    "castforge_hip_nf4_from_planes": (c_int32, [_P, _P, c_int64, c_int64, c_int64, _P, _P, _P, _E]),
    "castforge_hip_gemv_nf4_planes_batched": (c_int32, [POINTER(Nf4Problem), c_int32, c_int64, c_int32, _P, _E]),
    "castforge_hip_quantize_int4g_batched": (c_int32, [POINTER(QuantProblem), c_int32, c_int64, _P, _E]),
    "castforge_hip_quantize_int4g_awq_batched": (c_int32, [POINTER(QuantProblem), POINTER(_P), c_int32, c_int64, _P,
                                                           _E]),
    "castforge_hip_quantize_int8_batched": (c_int32, [POINTER(QuantProblem), c_int32, c_int32, c_int32, _P, _E]),
    "castforge_hip_gemm_fp8": (c_int32, [_P, _P, c_int64, _P, _P, c_int64, c_int64, _P, c_int32, _P, _E]),
    "castforge_hip_gemm_fp8_exact": (c_int32, [_P, _P, c_int64, _P, _P, c_int64, c_int64, _P, c_int32, _P, _E]),
    "castforge_hip_quantize_groupwise": (c_int32, [_P, c_int64, c_int32, c_int64, c_int32, ctypes.c_float, c_int32,
                                                   _P, _P, _P, POINTER(c_int64), _P, _E]),
    "castforge_hip_quantize_groupwise_noalloc": (c_int32, [_P, c_int64, c_int32, c_int64, c_int32, ctypes.c_float,
                                                           c_int32, _P, _P, POINTER(c_int64), _P, _E]),
    "castforge_hip_quantize_fp8_grid": (c_int32, [_P, c_int64, c_int32, c_int32, c_int64, _P, _P, _E]),
    "castforge_hip_qmatmul_epilogue": (c_int32, [_P, c_int64, _P, c_int64, _P, c_int64, c_int32, _P, _E]),
    "castforge_hip_static_quantize": (c_int32, [_P, c_int64, ctypes.c_float, c_int32, _P, _P, _E]),
    "castforge_hip_absmax_f32": (c_int32, [_P, c_int64, _P, _P, _E]),
    "castforge_hip_convert_f32_to_bf16": (c_int32, [_P, c_int64, _P, _P, _E]),
    "castforge_hip_convert_bf16_to_f32": (c_int32, [_P, c_int64, _P, _P, _E]),
    "castforge_hip_transpose": (c_int32, [_P, c_int64, c_int64, c_int32, _P, _P, _E]),
    "castforge_hip_matmul_f32": (c_int32, [_P, c_int64, c_int64, _P, c_int64, c_int32, _P, _P, _E]),
    "castforge_hip_rotate_hadamard": (c_int32, [_P, c_int64, c_int64, c_int64, c_int32, _P, _P, _E]),
    "castforge_hip_quantize_int4g_hadamard": (c_int32, [_P, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, _P, _E]),
    "castforge_hip_smoothquant_scales": (c_int32, [ctypes.c_float, ctypes.c_float, ctypes.c_float, c_int32, _P, _E]),
    "castforge_hip_smoothquant": (c_int32, [_P, c_int64, ctypes.c_float, ctypes.c_float, c_int32, _P, _P, _E]),
    "castforge_hip_gguf_payload_bytes": (c_int32, [c_int32, c_int64, POINTER(c_int64), _E]),
    "castforge_hip_gguf_decode": (c_int32, [c_int32, _P, c_int64, _P, _P, _E]),
    "castforge_hip_gguf_encode": (c_int32, [c_int32, _P, c_int64, ctypes.c_float, _P, _P, _E]),
    "castforge_hip_gguf_repack": (c_int32, [c_int32, _P, c_int64, c_int64, _P, _P, _P, _E]),
    "castforge_hip_gguf_unpack": (c_int32, [c_int32, _P, _P, c_int64, c_int64, _P, _P, _E]),
    "castforge_hip_gguf_q4_0_to_int4g": (c_int32, [_P, c_int64, c_int64, _P, _P, _P, _E]),
    "castforge_hip_dequantize_gguf": (c_int32, [c_int32, _P, _P, c_int64, c_int64, _P, _P, _E]),
    "castforge_hip_gemv_gguf": (c_int32, [c_int32, _P, c_int64, c_int64, c_int64, _P, _P, _P, c_int32, _P, _E]),
    "castforge_hip_gemv_gguf_batched": (c_int32, [c_int32, POINTER(GgufProblem), c_int32, c_int64, c_int32, _P, _E]),
    "castforge_hip_gguf_q4_0_to_gemv_planes": (c_int32, [_P, _P, c_int64, c_int64, _P, _P, _P, _E]),
    "castforge_hip_gguf_q4_0_from_gemv_planes": (c_int32, [_P, _P, c_int64, c_int64, _P, _P, _P, _E]),
    "castforge_hip_gemv_gguf_q4_0_planes_batched": (c_int32, [POINTER(GgufProblem), c_int32, c_int64, c_int32, _P, _E]),
}

_lib = None


def header_symbols() -> list[str]:
    """Function names declared in include/castforge_hip.h."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(castforge_hip_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() or python castforge_amd/build.py")
        l = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


def call(name: str, *args) -> None:
    """Calls an entry point that ends with `char** out_error` and raises on non-zero status."""
    err = c_char_p()
    rc = getattr(lib(), name)(*args, ctypes.byref(err))
    if rc != 0:
        msg = err.value.decode("utf-8", "replace") if err.value else "(no message)"
        if err.value is not None:
            lib().castforge_hip_free_string(ctypes.cast(err, c_void_p))
        raise CastForgeHipError(name, rc, msg)


def version() -> str:
    return lib().castforge_hip_version().decode()


def device_info() -> str:
    out = c_void_p()
    err = c_char_p()
    rc = lib().castforge_hip_device_info(ctypes.byref(out), ctypes.byref(err))
    if rc != 0:
        msg = err.value.decode() if err.value else ""
        if err.value is not None:
            lib().castforge_hip_free_string(ctypes.cast(err, c_void_p))
        raise CastForgeHipError("castforge_hip_device_info", rc, msg)
    s = ctypes.cast(out, c_char_p).value.decode()
    lib().castforge_hip_free_string(out)
    return s
