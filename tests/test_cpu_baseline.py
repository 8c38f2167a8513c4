"""The CPU-C best-effort host baseline (oracle/cpu_best.c) that bench.py times next to the port:
it must compute the same W4A16 GEMV as the oracle, within the north-star bound (its rounding is
not the reference's sequential loop), on ragged shapes, several group counts and thread counts."""
import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle_lib as O
from castforge_amd import synth

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "oracle" / "_build" / "libcf_cpubest.so"


def _lib():
    if not LIB.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "-s"], check=True)
    lib = ctypes.CDLL(str(LIB))
    P = ctypes.c_void_p
    lib.cpub_gemv_w4a16.argtypes = [P, ctypes.c_int64, ctypes.c_int64, P, P, P, P, ctypes.c_int]
    return lib


@pytest.mark.parametrize("n,k,threads", [(1, 128, 1), (37, 1024, 3), (256, 4096, 0), (64, 11008, 8)])
def test_cpu_best_effort_gemv_matches_oracle(n, k, threads):
    lib = _lib()
    w = synth.weight(91, 1, n, k)
    codes, scales, zeros = O.quantize_int4g(w, 128)
    xb = synth.activations_bf16(92, 7, 1, k)
    x = np.ascontiguousarray(O.bf16_bits_to_f32(xb).reshape(-1), dtype=np.float32)
    y = np.zeros(n, np.float32)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    lib.cpub_gemv_w4a16(ptr(x), n, k, ptr(codes), ptr(scales), ptr(zeros), ptr(y), threads)
    ref = O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128).reshape(-1)
    assert np.all(np.abs(y - ref) <= 1e-3 + 1e-2 * np.abs(ref))


CG_LIB = ROOT / "oracle" / "_build" / "libcf_cpucodegen.so"


@pytest.mark.parametrize("m,n,k", [(1, 1, 128), (1, 37, 1024), (2, 64, 4096), (1, 16, 11008)])
def test_cpu_codegen_faithful_gemv_equals_oracle_bits(m, n, k):
    """CPU-B (oracle/cpu_codegen.c), the emitted loop nest with the dequant inline, rounds every
    product and sum like the reference evaluator's dequantize + eval_matmul_2d: its outputs equal
    the oracle's bit for bit (f16 subnormal scales included)."""
    if not CG_LIB.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "-s"], check=True)
    lib = ctypes.CDLL(str(CG_LIB))
    P = ctypes.c_void_p
    lib.cpcg_gemv_w4a16.argtypes = [P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, P, P, P, P]
    w = synth.weight(93, 1, n, k)
    w[:, :128] *= np.float32(1e-6)  # group 0 of every row gets an f16 subnormal scale
    codes, scales, zeros = O.quantize_int4g(w, 128)
    assert (scales[:, 0] < 0x0400).all() and (scales[:, 0] > 0).any()
    xb = synth.activations_bf16(94, 7, m, k)
    x = np.ascontiguousarray(O.bf16_bits_to_f32(xb).reshape(m, k), dtype=np.float32)
    y = np.zeros((m, n), np.float32)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    lib.cpcg_gemv_w4a16(ptr(x), m, n, k, ptr(codes), ptr(scales), ptr(zeros), ptr(y))
    ref = O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128).reshape(m, n)
    assert np.array_equal(y, ref)
