"""Torch-tensor front end over the C ABI: allocates outputs on the input's device and enqueues
the HIP kernels on torch's current stream.  PyTorch is only used for device memory and
streams; every computation happens in libcastforge_hip.so.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import ffi
from .ffi import DTYPE_BF16, DTYPE_F32, GRAN_CHANNEL, GRAN_TENSOR, ROUND_HALF_AWAY, ROUND_HALF_EVEN

_ROUND = {"half_away": ROUND_HALF_AWAY, "half_even": ROUND_HALF_EVEN}
_GRAN = {"tensor": GRAN_TENSOR, "channel": GRAN_CHANNEL}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dev(t: torch.Tensor) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError("castforge_amd kernels take device tensors (HIP); got a CPU tensor")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    return t


def _out_dtype(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return DTYPE_F32
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    raise ValueError(f"output dtype must be float32 or bfloat16, got {dtype}")


# ---------------------------------------------------------------------------- INT8 ----
def quantize_int8(w: torch.Tensor, bits: int = 8, granularity: str = "channel",
                  round: str = "half_even") -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric absmax INT8 (or INT4-in-int8 when bits=4). Returns (codes i8, scales f32)."""
    w = _dev(w)
    if w.dtype != torch.float32:
        raise ValueError("quantize_int8 takes float32 weights")
    rows, cols = (w.shape[0], math.prod(w.shape[1:])) if w.dim() >= 2 else (1, w.numel())
    codes = torch.empty(w.shape, dtype=torch.int8, device=w.device)
    scales = torch.empty(rows if granularity == "channel" else 1, dtype=torch.float32, device=w.device)
    if granularity == "tensor":
        rows, cols = 1, w.numel()
    ffi.call("castforge_hip_quantize_int8", _ptr(w), rows, cols, bits, _GRAN[granularity],
             _ROUND[round], _ptr(codes), _ptr(scales), _stream(w))
    return codes, scales


def dequantize_int8(codes: torch.Tensor, scales: torch.Tensor, granularity: str = "channel") -> torch.Tensor:
    codes = _dev(codes)
    rows = codes.shape[0] if codes.dim() >= 2 else 1
    cols = codes.numel() // max(rows, 1) if rows else 0
    out = torch.empty(codes.shape, dtype=torch.float32, device=codes.device)
    ffi.call("castforge_hip_dequantize_int8", _ptr(codes), _ptr(_dev(scales)), rows, cols,
             _GRAN[granularity], _ptr(out), _stream(codes))
    return out


# --------------------------------------------------------------------------- INT4g ----
@dataclass
class Int4Packed:
    """INT4 asymmetric group-wise weights: codes u32 [N, K/8], scales f16 [N, 8*ceil(G/8)] (row-padded),
    zeros u32 [N, ceil(G/8)]."""
    codes: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    n: int
    k: int
    group: int

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.codes, self.scales, self.zeros))


def quantize_int4g(w: torch.Tensor, group: int = 128, in_scale: torch.Tensor | None = None) -> Int4Packed:
    """INT4 asymmetric group-wise; with `in_scale` (f32 [K]) the AWQ-style pre-scaled
    W * in_scale[k] is quantized (fused, one pass)."""
    w = _dev(w)
    if w.dtype != torch.float32 or w.dim() != 2:
        raise ValueError("quantize_int4g takes a 2-D float32 [N, K] weight")
    n, k = w.shape
    g = (k + group - 1) // group
    codes = torch.empty((n, k // 8), dtype=torch.int32, device=w.device)
    scales = torch.empty((n, (g + 7) // 8 * 8), dtype=torch.float16, device=w.device)
    zeros = torch.empty((n, (g + 7) // 8), dtype=torch.int32, device=w.device)
    if in_scale is None:
        ffi.call("castforge_hip_quantize_int4g", _ptr(w), n, k, group, _ptr(codes), _ptr(scales),
                 _ptr(zeros), _stream(w))
    else:
        in_scale = _dev(in_scale)
        if in_scale.dtype != torch.float32 or in_scale.numel() != k:
            raise ValueError("in_scale must be float32 [K]")
        ffi.call("castforge_hip_quantize_int4g_awq", _ptr(w), _ptr(in_scale), n, k, group, _ptr(codes),
                 _ptr(scales), _ptr(zeros), _stream(w))
    return Int4Packed(codes, scales, zeros, n, k, group)


def _quant_batch(ws: list[torch.Tensor]) -> list[torch.Tensor]:
    if len(ws) > ffi.MAX_BATCH:
        raise ValueError(f"at most {ffi.MAX_BATCH} matrices per batched call")
    ws = [_dev(w) for w in ws]
    for w in ws:
        if w.dtype != torch.float32 or w.dim() != 2:
            raise ValueError("batched quantize takes 2-D float32 [N, K] weights")
    return ws


def quantize_int4g_batched(ws: list[torch.Tensor], group: int = 128,
                           in_scales: list[torch.Tensor] | None = None) -> list[Int4Packed]:
    """quantize_int4g over several matrices in one launch per column count (bit-identical);
    with in_scales, the AWQ form (quantize_int4g(w, group, in_scale) per matrix)."""
    ws = _quant_batch(ws)
    if in_scales is not None:
        if len(in_scales) != len(ws):
            raise ValueError("in_scales must hold one f32 [K] tensor per matrix")
        in_scales = [_dev(s) for s in in_scales]
        for s, w in zip(in_scales, ws):
            if (s.dtype != torch.float32 or s.dim() != 1 or s.numel() != w.shape[1] or not s.is_contiguous()
                    or s.device != w.device or s.data_ptr() % 16):
                raise ValueError("each in_scale must be a contiguous 16-byte aligned float32 [K] on the "
                                 "weight's device")
    out, arr = [], (ffi.QuantProblem * max(1, len(ws)))()
    for i, w in enumerate(ws):
        n, k = w.shape
        g = (k + group - 1) // group
        codes = torch.empty((n, k // 8), dtype=torch.int32, device=w.device)
        scales = torch.empty((n, (g + 7) // 8 * 8), dtype=torch.float16, device=w.device)
        zeros = torch.empty((n, (g + 7) // 8), dtype=torch.int32, device=w.device)
        arr[i] = ffi.QuantProblem(_ptr(w), n, k, _ptr(codes), _ptr(scales), _ptr(zeros))
        out.append(Int4Packed(codes, scales, zeros, n, k, group))
    if ws and in_scales is not None:
        ptrs = (ctypes.c_void_p * len(ws))(*[s.data_ptr() for s in in_scales])
        ffi.call("castforge_hip_quantize_int4g_awq_batched", arr, ptrs, len(ws), group, _stream(ws[0]))
    elif ws:
        ffi.call("castforge_hip_quantize_int4g_batched", arr, len(ws), group, _stream(ws[0]))
    return out


def quantize_int8_batched(ws: list[torch.Tensor], bits: int = 8, round: str = "half_even"
                          ) -> list[tuple[torch.Tensor, torch.Tensor]]:
    """quantize_int8(granularity="channel") over several matrices in one launch per column count."""
    ws = _quant_batch(ws)
    out, arr = [], (ffi.QuantProblem * max(1, len(ws)))()
    for i, w in enumerate(ws):
        n, k = w.shape
        codes = torch.empty((n, k), dtype=torch.int8, device=w.device)
        scales = torch.empty(n, dtype=torch.float32, device=w.device)
        arr[i] = ffi.QuantProblem(_ptr(w), n, k, _ptr(codes), _ptr(scales), None)
        out.append((codes, scales))
    if ws:
        ffi.call("castforge_hip_quantize_int8_batched", arr, len(ws), bits, _ROUND[round], _stream(ws[0]))
    return out


def dequantize_int4g(p: Int4Packed) -> torch.Tensor:
    out = torch.empty((p.n, p.k), dtype=torch.float32, device=p.codes.device)
    ffi.call("castforge_hip_dequantize_int4g", _ptr(p.codes), _ptr(p.scales), _ptr(p.zeros), p.n,
             p.k, p.group, _ptr(out), _stream(p.codes))
    return out


# ----------------------------------------------------------------------------- NF4 ----
@dataclass
class Nf4Packed:
    codes: torch.Tensor
    absmax: torch.Tensor
    n: int
    k: int
    block: int

    def nbytes(self) -> int:
        return self.codes.numel() * 4 + self.absmax.numel() * 4


def quantize_nf4(w: torch.Tensor, block: int = 64) -> Nf4Packed:
    w = _dev(w)
    if w.dtype != torch.float32 or w.dim() != 2:
        raise ValueError("quantize_nf4 takes a 2-D float32 [N, K] weight")
    n, k = w.shape
    nb = (k + block - 1) // block
    codes = torch.empty((n, k // 8), dtype=torch.int32, device=w.device)
    absmax = torch.empty((n, nb), dtype=torch.float32, device=w.device)
    ffi.call("castforge_hip_quantize_nf4", _ptr(w), n, k, block, _ptr(codes), _ptr(absmax), _stream(w))
    return Nf4Packed(codes, absmax, n, k, block)


def dequantize_nf4(p: Nf4Packed) -> torch.Tensor:
    out = torch.empty((p.n, p.k), dtype=torch.float32, device=p.codes.device)
    ffi.call("castforge_hip_dequantize_nf4", _ptr(p.codes), _ptr(p.absmax), p.n, p.k, p.block,
             _ptr(out), _stream(p.codes))
    return out


# ----------------------------------------------------------------------------- FP8 ----
def quantize_fp8(v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row E4M3FN with scale absmax/448; v is float32 or bfloat16 [R, C]."""
    v = _dev(v)
    if v.dim() != 2:
        raise ValueError("quantize_fp8 takes a 2-D [rows, cols] tensor")
    if v.dtype == torch.float32:
        dt = DTYPE_F32
    elif v.dtype == torch.bfloat16:
        dt = DTYPE_BF16
    else:
        raise ValueError("quantize_fp8 takes float32 or bfloat16")
    r, c = v.shape
    codes = torch.empty((r, c), dtype=torch.uint8, device=v.device)
    scales = torch.empty(r, dtype=torch.float32, device=v.device)
    ffi.call("castforge_hip_quantize_fp8", _ptr(v), dt, r, c, _ptr(codes), _ptr(scales), _stream(v))
    return codes, scales


def dequantize_fp8(codes: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    codes = _dev(codes)
    r, c = codes.shape
    out = torch.empty((r, c), dtype=torch.float32, device=codes.device)
    ffi.call("castforge_hip_dequantize_fp8", _ptr(codes), _ptr(_dev(scales)), r, c, _ptr(out),
             _stream(codes))
    return out


# ------------------------------------------------------------------- fused matmuls ----
def _check_x(x: torch.Tensor, k: int) -> torch.Tensor:
    x = _dev(x)
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[1] != k:
        raise ValueError(f"x must be bfloat16 [M, {k}]")
    return x


def _check_batch(xs: list[torch.Tensor], ys: list[torch.Tensor], m: int, ns: list[int], ks: list[int]) -> int:
    """Validates the activations and preallocated outputs of a batched launch: every x bf16
    [m, k] and every y contiguous [m, n] on x's device, all y of ONE dtype (f32 or bf16, the
    C ABI takes a single y_dtype for the batch).  Returns that dtype's ABI code."""
    dev = xs[0].device
    for x, y, n, k in zip(xs, ys, ns, ks):
        _check_x(x, k)
        _dev(y)
        if x.device != dev or y.device != dev:
            raise ValueError("every x and y of a batch must be on the same device")
        if x.shape[0] != m or tuple(y.shape) != (m, n):
            raise ValueError("all problems must share M and y must be [M, n]")
        if y.dtype != ys[0].dtype:
            raise ValueError(f"every y of a batch must have one dtype: {ys[0].dtype} and {y.dtype}")
    return _out_dtype(ys[0].dtype)


def gemm_w4a16(x: torch.Tensor, p: Int4Packed, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    x = _check_x(x, p.k)
    y = torch.empty((x.shape[0], p.n), dtype=out_dtype, device=x.device)
    ffi.call("castforge_hip_gemv_w4a16", _ptr(x), x.shape[0], p.n, p.k, p.group, _ptr(p.codes),
             _ptr(p.scales), _ptr(p.zeros), _ptr(y), _out_dtype(out_dtype), _stream(x))
    return y


def gemm_w8a16(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor,
               granularity: str = "channel", out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    n, k = codes.shape
    x = _check_x(x, k)
    y = torch.empty((x.shape[0], n), dtype=out_dtype, device=x.device)
    ffi.call("castforge_hip_gemv_w8a16", _ptr(x), x.shape[0], n, k, _ptr(_dev(codes)),
             _ptr(_dev(scales)), _GRAN[granularity], _ptr(y), _out_dtype(out_dtype), _stream(x))
    return y


def gemm_nf4(x: torch.Tensor, p: Nf4Packed, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    x = _check_x(x, p.k)
    y = torch.empty((x.shape[0], p.n), dtype=out_dtype, device=x.device)
    ffi.call("castforge_hip_gemv_nf4", _ptr(x), x.shape[0], p.n, p.k, p.block, _ptr(p.codes),
             _ptr(p.absmax), _ptr(y), _out_dtype(out_dtype), _stream(x))
    return y


def gemm_fp8(qa: torch.Tensor, sa: torch.Tensor, qw: torch.Tensor, sw: torch.Tensor,
             out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.bfloat16,
             exact: bool = False) -> torch.Tensor:
    """W8A8: qa u8 E4M3 [M, K] with per-token sa [M]; qw u8 E4M3 [N, K] with per-row sw [N];
    returns [M, N] in out_dtype (bfloat16 or float32).

    exact=False runs the fp8 MFMA kernel, whose adder keeps ~13 bits below the largest
    product of each block of eight (near-zero outputs of outlier-heavy inputs can miss the
    f32 evaluator by more than 1e-3); exact=True widens the codes to f16 and runs f16 MFMA,
    which stays within 1e-2 relative / 1e-3 absolute of the f32 evaluator at about half the
    rate."""
    qa, qw = _dev(qa), _dev(qw)
    m, k = qa.shape
    n, k2 = qw.shape
    if k != k2 or qa.dtype != torch.uint8 or qw.dtype != torch.uint8:
        raise ValueError("qa [M, K] and qw [N, K] must be uint8 E4M3 codes with the same K")
    if out is not None:
        if (tuple(out.shape) != (m, n) or not out.is_contiguous() or out.device != qa.device
                or out.dtype not in (torch.bfloat16, torch.float32)):
            raise ValueError(f"out must be a contiguous bfloat16/float32 [{m}, {n}] tensor on {qa.device}")
    y = out if out is not None else torch.empty((m, n), dtype=out_dtype, device=qa.device)
    ffi.call("castforge_hip_gemm_fp8_exact" if exact else "castforge_hip_gemm_fp8", _ptr(qa),
             _ptr(_dev(sa)), m, _ptr(qw), _ptr(_dev(sw)), n, k, _ptr(y), _out_dtype(y.dtype), _stream(qa))
    return y


def gemv_w4a16_batched(xs: list[torch.Tensor], ps: list[Int4Packed], ys: list[torch.Tensor]) -> None:
    """One launch for several W4A16 problems with the same M (1..64); outputs preallocated."""
    if not (len(xs) == len(ps) == len(ys)) or len(ps) > ffi.MAX_BATCH:
        raise ValueError("xs, ps, ys must have the same length <= 8")
    if not ps:
        return
    m = xs[0].shape[0]
    yd = _check_batch(xs, ys, m, [p.n for p in ps], [p.k for p in ps])
    arr = (ffi.W4A16Problem * len(ps))()
    for i, (x, p, y) in enumerate(zip(xs, ps, ys)):
        arr[i] = ffi.W4A16Problem(_ptr(x), _ptr(p.codes), _ptr(p.scales), _ptr(p.zeros), _ptr(y),
                                  p.n, p.k, p.group)
    ffi.call("castforge_hip_gemv_w4a16_batched", arr, len(ps), m, yd, _stream(xs[0]))


@dataclass
class Int4Planes:
    """INT4 g128 weights in the GEMV planes layout (castforge_hip_int4g_to_planes): codes u8
    [T * G * 1024], scales f16 [T, G, 16], zeros u8 [T, G, 8] with T = ceil(N/16), G = K/128."""
    codes: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor
    n: int
    k: int
    group: int = 128

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.codes, self.scales, self.zeros))


def int4g_to_planes(p: Int4Packed) -> Int4Planes:
    """The GEMV planes of canonical INT4 g128 weights (built once, at load time)."""
    if p.group != 128 or p.k % 128:
        raise ValueError("GEMV planes hold INT4 weights with group 128 and k % 128 == 0")
    t, g = (p.n + 15) // 16, p.k // 128
    dev = p.codes.device
    pl = Int4Planes(torch.empty(t * g * 1024, dtype=torch.uint8, device=dev),
                    torch.empty((t, g, 16), dtype=torch.float16, device=dev),
                    torch.empty((t, g, 8), dtype=torch.uint8, device=dev), p.n, p.k, 128)
    ffi.call("castforge_hip_int4g_to_planes", _ptr(_dev(p.codes)), _ptr(_dev(p.scales)), _ptr(_dev(p.zeros)),
             p.n, p.k, 128, _ptr(pl.codes), _ptr(pl.scales), _ptr(pl.zeros), _stream(p.codes))
    return pl


def int4g_from_planes(pl: Int4Planes) -> Int4Packed:
    """Canonical INT4 g128 arrays back from GEMV planes (bit for bit)."""
    n, k = pl.n, pl.k
    g = k // 128
    dev = pl.codes.device
    p = Int4Packed(torch.empty((n, k // 8), dtype=torch.int32, device=dev),
                   torch.empty((n, (g + 7) // 8 * 8), dtype=torch.float16, device=dev),
                   torch.empty((n, (g + 7) // 8), dtype=torch.int32, device=dev), n, k, 128)
    ffi.call("castforge_hip_int4g_from_planes", _ptr(_dev(pl.codes)), _ptr(_dev(pl.scales)), _ptr(_dev(pl.zeros)),
             n, k, 128, _ptr(p.codes), _ptr(p.scales), _ptr(p.zeros), _stream(pl.codes))
    return p


def gemv_w4a16_planes_batched(xs: list[torch.Tensor], ps: list[Int4Planes], ys: list[torch.Tensor]) -> None:
    """Decode (M = 1..16 rows of x, the same M for every problem) over GEMV planes, all problems
    in one launch (one workgroup per CU)."""
    if not (len(xs) == len(ps) == len(ys)) or not 1 <= len(ps) <= ffi.MAX_BATCH:
        raise ValueError("xs, ps, ys must have the same length in 1..8")
    m = xs[0].shape[0] if xs[0].dim() == 2 else 0
    if not 1 <= m <= 16:
        raise ValueError("the GEMV planes kernels take x of 1..16 rows")
    yd = _check_batch(xs, ys, m, [p.n for p in ps], [p.k for p in ps])
    arr = (ffi.W4A16Problem * len(ps))()
    for i, (x, p, y) in enumerate(zip(xs, ps, ys)):
        arr[i] = ffi.W4A16Problem(_ptr(x), _ptr(p.codes), _ptr(p.scales), _ptr(p.zeros), _ptr(y), p.n, p.k, 128)
    ffi.call("castforge_hip_gemv_w4a16_planes_batched", arr, len(ps), m, yd, _stream(xs[0]))


def gemv_w4a16_planes(x: torch.Tensor, p: Int4Planes, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """y [M, n] for x bf16 [M, k], M = 1..16, over GEMV planes."""
    y = torch.empty((x.shape[0] if x.dim() == 2 else 1, p.n), dtype=out_dtype, device=x.device)
    gemv_w4a16_planes_batched([x], [p], [y])
    return y


def gemv_w8a16_batched(xs: list[torch.Tensor], qs: list[tuple[torch.Tensor, torch.Tensor]],
                       ys: list[torch.Tensor], granularity: str = "channel") -> None:
    """One launch for several W8A16 problems (codes i8 [n, k], scales f32) with the same M."""
    if not (len(xs) == len(qs) == len(ys)) or len(qs) > ffi.MAX_BATCH:
        raise ValueError("xs, qs, ys must have the same length <= 8")
    if not qs:
        return
    m = xs[0].shape[0]
    yd = _check_batch(xs, ys, m, [q.shape[0] for q, _ in qs], [q.shape[1] for q, _ in qs])
    arr = (ffi.W8A16Problem * len(qs))()
    for i, (x, (q, s), y) in enumerate(zip(xs, qs, ys)):
        n, k = q.shape
        arr[i] = ffi.W8A16Problem(_ptr(x), _ptr(_dev(q)), _ptr(_dev(s)), _ptr(y), n, k, _GRAN[granularity])
    ffi.call("castforge_hip_gemv_w8a16_batched", arr, len(qs), m, yd, _stream(xs[0]))


def gemv_nf4_batched(xs: list[torch.Tensor], ps: list["Nf4Packed"], ys: list[torch.Tensor]) -> None:
    """One launch for several NF4 problems with the same M and block size."""
    if not (len(xs) == len(ps) == len(ys)) or len(ps) > ffi.MAX_BATCH:
        raise ValueError("xs, ps, ys must have the same length <= 8")
    if not ps:
        return
    m = xs[0].shape[0]
    yd = _check_batch(xs, ys, m, [p.n for p in ps], [p.k for p in ps])
    arr = (ffi.Nf4Problem * len(ps))()
    for i, (x, p, y) in enumerate(zip(xs, ps, ys)):
        arr[i] = ffi.Nf4Problem(_ptr(x), _ptr(p.codes), _ptr(p.absmax), _ptr(y), p.n, p.k, p.block)
    ffi.call("castforge_hip_gemv_nf4_batched", arr, len(ps), m, yd, _stream(xs[0]))


@dataclass
class Nf4Planes:
    """NF4 weights in the GEMV planes layout (castforge_hip_nf4_to_planes): codes u8
    [T * G * 1024], absmax f32 [T, G, 16, nbpc] with T = ceil(N/16), G = K/128 and
    nbpc = max(1, 128 / block)."""
    codes: torch.Tensor
    absmax: torch.Tensor
    n: int
    k: int
    block: int

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.codes, self.absmax))


def _nf4_planes_block_ok(block: int) -> bool:
    return block >= 32 and block & (block - 1) == 0


def nf4_to_planes(p: Nf4Packed) -> Nf4Planes:
    """The GEMV planes of canonical NF4 weights (built once, at load time)."""
    if p.k % 128 or not _nf4_planes_block_ok(p.block):
        raise ValueError("NF4 planes need k % 128 == 0 and a power-of-two block >= 32")
    t, g = (p.n + 15) // 16, p.k // 128
    nbpc = max(1, 128 // p.block)
    dev = p.codes.device
    pl = Nf4Planes(torch.empty(t * g * 1024, dtype=torch.uint8, device=dev),
                   torch.empty((t, g, 16, nbpc), dtype=torch.float32, device=dev), p.n, p.k, p.block)
    ffi.call("castforge_hip_nf4_to_planes", _ptr(_dev(p.codes)), _ptr(_dev(p.absmax)), p.n, p.k, p.block,
             _ptr(pl.codes), _ptr(pl.absmax), _stream(p.codes))
    return pl


def nf4_from_planes(pl: Nf4Planes) -> Nf4Packed:
    """Canonical NF4 codes and absmax back from NF4 planes (bit for bit)."""
    n, k, block = pl.n, pl.k, pl.block
    dev = pl.codes.device
    p = Nf4Packed(torch.empty((n, k // 8), dtype=torch.int32, device=dev),
                  torch.empty((n, (k + block - 1) // block), dtype=torch.float32, device=dev), n, k, block)
    ffi.call("castforge_hip_nf4_from_planes", _ptr(_dev(pl.codes)), _ptr(_dev(pl.absmax)), n, k, block,
             _ptr(p.codes), _ptr(p.absmax), _stream(pl.codes))
    return p


def gemv_nf4_planes_batched(xs: list[torch.Tensor], ps: list[Nf4Planes], ys: list[torch.Tensor]) -> None:
    """NF4 decode (x of one row) over NF4 planes, all problems in one launch (one workgroup per
    CU); every problem has the same block size."""
    if not (len(xs) == len(ps) == len(ys)) or not 1 <= len(ps) <= ffi.MAX_BATCH:
        raise ValueError("xs, ps, ys must have the same length in 1..8")
    m = xs[0].shape[0] if xs[0].dim() == 2 else 0
    if m != 1:
        raise ValueError("the NF4 planes kernel takes x of one row")
    yd = _check_batch(xs, ys, m, [p.n for p in ps], [p.k for p in ps])
    arr = (ffi.Nf4Problem * len(ps))()
    for i, (x, p, y) in enumerate(zip(xs, ps, ys)):
        arr[i] = ffi.Nf4Problem(_ptr(x), _ptr(p.codes), _ptr(p.absmax), _ptr(y), p.n, p.k, p.block)
    ffi.call("castforge_hip_gemv_nf4_planes_batched", arr, len(ps), m, yd, _stream(xs[0]))


def gemv_nf4_planes(x: torch.Tensor, p: Nf4Planes, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """y [1, n] for x bf16 [1, k] over NF4 planes."""
    y = torch.empty((1, p.n), dtype=out_dtype, device=x.device)
    gemv_nf4_planes_batched([x], [p], [y])
    return y


# -------------------------------------------------------------- outlier suppression ----
def rotate_hadamard(w: torch.Tensor, block: int, axis: int = 0, out: torch.Tensor | None = None) -> torch.Tensor:
    """Walsh-Hadamard rotation of f32 [d0, d1] in blocks of `block` along `axis` (0: down the
    columns, rotate-hadamard's order; 1: along rows).  out may be w (in place)."""
    w = _dev(w)
    if w.dtype != torch.float32 or w.dim() != 2:
        raise ValueError("rotate_hadamard takes a float32 [d0, d1] tensor")
    out = torch.empty_like(w) if out is None else _dev(out)
    ffi.call("castforge_hip_rotate_hadamard", _ptr(w), w.shape[0], w.shape[1], block, axis, _ptr(out), _stream(w))
    return out


def quantize_int4g_hadamard(w: torch.Tensor, group: int = 128, block: int = 128) -> "Int4Packed":
    """INT4g codes of the row-wise (K-axis) Hadamard rotation of w [N, K], in one pass."""
    w = _dev(w)
    if w.dtype != torch.float32 or w.dim() != 2:
        raise ValueError("quantize_int4g_hadamard takes a float32 [N, K] tensor")
    n, k = w.shape
    g = (k + group - 1) // group
    zw = (g + 7) // 8
    codes = torch.empty((n, k // 8), dtype=torch.int32, device=w.device)
    scales = torch.empty((n, zw * 8), dtype=torch.float16, device=w.device)
    zeros = torch.empty((n, zw), dtype=torch.int32, device=w.device)
    ffi.call("castforge_hip_quantize_int4g_hadamard", _ptr(w), n, k, group, block, _ptr(codes), _ptr(scales),
             _ptr(zeros), _stream(w))
    return Int4Packed(codes, scales, zeros, n, k, group)


def smoothquant_scales(act_max: float, w_max: float, alpha: float, bits: int = 8) -> tuple[float, float]:
    """(s, e) of schemes.rs:231-233 with the C library's powf (host arithmetic)."""
    out = (ctypes.c_float * 2)()
    ffi.call("castforge_hip_smoothquant_scales", ctypes.c_float(act_max), ctypes.c_float(w_max),
             ctypes.c_float(alpha), bits, ctypes.addressof(out))
    return float(out[0]), float(out[1])


def smoothquant(w: torch.Tensor, smooth_scale: float, eff_qscale: float, bits: int = 8) -> torch.Tensor:
    """SmoothQuant fake quantization of a float32 tensor with precomputed (s, e)."""
    w = _dev(w)
    if w.dtype != torch.float32:
        raise ValueError("smoothquant takes float32 values")
    out = torch.empty_like(w)
    ffi.call("castforge_hip_smoothquant", _ptr(w), w.numel(), ctypes.c_float(smooth_scale),
             ctypes.c_float(eff_qscale), bits, _ptr(out), _stream(w))
    return out


# ----------------------------------------------------------------------------- GGUF ----
GGML_TYPES = {"F32": ffi.GGML_F32, "F16": ffi.GGML_F16, "Q4_0": ffi.GGML_Q4_0, "Q8_0": ffi.GGML_Q8_0,
              "BF16": ffi.GGML_BF16}


def _ggml(t) -> int:
    if isinstance(t, str):
        if t not in GGML_TYPES:
            raise ValueError(f"unknown GGML type {t!r}")
        return GGML_TYPES[t]
    return int(t)


def gguf_payload_bytes(ggml_type, num_elems: int) -> int:
    """Bytes of a GGUF tensor payload of num_elems elements (gguf.rs:491-550)."""
    out = ctypes.c_int64()
    ffi.call("castforge_hip_gguf_payload_bytes", _ggml(ggml_type), num_elems, ctypes.byref(out))
    return out.value


def gguf_decode(ggml_type, raw: torch.Tensor, num_elems: int) -> torch.Tensor:
    """f32 [num_elems] of a GGUF payload held in a device uint8 tensor (gguf.rs:486-550)."""
    raw = _dev(raw)
    t = _ggml(ggml_type)
    need = gguf_payload_bytes(t, num_elems)
    if raw.dtype != torch.uint8 or raw.numel() < need:
        raise ValueError(f"raw must be a uint8 tensor of at least {need} bytes")
    out = torch.empty(num_elems, dtype=torch.float32, device=raw.device)
    ffi.call("castforge_hip_gguf_decode", t, _ptr(raw), num_elems, _ptr(out), _stream(raw))
    return out


def gguf_encode(ggml_type, src: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """GGUF payload (device uint8) of a tensor: Q8_0 from int8 codes and their one scale
    (gguf.rs:283-296), F16 / BF16 / F32 from float32 values (gguf.rs:298-318)."""
    src = _dev(src)
    t = _ggml(ggml_type)
    n = src.numel()
    if t == ffi.GGML_Q8_0:
        if src.dtype != torch.int8:
            raise ValueError("Q8_0 export takes int8 codes")
        nbytes = (max(n, 1) + 31) // 32 * 34
    else:
        if src.dtype != torch.float32:
            raise ValueError("F32 / F16 / BF16 export takes float32 values")
        nbytes = gguf_payload_bytes(t, n)
    out = torch.empty(nbytes, dtype=torch.uint8, device=src.device)
    ffi.call("castforge_hip_gguf_encode", t, _ptr(src), n, ctypes.c_float(scale), _ptr(out), _stream(src))
    return out


@dataclass
class GgufPacked:
    """GGUF planes of a Q4_0 / Q8_0 matrix [n, k] (blocks of 32 along k): codes uint8
    [n, k/2] (Q4_0) or int8 [n, k] (Q8_0), scales f16 [n, GP]."""
    ggml_type: int
    codes: torch.Tensor
    scales: torch.Tensor
    n: int
    k: int

    def nbytes(self) -> int:
        return self.codes.numel() * self.codes.element_size() + self.scales.numel() * 2

    def payload_bytes(self) -> int:
        return gguf_payload_bytes(self.ggml_type, self.n * self.k)


def gguf_planes_ok(ggml_type, k: int) -> bool:
    t = _ggml(ggml_type)
    return t in (ffi.GGML_Q4_0, ffi.GGML_Q8_0) and k % (128 if t == ffi.GGML_Q4_0 else 64) == 0


def gguf_repack(ggml_type, raw: torch.Tensor, n: int, k: int) -> GgufPacked:
    """Q4_0 / Q8_0 blocks of a row-major [n, k] tensor -> the planes the GEMV reads."""
    raw = _dev(raw)
    t = _ggml(ggml_type)
    if raw.dtype != torch.uint8 or raw.numel() < gguf_payload_bytes(t, n * k):
        raise ValueError("raw must be a uint8 tensor holding the tensor's blocks")
    gp = (k // 32 + 7) // 8 * 8
    codes = torch.empty((n, k // 2 if t == ffi.GGML_Q4_0 else k),
                        dtype=torch.uint8 if t == ffi.GGML_Q4_0 else torch.int8, device=raw.device)
    scales = torch.empty((n, gp), dtype=torch.float16, device=raw.device)
    ffi.call("castforge_hip_gguf_repack", t, _ptr(raw), n, k, _ptr(codes), _ptr(scales), _stream(raw))
    return GgufPacked(t, codes, scales, n, k)


def gguf_unpack(p: GgufPacked) -> torch.Tensor:
    """The block payload (device uint8) of GGUF planes."""
    out = torch.empty(p.payload_bytes(), dtype=torch.uint8, device=p.codes.device)
    ffi.call("castforge_hip_gguf_unpack", p.ggml_type, _ptr(p.codes), _ptr(p.scales), p.n, p.k, _ptr(out),
             _stream(p.codes))
    return out


def dequantize_gguf(p: GgufPacked) -> torch.Tensor:
    out = torch.empty((p.n, p.k), dtype=torch.float32, device=p.codes.device)
    ffi.call("castforge_hip_dequantize_gguf", p.ggml_type, _ptr(p.codes), _ptr(p.scales), p.n, p.k, _ptr(out),
             _stream(p.codes))
    return out


def gguf_q4_0_to_int4g(p: GgufPacked) -> Int4Packed:
    """The INT4g form (group 32, zero point 8) of Q4_0 planes; the scale plane is shared."""
    if p.ggml_type != ffi.GGML_Q4_0:
        raise ValueError("only Q4_0 planes have an INT4g form")
    zw = (p.k // 32 + 7) // 8
    codes = torch.empty((p.n, p.k // 8), dtype=torch.int32, device=p.codes.device)
    zeros = torch.empty((p.n, zw), dtype=torch.int32, device=p.codes.device)
    ffi.call("castforge_hip_gguf_q4_0_to_int4g", _ptr(p.codes), p.n, p.k, _ptr(codes), _ptr(zeros), _stream(p.codes))
    return Int4Packed(codes, p.scales, zeros, p.n, p.k, 32)


def gemm_gguf(x: torch.Tensor, p: GgufPacked, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """y [M, n] = x [M, k] (bf16) times decode(W)^T over GGUF planes (split-K GEMV at M = 1 and
    2, the skinny MFMA kernel up to M = 64 (Q4_0: 32), the prefill MFMA kernel beyond)."""
    x = _check_x(x, p.k)
    y = torch.empty((x.shape[0], p.n), dtype=out_dtype, device=x.device)
    ffi.call("castforge_hip_gemv_gguf", p.ggml_type, _ptr(x), x.shape[0], p.n, p.k, _ptr(p.codes),
             _ptr(p.scales), _ptr(y), _out_dtype(out_dtype), _stream(x))
    return y


def gemv_gguf_batched(xs: list[torch.Tensor], ps: list[GgufPacked], ys: list[torch.Tensor]) -> None:
    """One launch for up to 8 GGUF matrices of one type with the same M (1..64); outputs
    preallocated."""
    if not (len(xs) == len(ps) == len(ys)) or len(ps) > ffi.MAX_BATCH:
        raise ValueError("xs, ps, ys must have the same length <= 8")
    if not ps:
        return
    t = ps[0].ggml_type
    m = xs[0].shape[0]
    if any(p.ggml_type != t for p in ps):
        raise ValueError("problems must share the GGML type and M, with x [M, k] and y [M, n]")
    yd = _check_batch(xs, ys, m, [p.n for p in ps], [p.k for p in ps])
    arr = (ffi.GgufProblem * len(ps))()
    for i, (x, p, y) in enumerate(zip(xs, ps, ys)):
        arr[i] = ffi.GgufProblem(_ptr(x), _ptr(p.codes), _ptr(p.scales), _ptr(y), p.n, p.k)
    ffi.call("castforge_hip_gemv_gguf_batched", t, arr, len(ps), m, yd, _stream(xs[0]))


@dataclass
class Q40Planes:
    """GGUF Q4_0 weights in the Q4_0 GEMV planes layout (castforge_hip_gguf_q4_0_to_gemv_planes):
    codes u8 [T * G * 1024], d f16 [T, G, 16, 4] with T = ceil(n/16), G = k/128."""
    codes: torch.Tensor
    scales: torch.Tensor
    n: int
    k: int

    def nbytes(self) -> int:
        return self.codes.numel() + self.scales.numel() * 2


def gguf_q4_0_to_gemv_planes(p: GgufPacked) -> Q40Planes:
    """The Q4_0 GEMV planes of GGUF Q4_0 planes (built once, at load time)."""
    if p.ggml_type != ffi.GGML_Q4_0 or p.k % 128:
        raise ValueError("Q4_0 GEMV planes hold GGUF Q4_0 matrices with k % 128 == 0")
    t, g = (p.n + 15) // 16, p.k // 128
    dev = p.codes.device
    pl = Q40Planes(torch.empty(t * g * 1024, dtype=torch.uint8, device=dev),
                   torch.empty((t, g, 16, 4), dtype=torch.float16, device=dev), p.n, p.k)
    ffi.call("castforge_hip_gguf_q4_0_to_gemv_planes", _ptr(_dev(p.codes)), _ptr(_dev(p.scales)), p.n, p.k,
             _ptr(pl.codes), _ptr(pl.scales), _stream(p.codes))
    return pl


def gguf_q4_0_from_gemv_planes(pl: Q40Planes) -> GgufPacked:
    """GGUF Q4_0 planes back from Q4_0 GEMV planes (bit for bit)."""
    n, k = pl.n, pl.k
    dev = pl.codes.device
    gp = (k // 32 + 7) // 8 * 8
    p = GgufPacked(ffi.GGML_Q4_0, torch.empty((n, k // 2), dtype=torch.uint8, device=dev),
                   torch.empty((n, gp), dtype=torch.float16, device=dev), n, k)
    ffi.call("castforge_hip_gguf_q4_0_from_gemv_planes", _ptr(_dev(pl.codes)), _ptr(_dev(pl.scales)), n, k,
             _ptr(p.codes), _ptr(p.scales), _stream(pl.codes))
    return p


def gemv_gguf_q4_0_planes_batched(xs: list[torch.Tensor], ps: list[Q40Planes], ys: list[torch.Tensor]) -> None:
    """Q4_0 decode (x of one row) over Q4_0 GEMV planes, all problems in one launch (one
    workgroup per CU)."""
    if not (len(xs) == len(ps) == len(ys)) or not 1 <= len(ps) <= ffi.MAX_BATCH:
        raise ValueError("xs, ps, ys must have the same length in 1..8")
    m = xs[0].shape[0] if xs[0].dim() == 2 else 0
    if m != 1:
        raise ValueError("the Q4_0 planes kernel takes x of one row")
    yd = _check_batch(xs, ys, m, [p.n for p in ps], [p.k for p in ps])
    arr = (ffi.GgufProblem * len(ps))()
    for i, (x, p, y) in enumerate(zip(xs, ps, ys)):
        arr[i] = ffi.GgufProblem(_ptr(x), _ptr(p.codes), _ptr(p.scales), _ptr(y), p.n, p.k)
    ffi.call("castforge_hip_gemv_gguf_q4_0_planes_batched", arr, len(ps), m, yd, _stream(xs[0]))


def gemv_gguf_q4_0_planes(x: torch.Tensor, p: Q40Planes, out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """y [1, n] for x bf16 [1, k] over Q4_0 GEMV planes."""
    y = torch.empty((1, p.n), dtype=out_dtype, device=x.device)
    gemv_gguf_q4_0_planes_batched([x], [p], [y])
    return y


# ------------------------------------------------------------- static W8A8 (calibrate) ----
def static_quantize(x: torch.Tensor, scale: float, bits: int = 8) -> torch.Tensor:
    """castforge.static_quantize (eval.rs:1369-1382): clamp(round(x / scale), +-qmax) * scale
    in f32 with scale already resolved to f32 (> 0); qmax = 7 for bits == 4, else 127."""
    x = _dev(x)
    if x.dtype != torch.float32:
        raise ValueError("static_quantize takes float32 values")
    x = x.contiguous()
    y = torch.empty_like(x)
    ffi.call("castforge_hip_static_quantize", _ptr(x), x.numel(), float(scale), int(bits), _ptr(y), _stream(x))
    return y


def absmax(x: torch.Tensor) -> float:
    """max |x| over the non-NaN elements of a float32 tensor (0.0 when empty)."""
    x = _dev(x)
    if x.dtype != torch.float32:
        raise ValueError("absmax takes float32 values")
    x = x.contiguous()
    out = torch.empty(1, dtype=torch.float32, device=x.device)
    ffi.call("castforge_hip_absmax_f32", _ptr(x), x.numel(), _ptr(out), _stream(x))
    return float(out.item())


# ------------------------------------------------------- reference write-back quantizers ----
def quantize_groupwise(w: torch.Tensor, bits: int = 4, group_size: int = 32, awq_salient: bool = True,
                       salient_ratio: float = 0.01, round: str = "half_away"
                       ) -> tuple[torch.Tensor, torch.Tensor, int]:
    """QuantizeGroupwisePass on one tensor (flattened): returns (dequantized f32 of w's shape,
    group scales f32, salient count)."""
    w = _dev(w)
    if w.dtype != torch.float32:
        raise ValueError("quantize_groupwise takes float32 values")
    n = w.numel()
    gs = max(int(group_size), 2)
    deq = torch.empty_like(w)
    scales = torch.empty(max(1, (n + gs - 1) // gs), dtype=torch.float32, device=w.device)
    ws = torch.empty(ffi.GROUPWISE_WORKSPACE_BYTES // 4, dtype=torch.int32, device=w.device)
    cnt = ctypes.c_int64(0)
    ffi.call("castforge_hip_quantize_groupwise", _ptr(w), n, bits, gs, 1 if awq_salient else 0,
             float(salient_ratio), _ROUND[round], _ptr(deq), _ptr(scales), _ptr(ws), ctypes.byref(cnt),
             _stream(w))
    return deq, scales[: (n + gs - 1) // gs], int(cnt.value)


def quantize_fp8_grid(w: torch.Tensor, fmt: str = "e4m3", mxfp8: bool = True, block_size: int = 32) -> torch.Tensor:
    """QuantizeFp8Pass on one tensor (flattened): dequantized f32 of w's shape."""
    w = _dev(w)
    if w.dtype != torch.float32:
        raise ValueError("quantize_fp8_grid takes float32 values")
    deq = torch.empty_like(w)
    ffi.call("castforge_hip_quantize_fp8_grid", _ptr(w), w.numel(), 1 if fmt.lower() == "e5m2" else 0,
             1 if mxfp8 else 0, int(block_size), _ptr(deq), _stream(w))
    return deq


# ----------------------------------------------------------- around the fused matmul ----
_EPI = {"bias": ffi.EPI_BIAS, "relu": ffi.EPI_RELU, "bias_relu": ffi.EPI_RELU, "tanh": ffi.EPI_TANH,
        "bias_tanh": ffi.EPI_TANH, "silu": ffi.EPI_SILU, "bias_silu": ffi.EPI_SILU, "gelu": ffi.EPI_GELU,
        "bias_gelu": ffi.EPI_GELU, "bias_scale": ffi.EPI_SCALE}


def qmatmul_epilogue(y: torch.Tensor, bias: torch.Tensor, z: torch.Tensor | None = None,
                     epilogue: str = "bias") -> torch.Tensor:
    """In place on f32 y: eval.rs:1151-1176 (unknown epilogue names keep val = mm + bias)."""
    y, bias = _dev(y), _dev(bias)
    if y.dtype != torch.float32 or bias.dtype != torch.float32:
        raise ValueError("epilogue runs on float32 y and bias")
    kind = _EPI.get(epilogue, ffi.EPI_BIAS)
    zl = 0 if z is None else z.numel()
    ffi.call("castforge_hip_qmatmul_epilogue", _ptr(y), y.numel(), _ptr(bias), bias.numel(),
             None if z is None else _ptr(_dev(z)), zl, kind, _stream(y))
    return y


def to_bf16(x: torch.Tensor) -> torch.Tensor:
    """f32 -> bf16 with round-to-nearest-even, on the GPU."""
    x = _dev(x)
    if x.dtype == torch.bfloat16:
        return x
    if x.dtype != torch.float32:
        raise ValueError("to_bf16 takes float32")
    out = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    ffi.call("castforge_hip_convert_f32_to_bf16", _ptr(x), x.numel(), _ptr(out), _stream(x))
    return out


def to_f32(x: torch.Tensor) -> torch.Tensor:
    x = _dev(x)
    if x.dtype == torch.float32:
        return x
    if x.dtype != torch.bfloat16:
        raise ValueError("to_f32 takes bfloat16")
    out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    ffi.call("castforge_hip_convert_bf16_to_f32", _ptr(x), x.numel(), _ptr(out), _stream(x))
    return out


def transpose2d(x: torch.Tensor) -> torch.Tensor:
    """[R, C] -> [C, R] for 1-, 2- or 4-byte elements, on the GPU."""
    x = _dev(x)
    if x.dim() != 2:
        raise ValueError("transpose2d takes a 2-D tensor")
    r, c = x.shape
    out = torch.empty((c, r), dtype=x.dtype, device=x.device)
    ffi.call("castforge_hip_transpose", _ptr(x), r, c, x.element_size(), _ptr(out), _stream(x))
    return out


def matmul_f32(a: torch.Tensor, b: torch.Tensor, packed_rhs: bool = False) -> torch.Tensor:
    """eval_matmul_2d on the GPU (bit-identical order): a [M, K] f32, b [K, N] or packed [N, K]."""
    a, b = _dev(a), _dev(b)
    if a.dtype != torch.float32 or b.dtype != torch.float32 or a.dim() != 2 or b.dim() != 2:
        raise ValueError("matmul_f32 takes 2-D float32 operands")
    m, k = a.shape
    n = b.shape[0] if packed_rhs else b.shape[1]
    if (b.shape[1] if packed_rhs else b.shape[0]) != k:
        raise ValueError("contracting dimensions differ")
    out = torch.empty((m, n), dtype=torch.float32, device=a.device)
    ffi.call("castforge_hip_matmul_f32", _ptr(a), m, k, _ptr(b), n, 1 if packed_rhs else 0, _ptr(out), _stream(a))
    return out
