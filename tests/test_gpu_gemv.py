"""GPU parity of the dequant-fused GEMV / skinny GEMM kernels against the oracle's evaluator
semantics (dequantize to f32, then eval_matmul_2d): |y - ref| <= 1e-3 + 1e-2 * |ref|, the
north-star tolerance for bf16 accumulation."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ops, synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _close(y, ref):
    y = y.float().cpu().numpy()
    err = np.abs(y - ref)
    bound = ATOL + RTOL * np.abs(ref)
    bad = err > bound
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}"


def _x(seed, m, k, dev):
    xb = synth.activations_bf16(seed, 7, m, k)
    return xb, torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)


@pytest.mark.parametrize("m", [1, 2, 8, 16, 17, 33, 64])
@pytest.mark.parametrize("n,k", [(48, 256), (100, 1024), (64, 11008), (4096, 4096)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_w4a16_skinny(cuda, m, n, k, out):
    w = synth.weight(51, 1, n, k)
    codes, scales, zeros = O.quantize_int4g(w, 128)
    xb, x = _x(52, m, k, cuda)
    p = ops.Int4Packed(torch.from_numpy(codes.view(np.int32)).to(cuda),
                       torch.from_numpy(scales.view(np.float16)).to(cuda),
                       torch.from_numpy(zeros.view(np.int32)).to(cuda), n, k, 128)
    y = ops.gemm_w4a16(x, p, out)
    torch.cuda.synchronize()
    _close(y, O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128))


@pytest.mark.parametrize("m,group,k", [(3, 64, 512), (20, 128, 256), (1, 32, 1000), (5, 256, 512)])
def test_w4a16_generic_paths(cuda, m, group, k):
    n = 37
    w = synth.weight(53, 1, n, k)
    xb, x = _x(54, m, k, cuda)
    p = ops.quantize_int4g(torch.from_numpy(w).to(cuda), group)
    y = ops.gemm_w4a16(x, p, torch.float32)
    ref = O.gemm_w4a16(xb, p.codes.cpu().numpy().view(np.uint32), p.scales.cpu().numpy().view(np.uint16),
                       p.zeros.cpu().numpy().view(np.uint32), n, k, group)
    _close(y, ref)


@pytest.mark.parametrize("m", [1, 5, 16, 17, 32, 33])
@pytest.mark.parametrize("gran", ["channel", "tensor"])
@pytest.mark.parametrize("n,k", [(40, 192), (4096, 4096), (33, 11008)])
def test_w8a16(cuda, m, gran, n, k):
    w = synth.weight(61, 1, n, k)
    xb, x = _x(62, m, k, cuda)
    q, s = ops.quantize_int8(torch.from_numpy(w).to(cuda), 8, gran, "half_even")
    y = ops.gemm_w8a16(x, q, s, gran, torch.float32)
    sc = s.cpu().numpy()
    sc = sc if gran == "channel" else np.full(n, sc[0], np.float32)
    _close(y, O.gemm_w8a16(xb, q.cpu().numpy(), sc))


@pytest.mark.parametrize("m", [1, 16, 17, 40, 64])
@pytest.mark.parametrize("block", [64, 32, 16])
def test_nf4(cuda, m, block):
    n, k = 96, 1024
    w = synth.weight(71, 1, n, k)
    xb, x = _x(72, m, k, cuda)
    p = ops.quantize_nf4(torch.from_numpy(w).to(cuda), block)
    y = ops.gemm_nf4(x, p, torch.float32)
    ref = O.gemm_nf4(xb, p.codes.cpu().numpy().view(np.uint32), p.absmax.cpu().numpy(), n, k, block)
    _close(y, ref)


def test_w4a16_batched_block_m1(cuda):
    """The bench's single launch: 7 projections of one LLaMA-7B block at M=1."""
    xs, ps, ys, refs = [], [], [], []
    for tid, (name, n, k) in enumerate(synth.LLAMA7B_BLOCK):
        w = synth.weight(0, tid, n, k)
        codes, scales, zeros = O.quantize_int4g(w, 128)
        xb, x = _x(100 + tid, 1, k, cuda)
        ps.append(ops.Int4Packed(torch.from_numpy(codes.view(np.int32)).to(cuda),
                                 torch.from_numpy(scales.view(np.float16)).to(cuda),
                                 torch.from_numpy(zeros.view(np.int32)).to(cuda), n, k, 128))
        xs.append(x)
        ys.append(torch.empty((1, n), dtype=torch.bfloat16, device=cuda))
        refs.append(O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128))
    ops.gemv_w4a16_batched(xs, ps, ys)
    torch.cuda.synchronize()
    for y, ref in zip(ys, refs):
        _close(y, ref)


def test_empty_and_degenerate(cuda):
    p = ops.quantize_int4g(torch.zeros((0, 256), device=cuda), 128)
    x = torch.zeros((1, 256), dtype=torch.bfloat16, device=cuda)
    assert ops.gemm_w4a16(x, p).shape == (1, 0)
    w = torch.zeros((16, 256), device=cuda)
    p = ops.quantize_int4g(w, 128)
    y = ops.gemm_w4a16(torch.ones((1, 256), dtype=torch.bfloat16, device=cuda), p, torch.float32)
    assert torch.all(y == 0)


@pytest.mark.parametrize("gran", ["channel", "tensor"])
@pytest.mark.parametrize("m", [1, 4])
def test_w8a16_batched(cuda, gran, m):
    """One launch over several INT8 problems: same bits as one call per problem, oracle tolerance."""
    shapes = [(40, 192), (4096, 4096), (33, 11008), (100, 64)]
    xs, qs, ys, singles, refs = [], [], [], [], []
    for i, (n, k) in enumerate(shapes):
        w = synth.weight(400 + i, 1, n, k)
        xb, x = _x(410 + i, m, k, cuda)
        q, s = ops.quantize_int8(torch.from_numpy(w).to(cuda), 8, gran, "half_even")
        xs.append(x)
        qs.append((q, s))
        ys.append(torch.empty((m, n), dtype=torch.float32, device=cuda))
        singles.append(ops.gemm_w8a16(x, q, s, gran, torch.float32))
        sc = s.cpu().numpy()
        refs.append(O.gemm_w8a16(xb, q.cpu().numpy(), sc if gran == "channel" else np.full(n, sc[0], np.float32)))
    ops.gemv_w8a16_batched(xs, qs, ys, gran)
    for y, y1, ref in zip(ys, singles, refs):
        assert torch.equal(y, y1)
        _close(y, ref)


@pytest.mark.parametrize("block", [64, 32])
def test_nf4_batched(cuda, block):
    shapes = [(96, 1024), (11008, 4096), (4096, 11008), (7, 512)]
    xs, ps, ys, singles, refs = [], [], [], [], []
    for i, (n, k) in enumerate(shapes):
        w = synth.weight(420 + i, 1, n, k)
        xb, x = _x(430 + i, 1, k, cuda)
        p = ops.quantize_nf4(torch.from_numpy(w).to(cuda), block)
        xs.append(x)
        ps.append(p)
        ys.append(torch.empty((1, n), dtype=torch.float32, device=cuda))
        singles.append(ops.gemm_nf4(x, p, torch.float32))
        refs.append(O.gemm_nf4(xb, p.codes.cpu().numpy().view(np.uint32), p.absmax.cpu().numpy(), n, k, block))
    ops.gemv_nf4_batched(xs, ps, ys)
    for y, y1, ref in zip(ys, singles, refs):
        assert torch.equal(y, y1)
        _close(y, ref)


@pytest.mark.parametrize("fmt", ["int4", "int8", "nf4"])
@pytest.mark.parametrize("m", [17, 40, 64])
def test_batched_mid_m(cuda, fmt, m):
    """M = 17..64 in one batched launch (x tiles of 16 rows sharing each decoded weight word):
    within tolerance of the oracle, and equal to one call per problem wherever that call runs
    the same kernel (INT8 single calls above M = 32 run the prefill kernel)."""
    shapes = [(96, 1024), (300, 2048), (64, 4096), (7, 512)]
    xs, ps, ys, refs = [], [], [], []
    for i, (n, k) in enumerate(shapes):
        w = torch.from_numpy(synth.weight(700 + i, 1, n, k)).to(cuda)
        xb, x = _x(710 + i, m, k, cuda)
        xs.append(x)
        ys.append(torch.empty((m, n), dtype=torch.float32, device=cuda))
        if fmt == "int4":
            p = ops.quantize_int4g(w, 128)
            refs.append(O.gemm_w4a16(xb, p.codes.cpu().numpy().view(np.uint32), p.scales.cpu().numpy().view(np.uint16),
                                     p.zeros.cpu().numpy().view(np.uint32), n, k, 128))
        elif fmt == "int8":
            p = ops.quantize_int8(w, 8, "channel", "half_even")
            refs.append(O.gemm_w8a16(xb, p[0].cpu().numpy(), p[1].cpu().numpy()))
        else:
            p = ops.quantize_nf4(w, 64)
            refs.append(O.gemm_nf4(xb, p.codes.cpu().numpy().view(np.uint32), p.absmax.cpu().numpy(), n, k, 64))
        ps.append(p)
    if fmt == "int4":
        ops.gemv_w4a16_batched(xs, ps, ys)
        singles = [ops.gemm_w4a16(x, p, torch.float32) for x, p in zip(xs, ps)]
    elif fmt == "int8":
        ops.gemv_w8a16_batched(xs, ps, ys, "channel")
        singles = [ops.gemm_w8a16(x, q, s, "channel", torch.float32) for x, (q, s) in zip(xs, ps)]
    else:
        ops.gemv_nf4_batched(xs, ps, ys)
        singles = [ops.gemm_nf4(x, p, torch.float32) for x, p in zip(xs, ps)]
    for y, y1, ref in zip(ys, singles, refs):
        if not (fmt == "int8" and m > 32):
            assert torch.equal(y, y1)
        _close(y, ref)
        _close(y1, ref)


def test_nf4_batched_rejects_mixed_blocks(cuda):
    ps = [ops.quantize_nf4(torch.zeros((16, 256), device=cuda), b) for b in (64, 32)]
    xs = [torch.zeros((1, 256), dtype=torch.bfloat16, device=cuda)] * 2
    ys = [torch.empty((1, 16), dtype=torch.float32, device=cuda) for _ in ps]
    with pytest.raises(Exception, match="block size"):
        ops.gemv_nf4_batched(xs, ps, ys)


def test_batched_wrappers_reject_mixed_or_strided_outputs(cuda):
    """Every batched wrapper validates each y (one dtype for the batch, contiguous, [M, n], on
    x's device) before the launch: the C ABI takes a single y_dtype, so a bf16 y after an f32
    one would be written 4 bytes per element."""
    n, k = 32, 256
    w = torch.from_numpy(synth.weight(5, 1, n, k)).to(cuda)
    x = torch.zeros((1, k), dtype=torch.bfloat16, device=cuda)
    p4 = ops.quantize_int4g(w, 128)
    q8 = ops.quantize_int8(w, 8, "channel", "half_even")
    nf = ops.quantize_nf4(w, 64)
    f32y = lambda: torch.empty((1, n), dtype=torch.float32, device=cuda)  # noqa: E731
    bad_sets = [
        ([f32y(), torch.empty((1, n), dtype=torch.bfloat16, device=cuda)], "one dtype"),
        ([f32y(), torch.empty((1, 2 * n), dtype=torch.float32, device=cuda)[:, ::2]], "contiguous"),
        ([f32y(), torch.empty((1, n + 1), dtype=torch.float32, device=cuda)], r"\[M, n\]"),
    ]
    calls = [
        lambda ys: ops.gemv_w4a16_batched([x, x], [p4, p4], ys),
        lambda ys: ops.gemv_w8a16_batched([x, x], [q8, q8], ys, "channel"),
        lambda ys: ops.gemv_nf4_batched([x, x], [nf, nf], ys),
    ]
    for call in calls:
        for ys, msg in bad_sets:
            with pytest.raises(ValueError, match=msg):
                call(ys)
        ys = [f32y(), f32y()]
        call(ys)  # a valid batch still runs
    torch.cuda.synchronize()
