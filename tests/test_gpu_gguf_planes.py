"""Q4_0 GEMV planes (castforge_hip_gguf_q4_0_to_gemv_planes / from_gemv_planes /
gemv_gguf_q4_0_planes_batched).

* Layout: the planes equal the header's definition written out with numpy reshapes, and
  from_gemv_planes restores the GGUF planes (pad d slots included) bit for bit.
* Numerics: M = 1 as the reference evaluates a GGUF weight (decode to f32, gguf.rs:513-550, then
  the f32 matmul loop of eval.rs:1465-1507) within |y - ref| <= 1e-3 + 1e-2 |ref|; the batched
  LLaMA-7B block against a torch fp32 matmul over the decoded weights and against the
  canonical-planes kernel; blocks with subnormal, zero, negative and largest-finite d.
* Activation range: y(2^e x) = 2^e y(x) bit for bit for e = -100..100.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ffi, ops, synth

pytestmark = pytest.mark.gpu

Q4_0 = 2
RTOL, ATOL = 1e-2, 1e-3
BLOCK = synth.LLAMA7B_BLOCK


def _blocks(nblocks, seed, special=False):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, nblocks * 18, dtype=np.uint8).reshape(nblocks, 18)
    d = (rng.standard_normal(nblocks) * 0.01).astype(np.float16)
    if special:  # subnormal, zero, -0, negative, largest finite
        sp = np.array([0x0001, 0x03FF, 0x0000, 0x8000, 0xBC00, 0x7BFF], np.uint16)
        d[:sp.size] = sp.view(np.float16)
    raw[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
    return raw.reshape(-1)


def _dev_u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8)).to(dev)


def _x(seed, k, dev):
    xb = synth.activations_bf16(seed, 7, 1, k)
    return xb, torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)


def _close(y, ref):
    y = y.float().cpu().numpy().reshape(ref.shape)
    err = np.abs(y - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}"


def _planes_numpy(codes, scales, n, k):
    """The Q4_0 GEMV planes written out with numpy reshapes (the header's definition)."""
    g, t = k // 128, (n + 15) // 16
    c = np.zeros((t * 16, k // 2), np.uint8)
    c[:n] = codes
    # row bytes: [g, part p, 16 B] -> [t, r, g, p, 16] -> [t, g, p, r, 16]
    pc = c.reshape(t, 16, g, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)
    d = np.zeros((t * 16, 4 * g), np.uint16)
    d[:n] = scales[:, :4 * g]
    pd = d.reshape(t, 16, g, 4).transpose(0, 2, 1, 3).copy()
    return pc, pd


@pytest.mark.parametrize("n,k", [(48, 256), (100, 1024), (7, 128), (33, 384), (4096, 11008), (11008, 4096)])
def test_q40_planes_layout_and_round_trip(cuda, n, k):
    raw = _blocks(n * k // 32, 600 + n + k)
    p = ops.gguf_repack(Q4_0, _dev_u8(raw, cuda), n, k)
    pl = ops.gguf_q4_0_to_gemv_planes(p)
    back = ops.gguf_q4_0_from_gemv_planes(pl)
    torch.cuda.synchronize()
    codes, scales = p.codes.cpu().numpy(), p.scales.cpu().numpy().view(np.uint16)
    pc, pd = _planes_numpy(codes, scales, n, k)
    assert np.array_equal(pl.codes.cpu().numpy(), pc)
    assert np.array_equal(pl.scales.cpu().numpy().view(np.uint16), pd)
    assert np.array_equal(back.codes.cpu().numpy(), codes)
    assert np.array_equal(back.scales.cpu().numpy().view(np.uint16), scales)


@pytest.mark.parametrize("n,k", [(48, 256), (100, 1024), (7, 128), (4097, 4096), (64, 11008)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("special", [False, True])
def test_q40_planes_gemv_matches_oracle(cuda, n, k, out, special):
    raw = _blocks(n * k // 32, 610 + n + k, special)
    p = ops.gguf_repack(Q4_0, _dev_u8(raw, cuda), n, k)
    pl = ops.gguf_q4_0_to_gemv_planes(p)
    xb, x = _x(611, k, cuda)
    y = ops.gemv_gguf_q4_0_planes(x, pl, out)
    torch.cuda.synchronize()
    w = O.gguf_decode(Q4_0, raw, n * k).reshape(n, k)
    ref = O.matmul_2d(O.bf16_bits_to_f32(xb.reshape(1, k)), w, packed_rhs=True)
    if out == torch.bfloat16:
        ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref))
    _close(y, ref)


def test_q40_planes_llama_block_batched(cuda):
    """The 7 projections of a LLaMA-7B block as Q4_0 in one launch: every row within the
    north-star bound of a torch fp32 matmul over the decoded weights (the oracle's decode), and
    of the canonical GGUF-planes kernel; a second launch gives the same bits."""
    xs, pls, ps, ys, refs = [], [], [], [], []
    for tid, (name, n, k) in enumerate(BLOCK):
        raw = _blocks(n * k // 32, 620 + tid)
        p = ops.gguf_repack(Q4_0, _dev_u8(raw, cuda), n, k)
        ps.append(p)
        pls.append(ops.gguf_q4_0_to_gemv_planes(p))
        xb, x = _x(630 + tid, k, cuda)
        xs.append(x)
        ys.append(torch.empty((1, n), dtype=torch.float32, device=cuda))
        w = torch.from_numpy(O.gguf_decode(Q4_0, raw, n * k).reshape(n, k)).to(cuda)
        refs.append((x.float() @ w.T).cpu().numpy())
    ops.gemv_gguf_q4_0_planes_batched(xs, pls, ys)
    canon = [torch.empty_like(y) for y in ys]
    ops.gemv_gguf_batched(xs, ps, canon)
    torch.cuda.synchronize()
    for y, c, ref in zip(ys, canon, refs):
        _close(y, ref)
        _close(y, c.cpu().numpy())
    ys2 = [torch.empty_like(y) for y in ys]
    ops.gemv_gguf_q4_0_planes_batched(xs, pls, ys2)
    for y, y2 in zip(ys, ys2):
        assert torch.equal(y, y2)


def test_q40_planes_power_of_two_scale_invariance(cuda):
    n, k = 200, 2048
    raw = _blocks(n * k // 32, 640)
    pl = ops.gguf_q4_0_to_gemv_planes(ops.gguf_repack(Q4_0, _dev_u8(raw, cuda), n, k))
    xb, x = _x(641, k, cuda)
    x32 = O.bf16_bits_to_f32(xb)
    y0 = ops.gemv_gguf_q4_0_planes(x, pl, torch.float32).cpu().numpy()
    for e in (-100, -30, -10, 5, 16, 20, 60, 100):
        xe = O.f32_to_bf16_bits((x32 * np.float32(2.0 ** e)).astype(np.float32))
        assert np.array_equal(O.bf16_bits_to_f32(xe), (x32 * np.float32(2.0 ** e)).astype(np.float32))
        xd = torch.from_numpy(xe.view(np.int16)).view(torch.bfloat16).to(cuda)
        ye = ops.gemv_gguf_q4_0_planes(xd, pl, torch.float32).cpu().numpy()
        assert np.all(np.isfinite(ye)), e
        assert np.array_equal(ye, (y0.astype(np.float64) * 2.0 ** e).astype(np.float32)), e


def test_q40_planes_rejects_bad_arguments(cuda):
    n, k = 32, 256
    p = ops.gguf_repack(Q4_0, _dev_u8(_blocks(n * k // 32, 650), cuda), n, k)
    pl = ops.gguf_q4_0_to_gemv_planes(p)
    x = torch.zeros((2, k), dtype=torch.bfloat16, device=cuda)
    y = torch.empty((2, n), dtype=torch.float32, device=cuda)
    arr = (ffi.GgufProblem * 1)()
    arr[0] = ffi.GgufProblem(x.data_ptr(), pl.codes.data_ptr(), pl.scales.data_ptr(), y.data_ptr(), n, k)
    with pytest.raises(ffi.CastForgeHipError, match="M = 1"):
        ffi.call("castforge_hip_gemv_gguf_q4_0_planes_batched", arr, 1, 2, ffi.DTYPE_F32, None)
    with pytest.raises(ValueError, match="one row"):
        ops.gemv_gguf_q4_0_planes(x, pl)
    q8 = ops.gguf_repack(8, _dev_u8(np.zeros(n * k // 32 * 34, np.uint8), cuda), n, k)
    with pytest.raises(ValueError, match="Q4_0"):
        ops.gguf_q4_0_to_gemv_planes(q8)
    # x must fit LDS (k = 81920: 160 KB of f16)
    kb = 81920
    pb = ops.gguf_repack(Q4_0, _dev_u8(np.zeros(16 * kb // 32 * 18, np.uint8), cuda), 16, kb)
    plb = ops.gguf_q4_0_to_gemv_planes(pb)
    with pytest.raises(ffi.CastForgeHipError, match="LDS"):
        ops.gemv_gguf_q4_0_planes_batched([torch.zeros((1, kb), dtype=torch.bfloat16, device=cuda)], [plb],
                                          [torch.empty((1, 16), device=cuda)])
    torch.cuda.synchronize()
