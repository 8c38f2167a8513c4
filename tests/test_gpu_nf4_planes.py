"""NF4 GEMV planes (castforge_hip_nf4_to_planes / from_planes / gemv_nf4_planes_batched).

* Layout: the planes equal the header's definition written out with numpy reshapes, and
  from_planes restores the canonical codes and absmax bit for bit (blocks 32 .. 256, ragged N).
* Numerics: M = 1 against the oracle's f32 loop (`orc_gemm_nf4`, eval.rs:1465-1507 over the NF4
  dequant) within the north-star 1e-2 relative / 1e-3 absolute, for every block size, f32 and
  bf16 outputs, single matrices and the batched LLaMA-7B MLP (W_gate, W_up, W_down of config 3).
* Activation range: y(2^e x) = 2^e y(x) bit for bit for e = -100..100; rows with |x| up to 3e6,
  a chunk of tiny values and a chunk of bf16 subnormals against the oracle; non-finite x gives
  non-finite rows.
* Outputs that cancel exactly: x = [v, -v] against weights whose halves are equal.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ffi, ops, synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3
MLP = [s for s in synth.LLAMA7B_BLOCK if s[0] in ("w_gate", "w_up", "w_down")]


def _xdev(xb, dev):
    return torch.from_numpy(np.ascontiguousarray(xb).view(np.int16)).view(torch.bfloat16).to(dev)


def _close(y, ref):
    y = y.float().cpu().numpy().reshape(ref.shape)
    err = np.abs(y - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}"


def _packed(w, block, dev):
    p = ops.quantize_nf4(torch.from_numpy(w).to(dev), block)
    return p, p.codes.cpu().numpy().view(np.uint32), p.absmax.cpu().numpy()


def _planes_numpy(codes, absmax, n, k, block):
    """The NF4 planes layout written out with numpy reshapes (the header's definition)."""
    g, t = k // 128, (n + 15) // 16
    c = np.zeros((t * 16, k // 8), np.uint32)
    c[:n] = codes
    # row words of chunk g: index 4 q + p  ->  [t, r, g, q, p] -> [t, g, p, r, q]
    pc = c.reshape(t, 16, g, 4, 4).transpose(0, 2, 4, 1, 3).reshape(-1).view(np.uint8)
    nbpc = max(1, 128 // block)
    a = np.zeros((t * 16, g, nbpc), np.float32)
    for gg in range(g):
        for j in range(nbpc):
            blk = gg * nbpc + j if block < 128 else gg * 128 // block
            a[:n, gg, j] = absmax[:, blk]
    pa = a.reshape(t, 16, g, nbpc).transpose(0, 2, 1, 3).copy()
    return pc, pa


@pytest.mark.parametrize("n,k,block", [(48, 256, 64), (100, 1024, 32), (7, 128, 128), (50, 512, 256),
                                       (33, 384, 256), (4096, 11008, 64), (11008, 4096, 64)])
def test_nf4_planes_layout_and_round_trip(cuda, n, k, block):
    w = synth.weight(161, 2, n, k)
    p, codes, absmax = _packed(w, block, cuda)
    pl = ops.nf4_to_planes(p)
    back = ops.nf4_from_planes(pl)
    torch.cuda.synchronize()
    pc, pa = _planes_numpy(codes, absmax, n, k, block)
    assert np.array_equal(pl.codes.cpu().numpy(), pc)
    assert np.array_equal(pl.absmax.cpu().numpy().view(np.uint32), pa.view(np.uint32))
    assert np.array_equal(back.codes.cpu().numpy().view(np.uint32), codes)
    assert np.array_equal(back.absmax.cpu().numpy().view(np.uint32), absmax.view(np.uint32))


@pytest.mark.parametrize("block", [32, 64, 128, 256])
@pytest.mark.parametrize("n,k", [(48, 256), (100, 1024), (7, 128), (4097, 4096), (64, 11008)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_nf4_planes_gemv_matches_oracle(cuda, block, n, k, out):
    w = synth.weight(162, 1, n, k)
    p, codes, absmax = _packed(w, block, cuda)
    pl = ops.nf4_to_planes(p)
    xb = synth.activations_bf16(163, 7, 1, k)
    y = ops.gemv_nf4_planes(_xdev(xb, cuda), pl, out)
    torch.cuda.synchronize()
    ref = O.gemm_nf4(xb, codes, absmax, n, k, block)
    if out == torch.bfloat16:
        ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref))
    _close(y, ref)


@pytest.mark.parametrize("shared_x", [True, False])
def test_nf4_planes_llama_mlp_batched(cuda, shared_x):
    """W_gate, W_up, W_down of a LLaMA-7B block (config 3, NF4 block 64) in one launch, every row
    against the oracle and against the canonical-layout batched kernel; a second launch gives
    the same bits."""
    xs_h, xs, pls, ps, ys, refs = {}, [], [], [], [], []
    for tid, (name, n, k) in enumerate(MLP):
        w = synth.weight(170 + tid, 1, n, k)
        p, codes, absmax = _packed(w, 64, cuda)
        ps.append(p)
        pls.append(ops.nf4_to_planes(p))
        key = "gate_up" if shared_x and name in ("w_gate", "w_up") else name
        if key not in xs_h:
            xb = synth.activations_bf16(180 + len(xs_h), 7, 1, k)
            xs_h[key] = (xb, _xdev(xb, cuda))
        xb, x = xs_h[key]
        xs.append(x)
        ys.append(torch.empty((1, n), dtype=torch.float32, device=cuda))
        refs.append(O.gemm_nf4(xb, codes, absmax, n, k, 64))
    ops.gemv_nf4_planes_batched(xs, pls, ys)
    canon = [torch.empty_like(y) for y in ys]
    ops.gemv_nf4_batched(xs, ps, canon)
    torch.cuda.synchronize()
    for y, c, ref in zip(ys, canon, refs):
        _close(y, ref)
        _close(y, c.cpu().numpy())
    ys2 = [torch.empty_like(y) for y in ys]
    ops.gemv_nf4_planes_batched(xs, pls, ys2)
    for y, y2 in zip(ys, ys2):
        assert torch.equal(y, y2)


@pytest.mark.parametrize("block", [32, 64, 256])
def test_nf4_planes_power_of_two_scale_invariance(cuda, block):
    """y(2^e x) == 2^e y(x) bit for bit, e in -100..100 (|x| beyond f16's range and below its
    subnormals: each chunk of x is pre-scaled by its own power of two)."""
    n, k = 200, 2048
    w = synth.weight(164, 1, n, k)
    p, codes, absmax = _packed(w, block, cuda)
    pl = ops.nf4_to_planes(p)
    xb = synth.activations_bf16(165, 7, 1, k)
    x32 = O.bf16_bits_to_f32(xb)
    y0 = ops.gemv_nf4_planes(_xdev(xb, cuda), pl, torch.float32).cpu().numpy()
    _close(torch.from_numpy(y0), O.gemm_nf4(xb, codes, absmax, n, k, block))
    for e in (-100, -30, -10, 5, 16, 20, 60, 100):
        xe = O.f32_to_bf16_bits((x32 * np.float32(2.0 ** e)).astype(np.float32))
        assert np.array_equal(O.bf16_bits_to_f32(xe), (x32 * np.float32(2.0 ** e)).astype(np.float32))
        ye = ops.gemv_nf4_planes(_xdev(xe, cuda), pl, torch.float32).cpu().numpy()
        assert np.all(np.isfinite(ye)), e
        assert np.array_equal(ye, (y0.astype(np.float64) * 2.0 ** e).astype(np.float32)), e


def test_nf4_planes_large_and_tiny_activations_vs_oracle(cuda):
    """Rows with |x| up to 3e6, a chunk of values near 1e-6 and a chunk of bf16 subnormals,
    against the oracle's f32 loop, except rows whose output cancels so far that the oracle's own
    sequential sum is off the exact (f64) value by more than 1e-3; there the row must be no
    further from the exact value than the oracle is, plus the plain bound."""
    n, k = 256, 4096
    w = synth.weight(166, 1, n, k)
    p, codes, absmax = _packed(w, 64, cuda)
    pl = ops.nf4_to_planes(p)
    rng = np.random.default_rng(167)
    x = rng.standard_normal(k).astype(np.float32)
    idx = rng.choice(k, 60, replace=False)
    x[idx] *= rng.choice([1e3, 6e4, 1e5, 3e6], 60).astype(np.float32)
    x[1024:1152] *= np.float32(1e-6)
    x[2048:2176] = np.float32(2.0 ** -130)
    xb = O.f32_to_bf16_bits(x).reshape(1, k)
    y = ops.gemv_nf4_planes(_xdev(xb, cuda), pl, torch.float32).cpu().numpy().reshape(-1)
    ref = O.gemm_nf4(xb, codes, absmax, n, k, 64).reshape(-1)
    deq = O.dequantize_nf4(codes, absmax, n, k, 64).astype(np.float64)
    exact = deq @ O.bf16_bits_to_f32(xb).reshape(-1).astype(np.float64)
    ref_err = np.abs(ref - exact)
    plain = np.abs(y - ref) <= ATOL + RTOL * np.abs(ref)
    assert np.all(plain | (ref_err > ATOL)), np.flatnonzero(~plain & (ref_err <= ATOL))
    assert np.all(np.abs(y - exact) <= ATOL + RTOL * np.abs(exact) + ref_err)


def test_nf4_planes_exact_cancellation(cuda):
    """x = [v, -v] with |v| up to 6e4 against weights whose two K halves are equal: the exact
    answer is 0 for every row.  Every row must be within the plain bound of 0 plus 2^-22 of the
    row's sum of |x w|, and no further from 0 than the oracle's own sequential f32 result."""
    n, kh = 96, 2048
    rng = np.random.default_rng(168)
    wh = (rng.standard_normal((n, kh)) * 0.02).astype(np.float32)
    w = np.concatenate([wh, wh], axis=1)
    p, codes, absmax = _packed(w, 64, cuda)
    pl = ops.nf4_to_planes(p)
    v = rng.standard_normal(kh).astype(np.float32)
    v[rng.choice(kh, 40, replace=False)] *= np.float32(6e4)
    xb = O.f32_to_bf16_bits(np.concatenate([v, -v])).reshape(1, 2 * kh)
    y = ops.gemv_nf4_planes(_xdev(xb, cuda), pl, torch.float32).cpu().numpy()
    ref = O.gemm_nf4(xb, codes, absmax, n, 2 * kh, 64).reshape(1, n)
    mag = np.abs(O.bf16_bits_to_f32(xb).astype(np.float64)) @ \
        np.abs(O.dequantize_nf4(codes, absmax, n, 2 * kh, 64).astype(np.float64)).T
    assert np.all(np.abs(y) <= ATOL + 2.0 ** -22 * mag), (np.abs(y).max(), np.abs(ref).max())
    assert np.abs(y).max() <= np.abs(ref).max()


def test_nf4_planes_nonfinite_x_gives_nonfinite_rows(cuda):
    n, k = 32, 256
    p, _, _ = _packed(synth.weight(169, 1, n, k), 64, cuda)
    pl = ops.nf4_to_planes(p)
    x = np.zeros(k, np.float32)
    x[5] = np.inf
    y = ops.gemv_nf4_planes(_xdev(O.f32_to_bf16_bits(x).reshape(1, k), cuda), pl, torch.float32)
    assert not torch.isfinite(y).any()


def test_nf4_planes_rejects_bad_arguments(cuda):
    w = torch.from_numpy(synth.weight(5, 1, 32, 256)).to(cuda)
    pl = ops.nf4_to_planes(ops.quantize_nf4(w, 64))
    x = torch.zeros((2, 256), dtype=torch.bfloat16, device=cuda)
    y = torch.empty((2, 32), dtype=torch.float32, device=cuda)
    arr = (ffi.Nf4Problem * 2)()
    arr[0] = ffi.Nf4Problem(x.data_ptr(), pl.codes.data_ptr(), pl.absmax.data_ptr(), y.data_ptr(), 32, 256, 64)
    with pytest.raises(ffi.CastForgeHipError, match="M = 1"):
        ffi.call("castforge_hip_gemv_nf4_planes_batched", arr, 1, 2, ffi.DTYPE_F32, None)
    with pytest.raises(ValueError, match="one row"):
        ops.gemv_nf4_planes(x, pl)
    arr[1] = ffi.Nf4Problem(x.data_ptr(), pl.codes.data_ptr(), pl.absmax.data_ptr(), y.data_ptr(), 32, 256, 32)
    with pytest.raises(ffi.CastForgeHipError, match="same NF4 block"):
        ffi.call("castforge_hip_gemv_nf4_planes_batched", arr, 2, 1, ffi.DTYPE_F32, None)
    arr[0].block = 48
    with pytest.raises(ffi.CastForgeHipError, match="power of two"):
        ffi.call("castforge_hip_gemv_nf4_planes_batched", arr, 1, 1, ffi.DTYPE_F32, None)
    with pytest.raises(ValueError, match="k % 128"):
        ops.nf4_to_planes(ops.quantize_nf4(torch.zeros((16, 192), device=cuda), 64))
    # the activations must fit LDS next to the 64 KB decode table (k = 49152: 96 KB of f16 x)
    big = torch.zeros((1, 49152), dtype=torch.bfloat16, device=cuda)
    plb = ops.nf4_to_planes(ops.quantize_nf4(torch.zeros((16, 49152), device=cuda), 64))
    with pytest.raises(ffi.CastForgeHipError, match="LDS"):
        ops.gemv_nf4_planes_batched([big], [plb], [torch.empty((1, 16), device=cuda)])
    torch.cuda.synchronize()
