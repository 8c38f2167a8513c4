"""GEMV planes: the INT4 g128 layout the decode kernels (M = 1..16) stream, and those kernels.

* The planes equal a numpy construction from the canonical arrays and convert back bit for bit.
* y matches the oracle's evaluator semantics (dequantize, then eval_matmul_2d, eval.rs:1465-1507)
  within |y - ref| <= 1e-3 + 1e-2 |ref|.
* Activations of any finite bf16 magnitude: the kernel brings each 128-value chunk of x into
  f16 range by a power of two and undoes it on the f32 partial, so y(2^e x) = 2^e y(x) bit for
  bit (in f32 output) across e = -100..100; x beyond f16's 65504 gives finite, correct rows.
* Outputs that cancel exactly: x = [v, -v] against weights whose halves are equal has the exact
  answer 0 with |v| up to 6e4.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ffi, ops, synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3
BLOCK = synth.LLAMA7B_BLOCK


def _packed(w, dev):
    codes, scales, zeros = O.quantize_int4g(w, 128)
    n, k = w.shape
    p = ops.Int4Packed(torch.from_numpy(codes.view(np.int32)).to(dev),
                       torch.from_numpy(scales.view(np.float16)).to(dev),
                       torch.from_numpy(zeros.view(np.int32)).to(dev), n, k, 128)
    return p, (codes, scales, zeros)


def _xdev(xb, dev):
    return torch.from_numpy(np.ascontiguousarray(xb).view(np.int16)).view(torch.bfloat16).to(dev)


def _close(y, ref):
    y = y.float().cpu().numpy().reshape(ref.shape)
    err = np.abs(y - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}"


def _planes_numpy(codes, scales, zeros, n, k):
    """The planes layout written out with numpy reshapes (the header's definition)."""
    g = k // 128
    t = (n + 15) // 16
    c = np.zeros((t * 16, k // 8), np.uint32)
    c[:n] = codes
    # [t, r, g, p, 4 words] -> [t, g, p, r, 4 words]
    pc = c.reshape(t, 16, g, 4, 4).transpose(0, 2, 3, 1, 4).reshape(-1).view(np.uint8)
    s = np.zeros((t * 16, g), np.uint16)
    s[:n] = scales[:, :g]
    ps = s.reshape(t, 16, g).transpose(0, 2, 1).copy()
    z = np.zeros((t * 16, g), np.uint8)
    zz = np.stack([(zeros[:, j // 8] >> (4 * (j % 8))) & 15 for j in range(g)], axis=1).astype(np.uint8)
    z[:n] = zz
    z = z.reshape(t, 16, g).transpose(0, 2, 1)
    pz = (z[:, :, 0::2] | (z[:, :, 1::2] << 4)).astype(np.uint8)
    return pc, ps, pz


@pytest.mark.parametrize("n,k", [(48, 256), (100, 1024), (7, 128), (4096, 11008), (11008, 4096)])
def test_planes_layout_and_round_trip(cuda, n, k):
    w = synth.weight(61, 2, n, k)
    p, (codes, scales, zeros) = _packed(w, cuda)
    pl = ops.int4g_to_planes(p)
    back = ops.int4g_from_planes(pl)
    torch.cuda.synchronize()
    pc, ps, pz = _planes_numpy(codes, scales, zeros, n, k)
    assert np.array_equal(pl.codes.cpu().numpy(), pc)
    assert np.array_equal(pl.scales.cpu().numpy().view(np.uint16), ps)
    assert np.array_equal(pl.zeros.cpu().numpy(), pz)
    assert np.array_equal(back.codes.cpu().numpy().view(np.uint32), codes)
    assert np.array_equal(back.scales.cpu().numpy().view(np.uint16), scales)
    assert np.array_equal(back.zeros.cpu().numpy().view(np.uint32), zeros)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 8, 9, 12, 16])
@pytest.mark.parametrize("n,k", [(48, 256), (100, 1024), (7, 128), (4097, 4096), (64, 11008), (4096, 4096)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_planes_gemv_matches_oracle(cuda, m, n, k, out):
    w = synth.weight(62, 1, n, k)
    p, (codes, scales, zeros) = _packed(w, cuda)
    pl = ops.int4g_to_planes(p)
    xb = synth.activations_bf16(63, 7, m, k)
    y = ops.gemv_w4a16_planes(_xdev(xb, cuda), pl, out)
    torch.cuda.synchronize()
    ref = O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128)
    if out == torch.bfloat16:
        ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref))
    _close(y, ref)


@pytest.mark.parametrize("m", [1, 4, 5, 8, 16])
@pytest.mark.parametrize("shared_x", [True, False])
def test_planes_llama_block_batched(cuda, shared_x, m):
    """The 7 projections of a LLaMA-7B block in one launch (x shared by q/k/v and by gate/up as in
    a decoder, or 7 distinct x); every row against the oracle."""
    xs_h, xs, pls, ys, refs = {}, [], [], [], []
    for tid, (name, n, k) in enumerate(BLOCK):
        w = synth.weight(70 + tid, 1, n, k)
        p, (codes, scales, zeros) = _packed(w, cuda)
        pls.append(ops.int4g_to_planes(p))
        key = name
        if shared_x and name in ("wq", "wk", "wv"):
            key = "qkv"
        elif shared_x and name in ("w_gate", "w_up"):
            key = "gate_up"
        if key not in xs_h:
            xb = synth.activations_bf16(80 + len(xs_h), 7, m, k)
            xs_h[key] = (xb, _xdev(xb, cuda))
        xb, x = xs_h[key]
        xs.append(x)
        ys.append(torch.empty((m, n), dtype=torch.float32, device=cuda))
        refs.append(O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128))
    ops.gemv_w4a16_planes_batched(xs, pls, ys)
    torch.cuda.synchronize()
    for y, ref in zip(ys, refs):
        _close(y, ref)
    # the same launch again gives the same bits (no state kept between calls)
    ys2 = [torch.empty_like(y) for y in ys]
    ops.gemv_w4a16_planes_batched(xs, pls, ys2)
    for y, y2 in zip(ys, ys2):
        assert torch.equal(y, y2)


@pytest.mark.parametrize("m", [1, 3, 7, 12])
def test_planes_power_of_two_scale_invariance(cuda, m):
    """y(2^e x) == 2^e y(x) bit for bit for every row, e in -100..100: each chunk of x is brought
    to the same f16 values whatever its power-of-two scale.  e >= 16 puts |x| beyond f16's
    65504 (the rows would be inf without the pre-scale); e = -30 puts it below f16's subnormals."""
    n, k = 200, 2048
    w = synth.weight(64, 1, n, k)
    p, (codes, scales, zeros) = _packed(w, cuda)
    pl = ops.int4g_to_planes(p)
    xb = synth.activations_bf16(65, 7, m, k)
    x32 = O.bf16_bits_to_f32(xb)
    y0 = ops.gemv_w4a16_planes(_xdev(xb, cuda), pl, torch.float32).cpu().numpy()
    _close(torch.from_numpy(y0), O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128))
    for e in (-100, -30, -10, 5, 16, 20, 60, 100):
        xe = O.f32_to_bf16_bits((x32 * np.float32(2.0 ** e)).astype(np.float32))
        assert np.array_equal(O.bf16_bits_to_f32(xe), (x32 * np.float32(2.0 ** e)).astype(np.float32))
        ye = ops.gemv_w4a16_planes(_xdev(xe, cuda), pl, torch.float32).cpu().numpy()
        assert np.all(np.isfinite(ye)), e
        assert np.array_equal(ye, (y0.astype(np.float64) * 2.0 ** e).astype(np.float32)), e


def test_planes_large_and_tiny_activations_vs_oracle(cuda):
    """Rows with channels reaching 1e3..6e4 and beyond f16 range (1e5, 3e6), chunks of tiny
    values (1e-6, bf16 subnormals) next to ordinary ones.  Every row meets the plain bound
    against the oracle's f32 loop, except rows whose output cancels so far that the oracle's
    own sequential f32 sum is off the exact (f64) value by more than 1e-3; there the row must
    be no further from the exact value than the oracle is, plus the plain bound."""
    n, k = 256, 4096
    w = synth.weight(66, 1, n, k)
    p, (codes, scales, zeros) = _packed(w, cuda)
    pl = ops.int4g_to_planes(p)
    rng = np.random.default_rng(67)
    x = rng.standard_normal(k).astype(np.float32)
    idx = rng.choice(k, 60, replace=False)
    x[idx] *= rng.choice([1e3, 6e4, 1e5, 3e6], 60).astype(np.float32)
    x[1024:1152] *= np.float32(1e-6)          # a whole chunk of tiny values
    x[2048:2176] = np.float32(2.0 ** -130)    # a chunk of bf16 subnormals
    xb = O.f32_to_bf16_bits(x).reshape(1, k)
    y = ops.gemv_w4a16_planes(_xdev(xb, cuda), pl, torch.float32).cpu().numpy().reshape(-1)
    ref = O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128).reshape(-1)
    deq = O.dequantize_int4g(codes, scales, zeros, n, k, 128).astype(np.float64)
    exact = deq @ O.bf16_bits_to_f32(xb).reshape(-1).astype(np.float64)
    ref_err = np.abs(ref - exact)
    plain = np.abs(y - ref) <= ATOL + RTOL * np.abs(ref)
    assert np.all(plain | (ref_err > ATOL)), np.flatnonzero(~plain & (ref_err <= ATOL))
    assert np.all(np.abs(y - exact) <= ATOL + RTOL * np.abs(exact) + ref_err)


@pytest.mark.parametrize("m", [1, 4, 8, 16])
def test_planes_exact_cancellation(cuda, m):
    """x = [v, -v] with |v| up to 6e4 against weights whose two K halves are equal: the exact
    answer is 0 for every row, reached only through partial sums of order 1e4.  The oracle's
    sequential f32 loop leaves rounding noise of up to ~1e-1 there; every row must be within
    the plain bound of 0 or no further from it than the oracle's own result."""
    n, kh = 96, 2048
    rng = np.random.default_rng(68)
    wh = (rng.standard_normal((n, kh)) * 0.02).astype(np.float32)
    w = np.concatenate([wh, wh], axis=1)
    p, (codes, scales, zeros) = _packed(w, cuda)
    pl = ops.int4g_to_planes(p)
    v = rng.standard_normal((m, kh)).astype(np.float32)
    for r in range(m):
        v[r, rng.choice(kh, 40, replace=False)] *= np.float32(6e4)
    xb = O.f32_to_bf16_bits(np.concatenate([v, -v], axis=1)).reshape(m, 2 * kh)
    y = ops.gemv_w4a16_planes(_xdev(xb, cuda), pl, torch.float32).cpu().numpy()
    ref = O.gemm_w4a16(xb, codes, scales, zeros, n, 2 * kh, 128).reshape(m, n)
    mag = np.abs(O.bf16_bits_to_f32(xb).astype(np.float64)) @ \
        np.abs(O.dequantize_int4g(codes, scales, zeros, n, 2 * kh, 128).astype(np.float64)).T
    assert np.all(np.abs(y) <= ATOL + 2.0 ** -22 * mag), (np.abs(y).max(), np.abs(ref).max())
    assert np.abs(y).max() <= np.abs(ref).max()


@pytest.mark.parametrize("m,k", [(2, 40960), (4, 40960), (16, 40960)])
def test_planes_long_rows_vs_oracle(cuda, m, k):
    """x of M = 2..4 rows too long for the LDS-staged kernel (about 2.1 M k bytes) runs on the
    kernel that keeps x in registers, as M = 5..16 does at any K."""
    n = 40
    w = synth.weight(71, 1, n, k)
    p, (codes, scales, zeros) = _packed(w, cuda)
    pl = ops.int4g_to_planes(p)
    xb = synth.activations_bf16(72, 7, m, k)
    y = ops.gemv_w4a16_planes(_xdev(xb, cuda), pl, torch.float32)
    _close(y, O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128))


@pytest.mark.parametrize("m", [3, 8, 16])
def test_planes_nonfinite_row_stays_in_its_row(cuda, m):
    """An inf in one row of x makes that row's outputs non-finite and leaves the other rows'
    outputs finite and equal to the oracle's (each row has its own per-chunk power of two)."""
    n, k = 64, 1024
    w = synth.weight(73, 1, n, k)
    p, (codes, scales, zeros) = _packed(w, cuda)
    pl = ops.int4g_to_planes(p)
    xb = synth.activations_bf16(74, 7, m, k)
    bad = m - 2
    x = O.bf16_bits_to_f32(xb).reshape(m, k).copy()
    x[bad, 300] = np.inf
    xb = O.f32_to_bf16_bits(x)
    y = ops.gemv_w4a16_planes(_xdev(xb, cuda), pl, torch.float32).cpu().numpy()
    assert not np.isfinite(y[bad]).any()
    ok = [r for r in range(m) if r != bad]
    ref = O.gemm_w4a16(xb, codes, scales, zeros, n, k, 128).reshape(m, n)
    _close(torch.from_numpy(y[ok]), ref[ok])


def test_planes_nonfinite_x_gives_nonfinite_rows(cuda):
    n, k = 32, 256
    w = synth.weight(69, 1, n, k)
    p, _ = _packed(w, cuda)
    pl = ops.int4g_to_planes(p)
    x = np.zeros(k, np.float32)
    x[5] = np.inf
    y = ops.gemv_w4a16_planes(_xdev(O.f32_to_bf16_bits(x).reshape(1, k), cuda), pl, torch.float32)
    assert not torch.isfinite(y).any()


def test_planes_rejects_bad_arguments(cuda):
    w = torch.from_numpy(synth.weight(5, 1, 32, 256)).to(cuda)
    p = ops.quantize_int4g(w, 128)
    pl = ops.int4g_to_planes(p)
    x = torch.zeros((2, 256), dtype=torch.bfloat16, device=cuda)
    y = torch.empty((2, 32), dtype=torch.float32, device=cuda)
    arr = (ffi.W4A16Problem * 1)()
    arr[0] = ffi.W4A16Problem(x.data_ptr(), pl.codes.data_ptr(), pl.scales.data_ptr(), pl.zeros.data_ptr(),
                              y.data_ptr(), 32, 256, 128)
    with pytest.raises(ffi.CastForgeHipError, match="M = 1..16"):
        ffi.call("castforge_hip_gemv_w4a16_planes_batched", arr, 1, 17, ffi.DTYPE_F32, None)
    with pytest.raises(ValueError, match="1..16 rows"):
        ops.gemv_w4a16_planes(torch.zeros((17, 256), dtype=torch.bfloat16, device=cuda), pl)
    arr[0].group = 64
    with pytest.raises(ffi.CastForgeHipError, match="groups of 128"):
        ffi.call("castforge_hip_gemv_w4a16_planes_batched", arr, 1, 1, ffi.DTYPE_F32, None)
    with pytest.raises(ValueError, match="group 128"):
        ops.int4g_to_planes(ops.quantize_int4g(w, 64))
    # a problem's activations must fit the kernel's LDS (k = 81920 does not: 160 KB of f16 alone)
    big = torch.zeros((1, 81920), dtype=torch.bfloat16, device=cuda)
    plb = ops.int4g_to_planes(ops.quantize_int4g(torch.zeros((16, 81920), device=cuda), 128))
    with pytest.raises(ffi.CastForgeHipError, match="LDS"):
        ops.gemv_w4a16_planes_batched([big], [plb], [torch.empty((1, 16), device=cuda)])
    torch.cuda.synchronize()
