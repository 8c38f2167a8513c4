"""GPU parity of the FP8 E4M3 W8A8 GEMM against the oracle (dequantize, then the evaluator's
sequential f32 loop, eval.rs:1465-1507) and against an fp64 GEMM of the same dequantized
operands.

Two kernels share the operand pipeline:
  * exact=True (castforge_hip_gemm_fp8_exact, the one the evaluator dispatches to): codes widened
    to exact f16 on f16 MFMA.  Checked at the plain bound |y - ref| <= 1e-3 + 1e-2 |ref| on every
    output, config 4's outlier inputs included.
  * exact=False (castforge_hip_gemm_fp8, fp8 MFMA): the MFMA sums each block of products in a
    fixed-point adder aligned to the block's largest product and keeps about 13 bits below it
    (a one-wave probe: 256 + 2^-6 -> 256, 256 + 63 * 2^-6 -> 256.875).  On config 4's inputs a
    few near-zero outputs miss the plain bound; the tests count them and hold every output to
    the plain bound plus the adder's own worst case, 2^-12 * 64 * (largest |a_k w_k| of each
    64-wide K step), and the whole product to a relative RMS error of 2e-3."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ops, synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3
# the fp8 adder keeps >= 12 bits below the largest product of the MFMA's 64-wide K step
FP8_ADDER = 2.0 ** -12 * 64


def _deq(q, s):
    return torch.from_numpy(q).view(torch.float8_e4m3fn).double().numpy() * s.astype(np.float64)[:, None]


def _step_max_sum(ad, wd):
    """sum over 64-wide K steps of max_k |a_k w_k|, for every (row of ad, row of wd)."""
    k = ad.shape[1]
    kp = (k + 63) // 64 * 64
    out = np.empty((ad.shape[0], wd.shape[0]))
    wp = np.zeros((wd.shape[0], kp))
    wp[:, :k] = np.abs(wd)
    for r in range(ad.shape[0]):
        ap = np.zeros(kp)
        ap[:k] = np.abs(ad[r])
        out[r] = (wp * ap).reshape(wd.shape[0], kp // 64, 64).max(axis=2).sum(axis=1)
    return out


def _check(y, qa, sa, qw, sw, exact, what):
    """y (any [m, n] array) against the oracle at the plain bound (exact kernel), or at the
    plain bound plus the fp8 adder bound with a count of the outputs past the plain bound."""
    y = y.float().cpu().numpy() if isinstance(y, torch.Tensor) else y
    ref = O.gemm_fp8(qa, sa, qw, sw)
    ad, wd = _deq(qa, sa), _deq(qw, sw)
    ex = ad @ wd.T
    plain = np.abs(y - ref) > ATOL + RTOL * np.abs(ref)
    if exact:
        assert not plain.any(), (f"{what}: {int(plain.sum())} / {plain.size} outputs past the plain bound; "
                                 f"max err {np.abs(y - ref).max():.3e}")
        return 0
    bound = ATOL + RTOL * np.abs(ex) + np.abs(ref - ex) + FP8_ADDER * _step_max_sum(ad, wd)
    far = np.abs(y - ex) > bound
    assert not far.any(), f"{what}: {int(far.sum())} outputs past the fp8 adder bound"
    rel = np.sqrt(np.mean((y - ex) ** 2) / max(np.mean(ex ** 2), 1e-300))
    assert rel <= 2e-3, f"{what}: relative RMS error {rel:.2e}"
    return int(plain.sum())


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("m,n,k", [(64, 128, 256), (300, 200, 384), (256, 128, 128), (17, 33, 1024),
                                   (5, 7, 100), (1, 16, 128)])
def test_fp8_gemm_vs_oracle(cuda, m, n, k, exact):
    a = synth.fp8_inputs(81, 1, m, k)
    w = synth.fp8_inputs(81, 2, n, k) * np.float32(0.02)
    qa_ref, sa_ref = O.quantize_fp8_rows(a)
    qw_ref, sw_ref = O.quantize_fp8_rows(w)
    qa, sa = ops.quantize_fp8(torch.from_numpy(a).to(cuda))
    qw, sw = ops.quantize_fp8(torch.from_numpy(w).to(cuda))
    assert np.array_equal(qa.cpu().numpy(), qa_ref) and np.array_equal(qw.cpu().numpy(), qw_ref)
    for out in (torch.bfloat16, torch.float32):
        # a bf16 output's rounding (<= 2^-9 relative) sits inside the 1e-2 relative term
        y = ops.gemm_fp8(qa, sa, qw, sw, out_dtype=out, exact=exact)
        _check(y, qa_ref, sa_ref, qw_ref, sw_ref, exact, f"{m}x{n}x{k} {out}")


def _config4(cuda, m, n, k, seed):
    """both operands N(0, 1) with 0.5% of the elements x30; activations
    quantized per token from bf16, weights per output row from f32."""
    g = torch.Generator(device=cuda)
    g.manual_seed(seed)
    a = torch.randn((m, k), generator=g, device=cuda)
    a[torch.rand((m, k), generator=g, device=cuda) < 0.005] *= 30
    w = torch.randn((n, k), generator=g, device=cuda)
    w[torch.rand((n, k), generator=g, device=cuda) < 0.005] *= 30
    qa, sa = ops.quantize_fp8(a.to(torch.bfloat16))
    qw, sw = ops.quantize_fp8(w)
    return qa, sa, qw, sw


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("m,n,k", [(4096, 11008, 4096), (4096, 4096, 11008)])
def test_fp8_gemm_config4_sampled_vs_oracle(cuda, m, n, k, exact):
    """Sampled outputs (48 rows x 192 columns) of the BASELINE shapes on config 4's inputs
    against the oracle's f32 loop, f32 output.  The exact kernel meets the plain bound on every
    sampled output; the fp8 kernel's count past it is printed (the measured deviation)."""
    qa, sa, qw, sw = _config4(cuda, m, n, k, 5)
    y = ops.gemm_fp8(qa, sa, qw, sw, out_dtype=torch.float32, exact=exact)
    torch.cuda.synchronize()
    rng = np.random.default_rng(m + n + k)
    rows = np.sort(rng.choice(m, 48, replace=False))
    cols = np.sort(rng.choice(n, 192, replace=False))
    ys = y.cpu().numpy()[rows][:, cols]
    nbad = _check(ys, qa.cpu().numpy()[rows], sa.cpu().numpy()[rows], qw.cpu().numpy()[cols],
                  sw.cpu().numpy()[cols], exact, f"config4 {m}x{n}x{k}")
    if not exact:
        print(f"fp8 MFMA, config4 {m}x{n}x{k}: {nbad} / {ys.size} sampled outputs past the plain bound")
        # the full-size rate is 0.23-0.27 % (test_fp8_gemm_baseline_shapes); a 9216-output
        # sample at that rate has a mean of 25 and a standard deviation of 5
        assert nbad <= ys.size * 5 // 1000


@pytest.mark.parametrize("exact", [True, False])
@pytest.mark.parametrize("m,n,k", [(4096, 11008, 4096), (4096, 4096, 11008)])
def test_fp8_gemm_baseline_shapes(cuda, m, n, k, exact):
    """Every output of the BASELINE shapes on config 4's inputs against an fp64 GEMM of the
    same dequantized operands.  Exact kernel: the plain bound on f32 and bf16 outputs (a bf16
    output's rounding, <= 2^-9 relative, sits inside the 1e-2 relative term).  fp8 kernel: the
    count past the plain bound and a relative RMS error of at most 2e-3."""
    qa, sa, qw, sw = _config4(cuda, m, n, k, 6)
    ad = qa.view(torch.float8_e4m3fn).double() * sa[:, None].double()
    wd = qw.view(torch.float8_e4m3fn).double() * sw[:, None].double()
    ref = ad @ wd.t()
    for out in (torch.float32, torch.bfloat16):
        y = ops.gemm_fp8(qa, sa, qw, sw, out_dtype=out, exact=exact)
        torch.cuda.synchronize()
        err = (y.double() - ref).abs()
        tol = ATOL + RTOL * ref.abs()
        nbad = int((err > tol).sum())
        if exact:
            assert nbad == 0, f"{nbad} outside the plain bound; max err {float(err.max()):.3e}"
        else:
            rel = float(((y.double() - ref) ** 2).mean().sqrt() / (ref ** 2).mean().sqrt())
            print(f"fp8 MFMA, config4 {m}x{n}x{k} {out}: {nbad} / {ref.numel()} outputs past the plain "
                  f"bound, max err {float(err.max()):.3e}, relative RMS {rel:.2e}")
            # measured: 0.23 % (n = 11008) and 0.27 % (n = 4096) of all outputs on these inputs
            assert rel <= 2e-3 and nbad <= ref.numel() * 3 // 1000


@pytest.mark.parametrize("exact", [True, False])
def test_fp8_gemm_zero_and_outliers(cuda, exact):
    m, n, k = 64, 64, 256
    a = np.zeros((m, k), np.float32)
    a[1, 3] = 1000.0
    a[2, :] = 1e-30
    w = synth.fp8_inputs(83, 1, n, k)
    qa, sa = ops.quantize_fp8(torch.from_numpy(a).to(cuda))
    qw, sw = ops.quantize_fp8(torch.from_numpy(w).to(cuda))
    y = ops.gemm_fp8(qa, sa, qw, sw, out_dtype=torch.float32, exact=exact)
    qa_ref, sa_ref = O.quantize_fp8_rows(a)
    qw_ref, sw_ref = O.quantize_fp8_rows(w)
    _check(y, qa_ref, sa_ref, qw_ref, sw_ref, exact, "zero/outlier rows")


def test_fp8_gemm_out_validation(cuda):
    qa = torch.zeros((4, 64), dtype=torch.uint8, device=cuda)
    qw = torch.zeros((8, 64), dtype=torch.uint8, device=cuda)
    s4, s8 = torch.ones(4, device=cuda), torch.ones(8, device=cuda)
    for bad in (torch.empty((8, 4), device=cuda), torch.empty((4, 16), device=cuda)[:, ::2],
                torch.empty((4, 8), dtype=torch.float16, device=cuda)):
        with pytest.raises(ValueError, match="out must be"):
            ops.gemm_fp8(qa, s4, qw, s8, out=bad)
