"""GPU parity of the FP8 E4M3 W8A8 GEMM: against the oracle (dequantize, eval_matmul_2d) at
small shapes and against a torch fp32 GEMM of the same dequantized operands at the BASELINE
shapes; tolerance |y - ref| <= 1e-3 + 1e-2 |ref|."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ops, synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _close(y, ref):
    y = y.float().cpu().numpy() if isinstance(y, torch.Tensor) else y
    ref = ref.cpu().numpy() if isinstance(ref, torch.Tensor) else ref
    err = np.abs(y - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}"


@pytest.mark.parametrize("m,n,k", [(64, 128, 256), (300, 200, 384), (256, 128, 128), (17, 33, 1024),
                                   (5, 7, 100), (1, 16, 128)])
def test_fp8_gemm_vs_oracle(cuda, m, n, k):
    a = synth.fp8_inputs(81, 1, m, k)
    w = synth.fp8_inputs(81, 2, n, k) * np.float32(0.02)
    qa_ref, sa_ref = O.quantize_fp8_rows(a)
    qw_ref, sw_ref = O.quantize_fp8_rows(w)
    qa, sa = ops.quantize_fp8(torch.from_numpy(a).to(cuda))
    qw, sw = ops.quantize_fp8(torch.from_numpy(w).to(cuda))
    assert np.array_equal(qa.cpu().numpy(), qa_ref) and np.array_equal(qw.cpu().numpy(), qw_ref)
    y = ops.gemm_fp8(qa, sa, qw, sw)
    _close(y, O.gemm_fp8(qa_ref, sa_ref, qw_ref, sw_ref))


@pytest.mark.parametrize("m,n,k", [(4096, 11008, 4096), (4096, 4096, 11008)])
def test_fp8_gemm_baseline_shapes(cuda, m, n, k):
    g = torch.Generator(device=cuda)
    g.manual_seed(5)
    a = torch.randn((m, k), generator=g, device=cuda)
    a[torch.rand((m, k), generator=g, device=cuda) < 0.005] *= 30
    w = torch.randn((n, k), generator=g, device=cuda) * 0.02
    qa, sa = ops.quantize_fp8(a.to(torch.bfloat16))
    qw, sw = ops.quantize_fp8(w)
    y = ops.gemm_fp8(qa, sa, qw, sw)
    ad = qa.view(torch.float8_e4m3fn).float() * sa[:, None]
    wd = qw.view(torch.float8_e4m3fn).float() * sw[:, None]
    ref = ad @ wd.t()
    torch.cuda.synchronize()
    err = (y.float() - ref).abs()
    bad = err > ATOL + RTOL * ref.abs()
    assert int(bad.sum()) == 0, f"{int(bad.sum())} outside tol; max err {float(err.max()):.3e}"


def test_fp8_gemm_zero_and_outliers(cuda):
    m, n, k = 64, 64, 256
    a = np.zeros((m, k), np.float32)
    a[1, 3] = 1000.0
    a[2, :] = 1e-30
    w = synth.fp8_inputs(83, 1, n, k)
    qa, sa = ops.quantize_fp8(torch.from_numpy(a).to(cuda))
    qw, sw = ops.quantize_fp8(torch.from_numpy(w).to(cuda))
    y = ops.gemm_fp8(qa, sa, qw, sw)
    qa_ref, sa_ref = O.quantize_fp8_rows(a)
    qw_ref, sw_ref = O.quantize_fp8_rows(w)
    _close(y, O.gemm_fp8(qa_ref, sa_ref, qw_ref, sw_ref))
