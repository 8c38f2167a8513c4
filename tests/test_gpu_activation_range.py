"""Activations of any finite bf16 magnitude through every fused-dequant GEMV / GEMM path.

The evaluator computes in f32 for any finite input (eval.rs:1492-1505).  The HIP kernels feed
f16 or bf16 MFMAs: f16 operands hold 2^-24 .. 65504 only, so each chunk of x is brought into
range by an exact power of two that its f32 partial undoes (M <= 16 kernels), or x stays bf16
(prefill).  Checked per format (INT4 g128/g64/g32, INT8 per channel, NF4 b64, GGUF Q4_0/Q8_0)
and per kernel (M = 1 split-K, M = 3 and 16 skinny, M = 40 and 300 prefill):
  * rows with channels reaching 1e3..6e4 and beyond f16 range (1e5, 3e6), a chunk of 1e-6
    values and a chunk of bf16 subnormals: every output meets the plain bound against the
    oracle wherever the oracle's own sequential f32 sum is within 1e-3 of the exact (f64)
    value, and is no further from the exact value than the oracle is (plus the plain bound)
    everywhere -- for NF4 at M > 16 (two bf16 terms of the table value) plus its stated
    2^-16 sum |x w|;
  * y(2^e x) == 2^e y(x) bit for bit for the M <= 16 kernels (e = -60 .. 60);
  * x = [v, -v] against weights whose two K halves are equal (exact answer 0, partial sums of
    order 1e4, where the evaluator's own f32 loop is off by up to ~1e-2): every output within
    1e-3 plus the worst case of the kernel's summation (one rounding per 16-wide MFMA step and
    weight term: (3 K / 16 + 8) 2^-24 sum |x w|) of 0, and the residuals' RMS no larger than
    the evaluator's;
  * a non-finite x gives non-finite rows.
INT4 g128 / g64 / g32, INT8 and GGUF Q4_0 / Q8_0 run a second time with the one-MFMA prefill
kernel forced (the *_one formats): exact (q - z) / q operands, one f32 partial per group
(GGUF: per 32-wide block; INT8: one sum, its row scale applied once) scaled into the total.
"""
import os

import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ops

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3
Q4_0, Q8_0 = ops.GGML_TYPES["Q4_0"], ops.GGML_TYPES["Q8_0"]
BB = {Q4_0: 18, Q8_0: 34}


def _xdev(xb, dev):
    return torch.from_numpy(np.ascontiguousarray(xb).view(np.int16)).view(torch.bfloat16).to(dev)


def _weight(seed, n, k, halves, positive=False):
    rng = np.random.default_rng(seed)
    if halves:
        wh = (rng.standard_normal((n, k // 2)) * 0.02).astype(np.float32)
        return np.concatenate([wh, wh], axis=1)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return np.abs(w) if positive else w


def _gguf_raw(ty, seed, n, k, halves, positive=False):
    rng = np.random.default_rng(seed)
    bpr = k // 32
    raw = rng.integers(0, 256, (n, bpr, BB[ty]), dtype=np.uint8)
    if positive:  # every code at its largest q - 8 (Q4_0: 7) or q (Q8_0: 127), d > 0
        raw[:] = 0xFF if ty == Q4_0 else 0x7F
    d = (rng.standard_normal((n, bpr)) * 0.002).astype(np.float16)
    if positive:
        d = np.abs(d)
    raw[:, :, 0:2] = d.view(np.uint8).reshape(n, bpr, 2)
    if halves:
        raw[:, bpr // 2:] = raw[:, : bpr // 2]
    return raw.reshape(-1)


class Case:
    """One packed weight: run(x) on the GPU, the oracle's f32 result and the exact f64 one."""

    def __init__(self, fmt, n, k, dev, seed=11, halves=False, positive=False):
        self.fmt, self.n, self.k = fmt, n, k
        if fmt.startswith("int4"):
            g = int(fmt.split("_")[1][1:])
            w = _weight(seed, n, k, halves, positive)
            c, s, z = O.quantize_int4g(w, g)
            self.p = ops.Int4Packed(torch.from_numpy(c.view(np.int32)).to(dev),
                                    torch.from_numpy(s.view(np.float16)).to(dev),
                                    torch.from_numpy(z.view(np.int32)).to(dev), n, k, g)
            if fmt.endswith("_one"):  # the one-MFMA prefill kernel, forced at every M > 64
                self.run = lambda x, out: _one_mfma(lambda: ops.gemm_w4a16(x, self.p, out))
            else:
                self.run = lambda x, out: ops.gemm_w4a16(x, self.p, out)
            self.oracle = lambda xb: O.gemm_w4a16(xb, c, s, z, n, k, g)
            self.deq = O.dequantize_int4g(c, s, z, n, k, g)
        elif fmt.startswith("int8"):
            w = _weight(seed, n, k, halves, positive)
            c, s = O.quantize_int8_rows(w)
            cd, sd = torch.from_numpy(c).to(dev), torch.from_numpy(s).to(dev)
            if fmt.endswith("_one"):  # the one-MFMA prefill kernel, forced at every M > 64
                self.run = lambda x, out: _one_mfma(lambda: ops.gemm_w8a16(x, cd, sd, "channel", out))
            else:
                self.run = lambda x, out: ops.gemm_w8a16(x, cd, sd, "channel", out)
            self.oracle = lambda xb: O.gemm_w8a16(xb, c, s)
            self.deq = c.astype(np.float32) * s[:, None]
        elif fmt == "nf4":
            w = _weight(seed, n, k, halves)
            c, am = O.quantize_nf4(w, 64)
            self.p = ops.Nf4Packed(torch.from_numpy(c.view(np.int32)).to(dev), torch.from_numpy(am).to(dev), n, k, 64)
            self.run = lambda x, out: ops.gemm_nf4(x, self.p, out)
            self.oracle = lambda xb: O.gemm_nf4(xb, c, am, n, k, 64)
            self.deq = O.dequantize_nf4(c, am, n, k, 64)
        else:
            ty = Q4_0 if fmt.startswith("q4_0") else Q8_0
            raw = _gguf_raw(ty, seed, n, k, halves, positive)
            self.p = ops.gguf_repack(ty, torch.from_numpy(raw).to(dev), n, k)
            if fmt.endswith("_one"):  # the one-MFMA prefill kernel, forced at every M > 64
                self.run = lambda x, out: _one_mfma(lambda: ops.gemm_gguf(x, self.p, out))
            else:
                self.run = lambda x, out: ops.gemm_gguf(x, self.p, out)
            wd = O.gguf_decode(ty, raw, n * k).reshape(n, k)
            self.oracle = lambda xb: O.matmul_2d(O.bf16_bits_to_f32(xb), wd, packed_rhs=True)
            self.deq = wd
        self.deq = np.asarray(self.deq, np.float64).reshape(n, k)


def _one_mfma(call):
    """Runs call with CASTFORGE_PREFILL_I4=1: INT4 prefill problems whose groups are whole
    128-wide K blocks take the one-MFMA kernel whatever their tile count."""
    old = os.environ.get("CASTFORGE_PREFILL_I4")
    os.environ["CASTFORGE_PREFILL_I4"] = "1"
    try:
        return call()
    finally:
        if old is None:
            del os.environ["CASTFORGE_PREFILL_I4"]
        else:
            os.environ["CASTFORGE_PREFILL_I4"] = old


FORMATS = ["int4_g128", "int4_g128_one", "int4_g64", "int4_g64_one", "int4_g32", "int4_g32_one", "int8", "int8_one",
           "nf4", "q4_0", "q4_0_one", "q8_0", "q8_0_one"]
MS = [1, 3, 16, 40, 300]


def _wide_x(seed, m, k):
    """bf16 rows: N(0, 1) with 1.5% of the channels x 1e3 / 6e4 / 1e5 / 3e6, a 128-value run of
    1e-6 values and a 128-value run of bf16 subnormals."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    for r in range(m):
        idx = rng.choice(k, max(1, int(0.015 * k)), replace=False)
        x[r, idx] *= rng.choice([1e3, 6e4, 1e5, 3e6], idx.size).astype(np.float32)
    x[:, k // 4: k // 4 + 128] *= np.float32(1e-6)
    x[:, k // 2: k // 2 + 128] = np.float32(2.0 ** -130)
    return O.f32_to_bf16_bits(x)


@pytest.mark.parametrize("m", MS)
@pytest.mark.parametrize("fmt", FORMATS)
def test_wide_activations_vs_oracle(cuda, fmt, m):
    n, k = 96, 2048
    c = Case(fmt, n, k, cuda)
    xb = _wide_x(100 + m, m, k)
    y = c.run(_xdev(xb, cuda), torch.float32).cpu().numpy()
    ref = c.oracle(xb)
    exact = O.bf16_bits_to_f32(xb).astype(np.float64) @ c.deq.T
    assert np.all(np.isfinite(y))
    ref_err = np.abs(ref - exact)
    plain = np.abs(y - ref) <= ATOL + RTOL * np.abs(ref)
    bad = ~plain & (ref_err <= ATOL)
    assert not bad.any(), (f"{int(bad.sum())} outputs past the plain bound where the oracle is exact; "
                           f"worst y {y[bad][0]:.6g} ref {ref[bad][0]:.6g}")
    slack = ref_err
    if fmt == "nf4" and m >= 17:
        # the NF4 MFMA kernel feeds T as T_hi + T_lo (16 significant bits): its stated bound adds
        # 2^-16 sum |x w| (below the evaluator's own worst case, K 2^-24 sum |x w|, at K >= 256)
        slack = ref_err + 2.0 ** -16 * (np.abs(O.bf16_bits_to_f32(xb).astype(np.float64)) @ np.abs(c.deq.T))
    far = np.abs(y - exact) > ATOL + RTOL * np.abs(exact) + slack
    assert not far.any(), f"{int(far.sum())} outputs further from the exact value than the oracle"


@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("fmt", FORMATS)
def test_power_of_two_scale_invariance(cuda, fmt, m):
    n, k = 80, 1024
    c = Case(fmt, n, k, cuda, seed=12)
    xb = _wide_x(200 + m, m, k)
    x32 = O.bf16_bits_to_f32(xb)
    y0 = c.run(_xdev(xb, cuda), torch.float32).cpu().numpy().astype(np.float64)
    for e in (-60, -20, 20, 60):
        xe = (x32 * np.float32(2.0 ** e)).astype(np.float32)
        xeb = O.f32_to_bf16_bits(xe)
        nz = xe != 0
        assert np.array_equal(O.bf16_bits_to_f32(xeb)[nz], xe[nz])
        ye = c.run(_xdev(xeb, cuda), torch.float32).cpu().numpy()
        assert np.array_equal(ye, (y0 * 2.0 ** e).astype(np.float32)), (fmt, m, e)


@pytest.mark.parametrize("m", MS)
@pytest.mark.parametrize("fmt", FORMATS)
def test_exact_cancellation(cuda, fmt, m):
    n, k = 64, 2048
    c = Case(fmt, n, k, cuda, seed=13, halves=True)
    rng = np.random.default_rng(300 + m)
    v = rng.standard_normal((m, k // 2)).astype(np.float32)
    for r in range(m):
        v[r, rng.choice(k // 2, 20, replace=False)] *= np.float32(6e4)
    xb = O.f32_to_bf16_bits(np.concatenate([v, -v], axis=1))
    y = c.run(_xdev(xb, cuda), torch.float32).cpu().numpy()
    ref = c.oracle(xb)
    mag = np.abs(O.bf16_bits_to_f32(xb).astype(np.float64)) @ np.abs(c.deq.T)
    # worst case of the kernel's own f32 summation: at most one rounding of the running sum
    # per 16-wide MFMA step and weight term (3 terms at most), plus the final scalings
    rounds = 3 * k // 16 + 8
    assert np.all(np.abs(y) <= ATOL + rounds * 2.0 ** -24 * mag), float(np.abs(y).max())
    # and on average no further from the exact 0 than the evaluator's sequential f32 loop
    rms, rms_ref = np.sqrt(np.mean(y.astype(np.float64) ** 2)), np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    assert rms <= rms_ref + ATOL, (rms, rms_ref)


@pytest.mark.parametrize("m", [1, 5, 40, 100])
@pytest.mark.parametrize("fmt", FORMATS)
def test_nonfinite_x_gives_nonfinite_rows(cuda, fmt, m):
    n, k = 32, 1024
    c = Case(fmt, n, k, cuda, seed=14)
    x = np.zeros((m, k), np.float32)
    x[:, 5] = np.inf
    y = c.run(_xdev(O.f32_to_bf16_bits(x), cuda), torch.float32)
    assert not torch.isfinite(y).any()


@pytest.mark.parametrize("fmt", [f for f in FORMATS if f.endswith("_one")])
def test_one_mfma_prefill_at_activation_bound(cuda, fmt):
    """The one-MFMA prefill kernel feeds the unscaled integer (q - z), q - 8 or q and scales
    the f32 partial afterwards, so its partials reach |x| * 127 * K.  Its documented range is
    |x| <= 2^100 with K <= 2^20 (2^100 * 2^7 * 2^20 = 2^127 < f32 max).  At that bound, with
    every activation of a row of one sign: every output is finite and equals 2^100 times the
    output for x / 2^100 bit for bit (nothing overflowed or rounded differently); with every
    weight positive or every code at its largest (the largest partials, no cancellation) each
    output also meets the plain bound against the oracle."""
    n, k, m = 64, 2048, 100
    rng = np.random.default_rng(15)
    x1 = rng.uniform(0.5, 1.0, (m, k)).astype(np.float32)
    x1[m // 2:] *= np.float32(-1.0)
    x1[:, 0] = np.float32(1.0)
    x = (x1 * np.float32(2.0 ** 100)).astype(np.float32)
    xb, x1b = O.f32_to_bf16_bits(x), O.f32_to_bf16_bits(x1)
    assert np.abs(O.bf16_bits_to_f32(xb)).max() == np.float32(2.0 ** 100)
    assert np.array_equal(O.bf16_bits_to_f32(xb), O.bf16_bits_to_f32(x1b) * np.float32(2.0 ** 100))
    for positive in (False, True):
        case = Case(fmt, n, k, cuda, seed=15, positive=positive)
        y = case.run(_xdev(xb, cuda), torch.float32).cpu().numpy()
        y1 = case.run(_xdev(x1b, cuda), torch.float32).cpu().numpy()
        assert np.all(np.isfinite(y))
        assert np.array_equal(y, (y1.astype(np.float64) * 2.0 ** 100).astype(np.float32)), (fmt, positive)
        if positive:
            ref = case.oracle(xb)
            assert np.all(np.isfinite(ref))
            assert np.all(np.abs(y - ref) <= ATOL + RTOL * np.abs(ref))
