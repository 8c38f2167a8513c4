"""Pins for the oracle functions whose values the reference's own tests do not fix: the
group-wise / AWQ write-back quantizer (schemes.rs:485-549), the FP8 / MXFP8 uniform-grid
quantizer (schemes.rs:681-713) and the relu / gelu / scale epilogues of fused_qmatmul
(eval.rs:1151-1176, 1733-1735).

Each check is one a plausible slip in the restatement would fail: f64 instead of f32
arithmetic, half-even instead of half-away rounding, `>` instead of `>=` at the salient
threshold, qmin taken as -qmax, a wrong grid step or GELU constant, the erf GELU in place of
the tanh form.  Checks are hand-computed known answers, an independent numpy restatement
(vectorised, written from the reference text, sharing no code with oracle/cf_oracle.c), and
float64 formulas."""
import math

import numpy as np
import pytest

import oracle_lib as O

f32 = np.float32


# ------------------------------------------------------------------ group-wise / AWQ ----
def test_groupwise_known_answer_2x2():
    """w = [[0.5, -0.25], [0.75, 0.5]], bits 4 ([-8, 7]), group 2, salient ratio 0.25
    (frontend_tests.rs:747-756 shape).  salient_count = ceil(4 * 0.25) = 1, threshold 0.75.
    Group 0: s0 = f32(0.5 / 7) = 0.0714285746; 0.5 / s0 = 6.9999995 -> 7 -> 7 * s0 = 0.5;
    -0.25 / s0 = -3.4999998 in f32 (-3.5 in f64, which would give -4) -> -3 -> -0.2142857313.
    Group 1: s1 = f32(0.75 / 7) = 0.1071428582; 0.75 is salient (>= 0.75): eff = s1 / 2,
    0.75 / eff = 14 -> clamp 7 -> 0.375 (0.75 without awq_salient); 0.5 / s1 = 4.6666665 -> 5
    -> 5 * s1 = 0.5357142687."""
    w = np.array([[0.5, -0.25], [0.75, 0.5]], f32)
    s0, s1 = f32(0.5) / f32(7), f32(0.75) / f32(7)
    assert s0 == f32(0.0714285746216774) and s1 == f32(0.1071428582072258)
    deq, scales, cnt, thr = O.quantize_groupwise(w, bits=4, group_size=2, awq_salient=True, salient_ratio=0.25)
    assert cnt == 1 and thr == 0.75
    assert scales.tolist() == [s0, s1]
    assert deq.tolist() == [0.5, f32(-3) * s0, f32(7) * (s1 * f32(0.5)), f32(5) * s1]
    assert deq.tolist() == [0.5, f32(-0.2142857313156128), 0.375, f32(0.5357142686843872)]
    deq2, _, _, _ = O.quantize_groupwise(w, bits=4, group_size=2, awq_salient=False, salient_ratio=0.25)
    assert deq2.tolist() == [0.5, f32(-0.2142857313156128), 0.75, f32(0.5357142686843872)]


def test_groupwise_ties_round_half_away_and_threshold_is_inclusive():
    """Group max 7 with bits 4 makes the scale exactly 1, so every x.5 is a true tie:
    half-away gives 3 / -3 / 1 / -1 / 4 / -7 where half-even gives 2 / -2 / 0 / -0 / 4 / -6.
    Salient ratio 1/8 makes only |v| >= 7 salient: both 7 and -7 (inclusive test) take scale
    0.5, 7 / 0.5 = 14 -> 7 -> 3.5 and -14 -> clamp to qmin = -8 -> -4 (not -3.5)."""
    v = np.array([7.0, 2.5, -2.5, 0.5, -0.5, 3.5, -6.5, -7.0], f32)
    deq, sc, cnt, thr = O.quantize_groupwise(v, bits=4, group_size=8, awq_salient=True, salient_ratio=0.125)
    assert cnt == 1 and thr == 7.0 and sc.tolist() == [1.0]
    assert deq.tolist() == [3.5, 3.0, -3.0, 1.0, -1.0, 4.0, -7.0, -4.0]
    deq, _, _, _ = O.quantize_groupwise(v, bits=4, group_size=8, awq_salient=False, salient_ratio=0.125)
    assert deq.tolist() == [7.0, 3.0, -3.0, 1.0, -1.0, 4.0, -7.0, -7.0]
    deq, _, _, _ = O.quantize_groupwise(v, bits=4, group_size=8, awq_salient=False, salient_ratio=0.125,
                                        round_mode=1)
    assert deq.tolist() == [7.0, 2.0, -2.0, 0.0, -0.0, 4.0, -6.0, -7.0]
    # 8-bit bounds: group max 127 -> scale 1; -126.5 and 124.5 are ties (half-away -127 / 125,
    # half-even -126 / 124); with the salient halving -127 reaches qmin: -254 -> -128 -> -64
    v8 = np.array([127.0, -126.5, 124.5, 0.0], f32)
    deq, _, _, _ = O.quantize_groupwise(v8, bits=8, group_size=4, awq_salient=False, salient_ratio=0.01)
    assert deq.tolist() == [127.0, -127.0, 125.0, 0.0]
    deq, _, _, _ = O.quantize_groupwise(v8, bits=8, group_size=4, awq_salient=False, salient_ratio=0.01,
                                        round_mode=1)
    assert deq.tolist() == [127.0, -126.0, 124.0, 0.0]
    v8 = np.array([127.0, -127.0, 3.0, 0.0], f32)
    deq, _, _, _ = O.quantize_groupwise(v8, bits=8, group_size=4, awq_salient=True, salient_ratio=0.25)
    assert deq.tolist() == [63.5, -64.0, 3.0, 0.0]


def _total_desc_abs(v):
    """|v| sorted descending in Rust's f32::total_cmp order.  |v| clears the sign bit, so
    every key is a non-negative float (or +NaN) whose bit pattern orders like total_cmp."""
    return np.sort(np.abs(v).view(np.uint32))[::-1].view(f32)


def _round_away(q):
    q64 = q.astype(np.float64)  # exact; x + 0.5 is exact in f64 for every f32 x
    return np.where(np.isfinite(q64), np.trunc(q64 + np.copysign(0.5, q64)), q64).astype(f32)


def groupwise_numpy(v, bits, gs, awq, ratio, round_mode=0):
    """schemes.rs:485-549 restated with vectorised numpy float32 operations."""
    v = np.ascontiguousarray(v, f32).ravel()
    qmin, qmax = (f32(-8), f32(7)) if bits == 4 else (f32(-128), f32(127))
    gs = max(gs, 2)
    ratio = f32(min(max(ratio, 0.001), 0.5))
    n = v.size
    cnt = int(np.ceil(f32(n) * ratio))
    cnt = min(max(cnt, 1), n)
    thr = _total_desc_abs(v)[cnt - 1]
    out = np.empty_like(v)
    scales = []
    for c0 in range(0, n, gs):
        ch = v[c0:c0 + gs]
        a = np.abs(ch)
        gmax = f32(0) if np.all(np.isnan(a)) else max(f32(0), np.nanmax(a))
        scale = f32(1) if gmax < f32(1e-12) else gmax / qmax
        scales.append(scale)
        eff = np.where(awq & (a >= thr), scale * f32(0.5), scale).astype(f32)
        with np.errstate(invalid="ignore", divide="ignore"):
            q = ch / eff
        r = _round_away(q) if round_mode == 0 else np.rint(q)
        out[c0:c0 + gs] = np.clip(r, qmin, qmax) * eff
    return out, np.array(scales, f32), cnt, thr


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("awq", [True, False])
@pytest.mark.parametrize("round_mode", [0, 1])
def test_groupwise_matches_numpy_restatement(bits, awq, round_mode):
    rng = np.random.default_rng(100 + bits + 2 * awq + 4 * round_mode)
    cases = [(rng.standard_normal(4096) * 0.02).astype(f32)]
    # tie-laden: group max 7 / 127 pins the scale to 1 and half-integers sit on ties
    qm = 7 if bits == 4 else 127
    t = (rng.integers(-2 * qm, 2 * qm, 1024) / 2).astype(f32)
    t[::32] = qm
    cases.append(t)
    # ragged last group, zeros, a duplicated salient value, NaN and inf
    s = (rng.standard_normal(1000) * 3).astype(f32)
    s[:40] = 0.0
    s[100] = s[200] = np.abs(s).max() * 2
    s[300] = np.nan
    s[301] = np.inf
    s[302] = -np.inf
    cases.append(s)
    for v in cases:
        for gs, ratio in ((32, 0.01), (128, 0.05), (7, 0.5), (1, 0.0001)):
            got, gsc, gcnt, gthr = O.quantize_groupwise(v, bits=bits, group_size=gs, awq_salient=awq,
                                                        salient_ratio=ratio, round_mode=round_mode)
            ref, rsc, rcnt, rthr = groupwise_numpy(v, bits, gs, awq, ratio, round_mode)
            assert gcnt == rcnt
            assert np.array_equal(np.array([gthr], f32), np.array([rthr], f32), equal_nan=True)
            assert np.array_equal(gsc, rsc, equal_nan=True)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (gs, ratio)


def test_groupwise_salient_count_uses_f32_product():
    """salient_count = ceil(f32(n) * ratio) with the product rounded to f32: f32(0.3) =
    0.30000001192..., and 10 * that = 3 + 2^-23 exactly, a tie between 3 and 3 + 2^-22 that
    rounds to 3.0 in f32 (count 3, threshold 8); an f64 product would ceil to 4."""
    v = np.arange(10, dtype=f32) + 1
    _, _, cnt, thr = O.quantize_groupwise(v, bits=4, group_size=2, awq_salient=True, salient_ratio=0.3)
    assert float(f32(0.3)) * 10 == 3.0 + 2.0 ** -23 and f32(10) * f32(0.3) == f32(3.0)
    assert cnt == 3 and thr == 8.0


# ----------------------------------------------------------------- FP8 uniform grid ----
STEP = {False: f32(448.0) / f32(31.0), True: f32(57344.0) / f32(15.0)}
FMAX = {False: f32(448.0), True: f32(57344.0)}


@pytest.mark.parametrize("e5m2", [False, True])
@pytest.mark.parametrize("mx_exp", [0, -10, 7])
def test_fp8_grid_points_are_fixed_points(e5m2, mx_exp):
    """With amax = fp8_max * 2^e the MX scale is exactly 2^e, so v = j * step * 2^e (every
    grid point, j = -steps..steps) must come back unchanged."""
    steps = 15 if e5m2 else 31
    step, sc = STEP[e5m2], f32(2.0 ** mx_exp)
    j = np.arange(-steps, steps + 1, dtype=f32)
    v = (j * step) * sc
    v = np.concatenate([v, np.zeros(-v.size % 32, f32)])  # whole 32-blocks (block_size 32)
    blocks = v.reshape(-1, 32).copy()
    blocks[:, 0] = FMAX[e5m2] * sc  # every block's absmax fixes its scale to 2^e
    v = blocks.ravel()
    deq = O.quantize_fp8_grid(v, e5m2=e5m2, mxfp8=True, block_size=32)
    assert np.array_equal(deq, v)


@pytest.mark.parametrize("e5m2", [False, True])
def test_fp8_grid_ties_round_away_from_zero(e5m2):
    """Values whose f32 quotient v / step is exactly k + 0.5 (found by searching f32
    neighbours of (k + 0.5) * step, scale 1) round to k + 1 away from zero; half-even would
    take the even k for even k."""
    step = STEP[e5m2]
    ties, want = [], []
    for k in range(0, 15 if e5m2 else 31):
        c = f32((k + 0.5) * float(step))
        for d in range(-4, 5):
            x = np.nextafter(c, np.inf if d > 0 else -np.inf, dtype=f32) if d else c
            for _ in range(abs(d) - 1):
                x = np.nextafter(x, np.inf if d > 0 else -np.inf, dtype=f32)
            if x / step == f32(k + 0.5):
                ties += [x, -x]
                want += [f32(k + 1) * step, -(f32(k + 1) * step)]
                break
    assert len(ties) >= 20  # exact ties exist for most k
    n = len(ties)
    v = np.array(ties + [FMAX[e5m2]] * (32 - n % 32), f32)  # amax = fp8_max: scale 1
    # one block holding everything (block_size covers the whole tensor)
    deq = O.quantize_fp8_grid(v, e5m2=e5m2, mxfp8=True, block_size=v.size)
    assert np.array_equal(deq[:n], np.array(want, f32))
    even = [k for k in range(31) if k % 2 == 0]
    assert even  # half-even differs from half-away on these


@pytest.mark.parametrize("e5m2", [False, True])
def test_fp8_grid_max_maps_to_last_step(e5m2):
    """The block's absmax element lands on +-steps grid steps (31 for E4M3, 15 for E5M2),
    never beyond fp8_max: 448 = 31 * (448 / 31), 57344 = 15 * (57344 / 15)."""
    rng = np.random.default_rng(5)
    for mx in (True, False):
        v = (rng.standard_normal(256) * 3).astype(f32)
        v[7] = -np.abs(v).max() * 1.5
        deq = O.quantize_fp8_grid(v, e5m2=e5m2, mxfp8=mx, block_size=256)
        a = np.abs(v).max()
        raw = a / FMAX[e5m2]
        scale = f32(2.0 ** math.ceil(math.log2(raw))) if mx else raw
        steps = 15 if e5m2 else 31
        q = np.abs(np.float64(deq[7]) / (np.float64(STEP[e5m2]) * np.float64(scale)))
        assert round(q) <= steps and abs(q - round(q)) < 1e-5
        if not mx:
            assert round(q) == steps


@pytest.mark.parametrize("e5m2", [False, True])
def test_fp8_grid_plain_scale_closed_form(e5m2):
    """mxfp8 = false: scale = amax / fp8_max and step = fp8_max / steps, so deq =
    round(steps * v / amax) * amax / steps up to f32 rounding: the integer multiplier equals
    the f64 closed form's (away from exact ties) and the value is within a few ulps."""
    steps = 15 if e5m2 else 31
    rng = np.random.default_rng(11)
    v = (rng.standard_normal(64 * 32) * rng.choice([1e-3, 1.0, 50.0], 64).repeat(32)).astype(f32)
    deq = O.quantize_fp8_grid(v, e5m2=e5m2, mxfp8=False, block_size=32)
    for b in range(64):
        blk = v[32 * b:32 * b + 32].astype(np.float64)
        amax = np.abs(blk).max()
        t = steps * blk / amax
        far = np.abs(np.abs(t - np.trunc(t)) - 0.5) > 1e-4  # not near a tie
        mult = np.trunc(t + np.copysign(0.5, t))
        ref = mult * amax / steps
        got = deq[32 * b:32 * b + 32].astype(np.float64)
        np.testing.assert_allclose(got[far], ref[far], rtol=4e-7, atol=0)
        gm = np.round(got / (amax / steps))
        assert np.array_equal(gm[far], mult[far])


# ------------------------------------------------------------------------ epilogues ----
MODES = {"bias": 1, "relu": 2, "tanh": 3, "silu": 4, "gelu": 5, "scale": 6}


def _epi(out, bias, z, mode):
    o = np.array(out, f32)
    b = np.array(bias, f32)
    zz = None if z is None else np.array(z, f32)
    O.lib().orc_epilogue(O._p(o), o.size, O._p(b), b.size, None if zz is None else O._p(zz),
                         0 if zz is None else zz.size, MODES[mode])
    return o


def test_relu_epilogue_known_answers():
    """val = mm + bias[i % len]; relu is val.max(z[i % len]) with z = 0 by default, and
    f32::max ignores NaN (NaN.max(0) = 0)."""
    assert _epi([1.0, -2.0, 0.5, np.nan], [0.5], None, "relu").tolist() == [1.5, 0.0, 1.0, 0.0]
    assert _epi([1.0, -2.0, 0.5, -9.0], [0.5, -1.0], [-1.0, 3.0], "relu").tolist() == [1.5, 3.0, 1.0, 3.0]


def test_scale_epilogue_known_answers():
    """bias_scale: (mm + bias) * z[i % len]; z defaults to 0."""
    assert _epi([1.0, -2.0, 0.5], [0.5], [2.0, -0.25, 4.0], "scale").tolist() == [3.0, 0.375, 4.0]
    assert _epi([1.0, -2.0], [0.5], None, "scale").tolist() == [0.0, -0.0]


def _gelu64(x):
    """Hendrycks & Gimpel's tanh approximation, float64."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def test_gelu_epilogue_is_the_tanh_form():
    x = np.concatenate([np.linspace(-6, 6, 241), [-20.0, -3e-3, 0.0, 1e-7, 3.0, 20.0]]).astype(f32)
    got = _epi(x, [0.0], None, "gelu").astype(np.float64)
    ref = _gelu64(x.astype(np.float64))
    # f32 evaluation of the same formula: a few ulps of |x| plus tanh's near 1
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-7)
    # the known answer gelu(1) = 0.841192 (tanh form); the erf form gives 0.841345
    g1 = _epi([1.0], [0.0], None, "gelu")[0]
    assert abs(g1 - 0.8411920) < 2e-7
    assert abs(g1 - 0.5 * (1 + math.erf(1 / math.sqrt(2)))) > 1e-4
    assert _epi([0.0], [0.0], None, "gelu")[0] == 0.0
    # a constant off in its fourth digit is visible: 0.7978 instead of 0.7978846
    wrong = 0.5 * 1.0 * (1.0 + math.tanh(0.7978 * (1.0 + 0.044715)))
    assert abs(g1 - wrong) > 2e-5


def test_tanh_silu_epilogues_vs_float64():
    x = np.linspace(-12, 12, 97).astype(f32)
    t = _epi(x, [0.25], None, "tanh").astype(np.float64)
    np.testing.assert_allclose(t, np.tanh(x.astype(np.float64) + 0.25), rtol=2e-7, atol=1e-7)
    s = _epi(x, [0.25], None, "silu").astype(np.float64)
    v = x.astype(np.float64) + 0.25
    np.testing.assert_allclose(s, v / (1.0 + np.exp(-v)), rtol=1e-6, atol=1e-7)


# --------------------------------------------------- composed dequant + matmul functions ----
# orc_gemm_w8a16 / orc_gemm_nf4 / orc_gemm_fp8 restate eval.rs:303-318 (dequantize the constant
# to f32) followed by eval_matmul_2d (eval.rs:1465-1507) over packed [N, K] weights.  Each is
# checked against float64 products of weights decoded here from their bit layouts with numpy
# (nibble k % 8 of word k / 8, block k // b, E4M3 through torch's float8 view), so a wrong
# nibble order, block index, scale index (row vs column), or a transposed operand fails.
def _nibbles(codes: np.ndarray, k: int) -> np.ndarray:
    return np.stack([(codes >> (4 * i)) & 15 for i in range(8)], axis=-1).reshape(codes.shape[0], k)


def test_dequantize_nf4_is_table_times_block_absmax():
    """Bit-exact: out[r, i] = T[code] * absmax[r, i // block] as one f32 product; the absmax of
    each block differs so a wrong block index changes the bits."""
    rng = np.random.default_rng(101)
    for n, k, block in [(5, 256, 32), (3, 512, 64), (4, 384, 128)]:
        codes = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
        absmax = (rng.random((n, (k + block - 1) // block)) * 3 + 0.5).astype(np.float32)
        got = O.dequantize_nf4(codes, absmax, n, k, block)
        t = O.nf4_table().astype(np.float32)
        want = (t[_nibbles(codes, k)] * np.repeat(absmax, block, axis=1)[:, :k]).astype(np.float32)
        assert np.array_equal(got, want)


def test_gemm_nf4_oracle_vs_float64():
    rng = np.random.default_rng(102)
    n, k, m, block = 20, 512, 3, 64
    codes = rng.integers(0, 2 ** 32, (n, k // 8), dtype=np.uint64).astype(np.uint32)
    absmax = (rng.random((n, k // block)) * 0.05 + 0.01).astype(np.float32)
    x = O.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    y = O.gemm_nf4(x, codes, absmax, n, k, block)
    t = O.nf4_table().astype(np.float64)
    w = t[_nibbles(codes, k)] * np.repeat(absmax.astype(np.float64), block, axis=1)
    ref = O.bf16_bits_to_f32(x).astype(np.float64) @ w.T
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_gemm_w8a16_oracle_vs_float64():
    """Per-row (output channel) scales: swapping rows and columns of the scale, or reading
    the codes unsigned, fails."""
    rng = np.random.default_rng(103)
    n, k, m = 24, 320, 4
    codes = rng.integers(-127, 128, (n, k)).astype(np.int8)
    scales = (rng.random(n) * 0.01 + 1e-3).astype(np.float32)
    x = O.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    y = O.gemm_w8a16(x, codes, scales)
    ref = O.bf16_bits_to_f32(x).astype(np.float64) @ (codes.astype(np.float64) * scales[:, None].astype(np.float64)).T
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_gemm_fp8_oracle_vs_float64():
    """Activations per token (row of A) and weights per row of W, both E4M3FN codes: decoded
    here by torch's float8_e4m3fn view (not the oracle's codec)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(104)
    m, n, k = 6, 10, 256
    qa = rng.integers(0, 256, (m, k)).astype(np.uint8)
    qw = rng.integers(0, 256, (n, k)).astype(np.uint8)
    qa[(qa & 0x7F) == 0x7F] = 0x10   # the two NaN codes
    qw[(qw & 0x7F) == 0x7F] = 0x22
    sa = (rng.random(m) + 0.25).astype(np.float32)
    sw = (rng.random(n) * 0.01 + 1e-3).astype(np.float32)
    y = O.gemm_fp8(qa, sa, qw, sw)
    da = torch.from_numpy(qa).view(torch.float8_e4m3fn).double().numpy()
    dw = torch.from_numpy(qw).view(torch.float8_e4m3fn).double().numpy()
    ref = (da * sa[:, None].astype(np.float64)) @ (dw * sw[:, None].astype(np.float64)).T
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-5)


def test_quantize_int4g_awq_prescales_columns():
    """AWQ pre-scale W'[r, c] = f32(W[r, c] * s[c]) (per input channel, i.e. column):
    * s = 1 gives the plain quantizer's arrays;
    * s = 2^j for all columns leaves codes and zero points unchanged and multiplies every f16
      scale by exactly 2^j (every step of the quantizer is homogeneous in powers of two);
    * per-column s on a non-square matrix matches the plain quantizer of numpy's f32 W * s,
      and not of W * s applied along rows."""
    rng = np.random.default_rng(105)
    n, k = 12, 384
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    base = O.quantize_int4g(w, 128)
    for a, b in zip(O.quantize_int4g_awq(w, np.ones(k, np.float32), 128), base):
        assert np.array_equal(a, b)
    c4, s4, z4 = O.quantize_int4g_awq(w, np.full(k, 4.0, np.float32), 128)
    assert np.array_equal(c4, base[0]) and np.array_equal(z4, base[2])
    g = k // 128
    assert np.array_equal(s4[:, :g].view(np.float16).astype(np.float32),
                          base[1][:, :g].view(np.float16).astype(np.float32) * 4)
    s = np.exp(rng.standard_normal(k) * 0.5).astype(np.float32)
    got = O.quantize_int4g_awq(w, s, 128)
    want = O.quantize_int4g((w * s[None, :]).astype(np.float32), 128)
    for a, b in zip(got, want):
        assert np.array_equal(a, b)
    wrong = O.quantize_int4g((w * s[:n, None]).astype(np.float32), 128)
    assert not np.array_equal(got[0], wrong[0])
