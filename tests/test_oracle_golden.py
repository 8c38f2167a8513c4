"""Pins the CPU oracle: the reference's own known answers, independent implementations
(numpy / torch converters, scipy's normal quantiles) and brute force on small inputs."""
import json
import math
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle_lib as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


# ------------------------------------------------------------ reference known answers ----
def test_int_bounds_known_answer():
    import ctypes
    for bits, (eb, qmin, qmax) in GOLDEN["int_bounds"].items():
        e, lo, hi = ctypes.c_int(), ctypes.c_float(), ctypes.c_float()
        O.lib().orc_int_bounds(int(bits), ctypes.byref(e), ctypes.byref(lo), ctypes.byref(hi))
        assert (e.value, lo.value, hi.value) == (eb, qmin, qmax)
    # anything other than 4 takes the 8-bit bounds (formats.rs:655-659)
    e, lo, hi = ctypes.c_int(), ctypes.c_float(), ctypes.c_float()
    O.lib().orc_int_bounds(3, ctypes.byref(e), ctypes.byref(lo), ctypes.byref(hi))
    assert (e.value, lo.value, hi.value) == (8, -128.0, 127.0)


def test_int8_per_tensor_known_answer():
    g = GOLDEN["int8_per_tensor"]
    q, s = O.quantize_symmetric(np.array(g["weights"], np.float32), 8, 0)
    assert q.tolist() == g["codes"]
    assert f32_bits(float(s)) == g["scale_bits"]
    assert O.scale_string(float(s)) == g["scale_string"]
    sc = np.float32(float(g["scale_string"]))
    deq = q.astype(np.float32) * sc
    np.testing.assert_allclose(deq, g["dequant_with_string_scale"], rtol=0, atol=5e-7)


def test_scale_string_forms():
    assert O.scale_string(1.0) == "1.0"
    assert O.scale_string(0.5) == "0.5"
    assert O.scale_string(2.0) == "2.0"
    assert O.scale_string(1e-9) == "0.0"
    assert O.scale_string(0.1234564) == "0.123456"


def test_e4m3_known_answers():
    g = GOLDEN["e4m3fn"]
    for v, code in g["encode"]:
        f = float("nan") if v == "nan" else v
        assert O.lib().orc_f32_to_e4m3fn(f) == code
        assert O.lib().orc_f32_to_e4m3fn_fast(f) == code
    for code, v in g["decode"]:
        out = O.lib().orc_e4m3fn_to_f32(code)
        assert math.isnan(out) if v == "nan" else out == v
    for v in g["roundtrip"]:
        c = O.lib().orc_f32_to_e4m3fn(v)
        assert O.lib().orc_e4m3fn_to_f32(c) == v


def test_f16_trunc_known_answer():
    for v, bits in GOLDEN["f16_trunc"]:
        assert O.lib().orc_f32_to_f16_trunc(v) == bits


def test_awq_salient_count_known_answer():
    g = GOLDEN["awq_salient_count"]
    w = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    _, _, cnt, thr = O.quantize_groupwise(w, bits=4, group_size=2, awq_salient=True,
                                          salient_ratio=g["ratio"])
    assert cnt == g["count"]
    assert thr == 4.0


def test_eval_synthetic_formula():
    got = [((i * 7 + 0 * 13 + 3) % 19 - 9) * 0.1 for i in range(8)]
    assert got == pytest.approx(GOLDEN["eval_synthetic_arg0"])


# ---------------------------------------------------------------- E4M3 codec pins ----
def test_e4m3_quirk_encoder_equals_faithful_codec_everywhere():
    """Every one of the 2^32 f32 patterns: the quirk-aware integer encoder (the rule the GPU
    implements) equals the faithful restatement of the reference codec."""
    import ctypes
    fb = ctypes.c_uint32()
    bad = O.lib().orc_e4m3_crosscheck(0, 0xFFFFFFFF, 1, 1, ctypes.byref(fb))
    assert bad == 0, hex(fb.value)
    last = 0xFFFFFFFF
    assert O.lib().orc_f32_to_e4m3fn(struct.unpack("<f", struct.pack("<I", last))[0]) == \
        O.lib().orc_f32_to_e4m3fn_fast(struct.unpack("<f", struct.pack("<I", last))[0])


def test_e4m3_reference_quirk_is_exactly_32_patterns():
    """The reference's log2-based exponent differs from true RNE on exactly 16 magnitudes."""
    import ctypes
    fb = ctypes.c_uint32()
    bad = O.lib().orc_e4m3_crosscheck(0, 0xFFFFFFFF, 1, 0, ctypes.byref(fb))
    assert bad == 32 and fb.value == 0x3CFFFFFE


def test_e4m3_matches_torch_float8_rne_inside_range():
    """torch's float8_e4m3fn cast (RNE) is an independent encoder for |v| < 448."""
    rng = np.random.default_rng(0)
    v = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(40.0),
        rng.uniform(-447.9, 447.9, 100000).astype(np.float32),
        (rng.standard_normal(50000) * 1e-3).astype(np.float32),
        np.arange(-448, 448, 0.0625, dtype=np.float32),   # many exact ties
    ])
    v = v[np.abs(v) < 448]
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ours = np.array([O.lib().orc_f32_to_e4m3fn_int(float(x)) for x in v[:20000]], np.uint8)
    assert np.array_equal(ours, ref[:20000])
    # decode: all 256 codes against torch
    codes = np.arange(256, dtype=np.uint8)
    tdec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    odec = np.array([O.lib().orc_e4m3fn_to_f32(int(c)) for c in codes], np.float32)
    both_nan = np.isnan(tdec) & np.isnan(odec)
    assert np.array_equal(np.where(both_nan, 0, tdec).view(np.uint32), np.where(both_nan, 0, odec).view(np.uint32))


# ------------------------------------------------------------------ f16 / bf16 pins ----
def test_f16_rne_matches_numpy_everywhere_sampled():
    xs = np.arange(0, 2**32, 9973, dtype=np.uint64).astype(np.uint32)
    xs = np.concatenate([xs, np.array([0x33000000, 0x33000001, 0x387FE000, 0x38800000, 0x477FEFFF,
                                       0x477FF000, 0x7F800000, 0xFF800000], np.uint32)])
    f = xs.view(np.float32)
    ref = f.astype(np.float16).view(np.uint16)
    ours = np.array([O.lib().orc_f32_to_f16_rne(float(x)) for x in f], np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all((ours[nan] & 0x7C00) == 0x7C00) and np.all((ours[nan] & 0x3FF) != 0)


def test_f16_to_f32_exact_all_codes():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    ours = np.array([O.lib().orc_f16_to_f32(int(x)) for x in h], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(ours[nan]))


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    f = np.concatenate([rng.standard_normal(50000).astype(np.float32),
                        np.array([1.00390625, 1.01171875, -3.0e38, 1e-40], np.float32)])
    ref = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ours = np.array([O.lib().orc_f32_to_bf16_rne(float(x)) for x in f], np.uint16)
    assert np.array_equal(ours, ref)
    assert np.array_equal(O.f32_to_bf16_bits(f), ref)


# ----------------------------------------------------------------- INT8 invariants ----
@pytest.mark.parametrize("mode", [0, 1])
def test_int8_invariants(mode):
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 96)) * 0.02).astype(np.float32)
    q, s = O.quantize_int8_rows(w, 8, mode)
    for r in range(64):
        am = np.abs(w[r]).max()
        assert s[r] == np.float32(am) / np.float32(127.0)
        i = np.abs(w[r]).argmax()
        assert abs(int(q[r, i])) == 127
    assert np.abs(q.astype(np.int32)).max() <= 127
    # brute force vs an independent numpy restatement
    sc = (np.abs(w).max(axis=1) / np.float32(127)).astype(np.float32)
    t = (w / sc[:, None]).astype(np.float32)
    if mode == 1:
        r = np.rint(t)
    else:
        r = np.sign(t) * np.floor(np.abs(t) + np.float32(0.5))
    assert np.array_equal(q, np.clip(r, -128, 127).astype(np.int8))


def test_int8_ties_and_specials():
    # exact ties: v/scale = k + 0.5 with scale 1 (amax 127)
    w = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -2.5, np.nan, 0.0, -0.0], np.float32)
    qa, _ = O.quantize_symmetric(w, 8, 0)
    qe, _ = O.quantize_symmetric(w, 8, 1)
    assert qa.tolist() == [127, 1, 2, 3, -1, -3, 0, 0, 0]
    assert qe.tolist() == [127, 0, 2, 2, 0, -2, 0, 0, 0]
    # all-zero tensor -> scale 1.0 (formats.rs:674)
    _, s = O.quantize_symmetric(np.zeros(5, np.float32), 8, 0)
    assert s == 1.0
    # bits=4 clamps to [-8, 7]
    q4, s4 = O.quantize_symmetric(np.array([-7.0, 7.0, -8.0], np.float32), 4, 0)
    assert s4 == np.float32(8.0) / np.float32(7.0) and q4.tolist() == [-6, 6, -7]


# ----------------------------------------------------------------- INT4 asym g128 ----
def _int4_numpy(w, group):
    """Independent numpy restatement (numpy's own f16 RNE and rint)."""
    n, k = w.shape
    G = (k + group - 1) // group
    codes = np.zeros((n, k), np.uint32)
    scales = np.zeros((n, (G + 7) // 8 * 8), np.uint16)
    zeros = np.zeros((n, G), np.uint32)
    for g in range(G):
        blk = w[:, g * group:(g + 1) * group]
        mx = np.nanmax(blk, axis=1).astype(np.float32)
        mn = np.nanmin(blk, axis=1).astype(np.float32)
        rng_ = (mx - mn).astype(np.float32)
        h = np.where(rng_ >= np.float32(1e-12), (rng_ / np.float32(15)).astype(np.float16), np.float16(1.0))
        hb = h.view(np.uint16).copy()
        hb[hb == 0] = 1
        hb[hb == 0x7C00] = 0x7BFF
        s = hb.view(np.float16).astype(np.float32)
        z = np.clip(np.rint(-mn / s), 0, 15)
        q = np.clip(np.rint(blk / s[:, None]) + z[:, None], 0, 15)
        codes[:, g * group:(g + 1) * group] = q.astype(np.uint32)
        scales[:, g] = hb
        zeros[:, g] = z.astype(np.uint32)
    packed = np.zeros((n, k // 8), np.uint32)
    for j in range(8):
        packed |= codes[:, j::8] << np.uint32(4 * j)
    zw = np.zeros((n, (G + 7) // 8), np.uint32)
    for g in range(G):
        zw[:, g // 8] |= zeros[:, g] << np.uint32(4 * (g % 8))
    return packed, scales, zw


@pytest.mark.parametrize("shape,group", [((8, 256), 128), ((5, 200), 64), ((3, 136), 128), ((4, 64), 32), ((2, 512), 256)])
def test_int4g_matches_numpy_restatement(shape, group):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    a = O.quantize_int4g(w, group)
    b = _int4_numpy(w, group)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_int4g_closed_forms():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((16, 1024)) * 0.02).astype(np.float32)
    codes, scales, zeros = O.quantize_int4g(w, 128)
    q = np.stack([(codes >> np.uint32(4 * j)) & 15 for j in range(8)], axis=-1).reshape(16, 1024)
    for r in range(16):
        for g in range(8):
            blk = w[r, g * 128:(g + 1) * 128]
            qq = q[r, g * 128:(g + 1) * 128]
            assert qq[blk.argmin()] == 0          # the minimum maps to code 0 (min <= 0 here)
            assert qq[blk.argmax()] >= 14         # the maximum maps to the top of the range
    deq = O.dequantize_int4g(codes, scales, zeros, 16, 1024, 128)
    s = np.repeat(scales[:, :8].view(np.float16).astype(np.float32), 128, axis=1)
    assert np.all(np.abs(deq - w) <= s * 1.0 + 1e-7)   # rounding of v/s and of z: <= s


def test_int4g_edge_groups():
    w = np.zeros((3, 128), np.float32)
    w[1, :] = 0.25                         # constant group: range 0 -> scale 1.0
    w[2, :5] = np.nan                      # NaN codes dequantize to 0
    w[2, 5:] = np.linspace(-1, 1, 123, dtype=np.float32)
    codes, scales, zeros = O.quantize_int4g(w, 128)
    assert scales[0, 0] == 0x3C00 and scales[1, 0] == 0x3C00
    deq = O.dequantize_int4g(codes, scales, zeros, 3, 128, 128)
    assert np.all(deq[0] == 0)
    assert np.all(deq[2, :5] == 0)


# --------------------------------------------------------------------------- NF4 ----
def test_nf4_table_is_the_normal_float_construction():
    """QLoRA NF4: 8 positive quantiles of N(0,1) over linspace(offset, 0.5, 9)[:-1] and 7
    negative ones over linspace(offset, 0.5, 8)[:-1], offset 0.9677083, plus 0, normalised."""
    from scipy.stats import norm
    off = 0.9677083
    v1 = norm.ppf(np.linspace(off, 0.5, 9)[:-1])
    v3 = -norm.ppf(np.linspace(off, 0.5, 8)[:-1])
    v = np.sort(np.concatenate([v1, [0.0], v3]))
    v = v / np.abs(v).max()
    np.testing.assert_allclose(O.nf4_table(), v, rtol=0, atol=2e-7)


def test_nf4_code_is_nearest_entry():
    T = O.nf4_table().astype(np.float64)
    xs = np.concatenate([np.linspace(-1, 1, 20001), [-1.0, 0.0, 1.0, -1e-30, 1e-30]]).astype(np.float32)
    for x in xs:
        c = O.lib().orc_nf4_code(float(x))
        d = np.abs(T - float(x))
        best = d.min()
        assert d[c] <= best + 1e-7, (x, c)
    assert O.lib().orc_nf4_code(float("nan")) == 7
    assert O.lib().orc_nf4_code(-1.0) == 0 and O.lib().orc_nf4_code(1.0) == 15 and O.lib().orc_nf4_code(0.0) == 7


def test_nf4_roundtrip_bound():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((8, 640)) * 0.02).astype(np.float32)
    codes, absmax = O.quantize_nf4(w, 64)
    deq = O.dequantize_nf4(codes, absmax, 8, 640, 64)
    T = O.nf4_table()
    maxgap = np.max(np.diff(T)) / 2
    am = np.repeat(absmax, 64, axis=1)
    assert np.all(np.abs(deq - w) <= am * maxgap + 1e-7)
    assert np.allclose(absmax, np.abs(w).reshape(8, 10, 64).max(-1))


# --------------------------------------------------------------------------- FP8 ----
def test_fp8_rows_scale_and_range():
    rng = np.random.default_rng(6)
    v = rng.standard_normal((16, 300)).astype(np.float32)
    v[3, 7] = 30.0
    codes, scales = O.quantize_fp8_rows(v)
    assert np.array_equal(scales, (np.abs(v).max(1) / np.float32(448)).astype(np.float32))
    dec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.all(np.abs(dec) <= 448)
    rowmax = np.abs(dec).max(axis=1)
    assert np.all(rowmax == 448.0)
    rel = np.abs(dec * scales[:, None] - v) / np.maximum(np.abs(v), 1e-3)
    assert np.median(rel) < 0.04


# ---------------------------------------------------------------- evaluator GEMM ----
def test_matmul_2d_exact_on_small_integers():
    rng = np.random.default_rng(7)
    a = rng.integers(-8, 8, (5, 33)).astype(np.float32)
    b = rng.integers(-8, 8, (33, 7)).astype(np.float32)
    assert np.array_equal(O.matmul_2d(a, b, False), (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))
    assert np.array_equal(O.matmul_2d(a, np.ascontiguousarray(b.T), True), O.matmul_2d(a, b, False))


def test_matmul_2d_sequential_f32_accumulation():
    """k ascending, f32 accumulator, separately rounded products (no FMA)."""
    rng = np.random.default_rng(8)
    a = rng.standard_normal((2, 257)).astype(np.float32)
    b = rng.standard_normal((257, 3)).astype(np.float32)
    ref = np.zeros((2, 3), np.float32)
    for i in range(2):
        for j in range(3):
            acc = np.float32(0)
            for kk in range(257):
                acc = np.float32(acc + np.float32(a[i, kk] * b[kk, j]))
            ref[i, j] = acc
    assert np.array_equal(O.matmul_2d(a, b, False), ref)


def test_gemm_w4a16_oracle_vs_float64():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((24, 256)) * 0.02).astype(np.float32)
    codes, scales, zeros = O.quantize_int4g(w, 128)
    x = O.f32_to_bf16_bits(rng.standard_normal((3, 256)).astype(np.float32))
    y = O.gemm_w4a16(x, codes, scales, zeros, 24, 256, 128)
    deq = O.dequantize_int4g(codes, scales, zeros, 24, 256, 128).astype(np.float64)
    ref = O.bf16_bits_to_f32(x).astype(np.float64) @ deq.T
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)


def test_dot_general_flat_oracle_vs_float64():
    """The batched / rank-3 form of eval_dot_general (eval.rs:1509-1604): every batch against a
    float64 product of the same slices, both rhs layouts; batch = 1 is eval_matmul_2d itself,
    and a batch-swapped rhs (a plausible indexing slip) is caught."""
    rng = np.random.default_rng(12)
    bt, m, k, n = 3, 5, 40, 7
    a = rng.standard_normal((bt, m, k)).astype(np.float32)
    bkn = rng.standard_normal((bt, k, n)).astype(np.float32)
    bnk = np.ascontiguousarray(bkn.transpose(0, 2, 1))
    ref = np.einsum("bmk,bkn->bmn", a.astype(np.float64), bkn.astype(np.float64))
    bound = 1e-6 * np.einsum("bmk,bkn->bmn", np.abs(a).astype(np.float64), np.abs(bkn).astype(np.float64))
    for y in (O.dot_general_flat(a, bkn, bt, k, False), O.dot_general_flat(a, bnk, bt, k, True)):
        assert y.shape == (bt, m, n)
        assert np.all(np.abs(y - ref) <= bound)
    assert np.array_equal(O.dot_general_flat(a[:1], bkn[:1], 1, k, False)[0], O.matmul_2d(a[0], bkn[0], False))
    wrong = O.dot_general_flat(a, bkn[::-1].copy(), bt, k, False)
    assert not np.all(np.abs(wrong - ref) <= bound)
    with pytest.raises(ValueError):
        O.dot_general_flat(a, bkn[:, :, :3].reshape(-1)[:-1], bt, k, False)


def test_epilogues():
    out = np.array([1.0, -2.0, 0.5], np.float32)
    bias = np.array([0.5], np.float32)
    for mode, fn in [(1, lambda v: v), (3, np.tanh), (4, lambda v: v / (1 + np.exp(-v)))]:
        o = out.copy()
        O.lib().orc_epilogue(O._p(o), 3, O._p(bias), 1, None, 0, mode)
        np.testing.assert_allclose(o, fn(out + 0.5), rtol=1e-6)


def test_mx_scale_exponent_closed_form_matches_glibc_log2f():
    """The MX scale exponent ceilf(log2f(amax / max)) (schemes.rs:706), computed by the GPU
    kernel in closed form, equals glibc's ceilf(log2f(x)) for every positive normal f32 x
    (2^31 inputs); 3676 of them sit just above a power of two where log2f rounds to the
    integer and the reference keeps the smaller scale."""
    import ctypes

    first = ctypes.c_uint32(0)
    bad = O.lib().orc_mx_scale_crosscheck(0x00800000, 0x7F800000, ctypes.byref(first))
    assert bad == 0, f"first mismatch at bits {first.value:#010x}"
    quirks = 0
    for e in range(-126, 128):
        for m in range(1, 64):
            x = np.array([(e + 127) << 23 | m], np.uint32).view(np.float32)[0]
            quirks += O.lib().orc_mx_scale_exp_model(float(x)) == e
    assert quirks == 3676
