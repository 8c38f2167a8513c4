"""GPU parity of the quantize / dequantize kernels against the CPU oracle: bit-exact codes,
scales and zero points on the same seeded inputs, edge cases, and the BASELINE block shapes."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ops, synth

pytestmark = pytest.mark.gpu

SPECIALS = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-30, -1e-38, 3.0e38], np.float32)


def _w(seed, n, k, std=0.02, specials=False):
    w = synth.weight(seed, 1, n, k, std)
    if specials and w.size >= 64:
        flat = w.reshape(-1)
        r = synth.rng(seed, 2)
        idx = r.choice(flat.size, size=min(len(SPECIALS) * 2, flat.size // 4), replace=False)
        flat[idx] = np.resize(SPECIALS, idx.size)
    return w


def _u32(t):
    return t.cpu().numpy().view(np.uint32)


# --------------------------------------------------------------------------- INT8 ----
@pytest.mark.parametrize("n,k", [(64, 96), (7, 13), (33, 4096), (3, 70000), (1, 4), (5, 11008)])
@pytest.mark.parametrize("mode", ["half_away", "half_even"])
def test_int8_per_channel_bit_exact(cuda, n, k, mode):
    w = _w(11, n, k, specials=(n * k >= 200))
    q_ref, s_ref = O.quantize_int8_rows(w, 8, 0 if mode == "half_away" else 1)
    q, s = ops.quantize_int8(torch.from_numpy(w).to(cuda), 8, "channel", mode)
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_int8_ties_exact(cuda):
    # v/scale lands exactly on .5 (scale = 1 with amax 127)
    w = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -2.5, -126.5, 126.5]], np.float32)
    for mode, m in (("half_away", 0), ("half_even", 1)):
        q_ref, _ = O.quantize_int8_rows(w, 8, m)
        q, _ = ops.quantize_int8(torch.from_numpy(w).to(cuda), 8, "channel", mode)
        assert np.array_equal(q.cpu().numpy(), q_ref)


def _ulp_steps(v, d):
    """v moved by d units in the last place (f32 bit pattern arithmetic, sign kept)."""
    u = v.view(np.int32).astype(np.int64) + d
    return u.astype(np.int32).view(np.float32)


@pytest.mark.parametrize("mode", ["half_away", "half_even"])
@pytest.mark.parametrize("bits", [8, 4])
def test_int8_rows_ties_many_scale_decades(cuda, mode, bits):
    # Each row has its own absmax (1e-10 .. 1e30), so scale = amax / qmax is an arbitrary f32;
    # the other values sit on exact ties (k + 1/2) * scale and +-1..3 ulp around them, where a
    # quotient one ulp off changes the code.
    qmax = 127 if bits == 8 else 7
    rows, cols = 384, 1024
    r = np.random.default_rng(7 + bits)
    amax = (10.0 ** r.uniform(-10, 30, rows)).astype(np.float32)
    scale = amax / np.float32(qmax)
    k = r.integers(-qmax, qmax, (rows, cols)).astype(np.float32)
    w = ((k + np.float32(0.5)) * scale[:, None]).astype(np.float32)
    w = _ulp_steps(w, r.integers(-3, 4, (rows, cols)))
    w = np.clip(w, -amax[:, None], amax[:, None])
    w[:, 0] = amax * np.where(r.random(rows) < 0.5, 1, -1).astype(np.float32)
    w[:4, 1:5] = [np.inf, -np.inf, np.nan, 0.0]  # rows 0..3: infinite absmax, NaN values
    q_ref, s_ref = O.quantize_int8_rows(w, bits, 0 if mode == "half_away" else 1)
    q, s = ops.quantize_int8(torch.from_numpy(w).to(cuda), bits, "channel", mode)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize("shape", [(2, 2), (1, 1), (4096, 4096), (1, 1001), (3, 5, 7)])
def test_int8_per_tensor_bit_exact(cuda, shape):
    w = synth.weight(12, 3, int(np.prod(shape[:-1])), shape[-1]).reshape(shape)
    q_ref, s_ref = O.quantize_symmetric(w, 8, 0)
    q, s = ops.quantize_int8(torch.from_numpy(w).to(cuda), 8, "tensor", "half_away")
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert s.cpu().numpy()[0].view(np.uint32) == np.float32(s_ref).view(np.uint32)


def test_int8_reference_known_answer(cuda):
    w = torch.tensor([[0.5, -0.25], [0.75, 0.5]], device=cuda)
    q, s = ops.quantize_int8(w, 8, "tensor", "half_away")
    assert q.cpu().flatten().tolist() == [85, -42, 127, 85]
    assert s.cpu().numpy().view(np.uint32)[0] == 0x3BC18306


def test_int4_symmetric_bits4(cuda):
    w = _w(13, 16, 256)
    q_ref, s_ref = O.quantize_int8_rows(w, 4, 0)
    q, s = ops.quantize_int8(torch.from_numpy(w).to(cuda), 4, "channel", "half_away")
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)


def test_int8_dequant_matches_oracle(cuda):
    w = _w(14, 32, 100)
    q, s = ops.quantize_int8(torch.from_numpy(w).to(cuda), 8, "channel", "half_even")
    d = ops.dequantize_int8(q, s, "channel").cpu().numpy()
    ref = q.cpu().numpy().astype(np.float32) * s.cpu().numpy()[:, None]
    assert np.array_equal(d, ref)


# -------------------------------------------------------------------------- INT4g ----
@pytest.mark.parametrize("group", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("n,k", [(16, 1024), (5, 200), (3, 11008), (1, 8)])
def test_int4g_bit_exact(cuda, group, n, k):
    w = _w(21, n, k, specials=(n * k >= 1024))
    c_ref, s_ref, z_ref = O.quantize_int4g(w, group)
    p = ops.quantize_int4g(torch.from_numpy(w).to(cuda), group)
    assert np.array_equal(_u32(p.codes), c_ref)
    assert np.array_equal(p.scales.cpu().numpy().view(np.uint16), s_ref)
    assert np.array_equal(_u32(p.zeros), z_ref)
    d = ops.dequantize_int4g(p).cpu().numpy()
    d_ref = O.dequantize_int4g(c_ref, s_ref, z_ref, n, k, group)
    assert np.array_equal(d.view(np.uint32), d_ref.view(np.uint32))


@pytest.mark.parametrize("group", [16, 128, 256])
def test_int4g_exact_ties_every_scale_decade(cuda, group):
    """Groups whose quotients x / s are exact halves (k + 0.5) and their neighbours one ulp
    away, for scales s from f16 subnormals to 2^15: the kernel's reciprocal-and-correction
    quotient must round every tie exactly as x / s does (round half to even)."""
    rng = np.random.default_rng(5)
    hs = np.concatenate([np.array([1, 2, 3, 0x3ff, 0x400, 0x3c00, 0x7bff], np.uint16),
                         rng.integers(1, 0x7c00, 120).astype(np.uint16)])
    svals = hs.view(np.float16).astype(np.float32)
    rows = []
    for sv in svals:
        g = np.zeros(group, np.float32)
        g[1] = np.float32(15) * sv                      # range 15 s: the scale is exactly s
        ties = (np.arange(group - 2) % 15 + np.float32(0.5)).astype(np.float32) * sv
        step = (np.arange(group - 2) % 3 - 1).astype(np.int32)  # -1, 0, +1 ulp
        g[2:] = (ties.view(np.int32) + step).view(np.float32)
        g[2:] = np.clip(g[2:], 0, g[1])
        rows.append(np.tile(g, 2))
    w = np.stack(rows).astype(np.float32)
    c_ref, s_ref, z_ref = O.quantize_int4g(w, group)
    p = ops.quantize_int4g(torch.from_numpy(w).to(cuda), group)
    assert np.array_equal(_u32(p.codes), c_ref)
    assert np.array_equal(p.scales.cpu().numpy().view(np.uint16), s_ref)
    assert np.array_equal(_u32(p.zeros), z_ref)


def test_int4g_edge_groups(cuda):
    w = np.zeros((4, 256), np.float32)
    w[1, :] = 0.25
    w[2, :5] = np.nan
    w[2, 5:] = np.linspace(-1, 1, 251, dtype=np.float32)
    w[3, :128] = 1e-9  # tiny range -> guarded scales
    w[3, 128:] = np.linspace(-70000, 70000, 128, dtype=np.float32)  # fp16 scale saturates
    c_ref, s_ref, z_ref = O.quantize_int4g(w, 128)
    p = ops.quantize_int4g(torch.from_numpy(w).to(cuda), 128)
    assert np.array_equal(_u32(p.codes), c_ref)
    assert np.array_equal(p.scales.cpu().numpy().view(np.uint16), s_ref)
    assert np.array_equal(_u32(p.zeros), z_ref)


@pytest.mark.parametrize("group", [32, 128, 256])
@pytest.mark.parametrize("n,k", [(16, 1024), (3, 11008), (12, 2304), (4096, 4096)])
def test_int4g_awq_prescale_bit_exact(cuda, group, n, k):
    """W' = W * a^0.5 per input channel, quantized INT4 g128 in one pass;
    codes / scales / zeros equal the oracle's quantization of f32(W * s).  Row counts that are
    multiples of 4 take the kernel's several-rows-per-thread form, 3 rows the one-row form."""
    w = _w(23, n, k, specials=(n * k >= 1024))
    s = synth.awq_channel_scales(23, 9, k)
    c_ref, s_ref, z_ref = O.quantize_int4g_awq(w, s, group)
    p = ops.quantize_int4g(torch.from_numpy(w).to(cuda), group, torch.from_numpy(s).to(cuda))
    assert np.array_equal(_u32(p.codes), c_ref)
    assert np.array_equal(p.scales.cpu().numpy().view(np.uint16), s_ref)
    assert np.array_equal(_u32(p.zeros), z_ref)


def test_int4g_awq_rejects_bad_scale(cuda):
    from castforge_amd.ffi import CastForgeHipError

    w = torch.zeros((4, 64), device=cuda)
    with pytest.raises(ValueError):
        ops.quantize_int4g(w, 32, torch.zeros(63, device=cuda))
    from castforge_amd import ffi
    p = ops.quantize_int4g(w, 32)
    with pytest.raises(CastForgeHipError, match="in_scale must not be NULL"):
        ffi.call("castforge_hip_quantize_int4g_awq", w.data_ptr(), None, 4, 64, 32, p.codes.data_ptr(),
                 p.scales.data_ptr(), p.zeros.data_ptr(), torch.cuda.current_stream().cuda_stream)


# ---------------------------------------------------------------------------- NF4 ----
@pytest.mark.parametrize("block", [8, 32, 64, 128, 512])
@pytest.mark.parametrize("n,k", [(16, 1024), (7, 200), (2, 11008)])
def test_nf4_bit_exact(cuda, block, n, k):
    w = _w(31, n, k, specials=(n * k >= 1024))
    c_ref, a_ref = O.quantize_nf4(w, block)
    p = ops.quantize_nf4(torch.from_numpy(w).to(cuda), block)
    assert np.array_equal(_u32(p.codes), c_ref)
    assert np.array_equal(p.absmax.cpu().numpy().view(np.uint32), a_ref.view(np.uint32))
    d = ops.dequantize_nf4(p).cpu().numpy()
    assert np.array_equal(d.view(np.uint32), O.dequantize_nf4(c_ref, a_ref, n, k, block).view(np.uint32))


# ---------------------------------------------------------------------------- FP8 ----
QUIRK = np.array([0x3CFFFFFE, 0x3CFFFFFF, 0x3D7FFFFE, 0x3D7FFFFF, 0x3DFFFFFF, 0x3E7FFFFF,
                  0x40FFFFFF, 0x417FFFFF, 0x41FFFFFE, 0x41FFFFFF, 0x427FFFFE, 0x427FFFFF,
                  0x42FFFFFE, 0x42FFFFFF, 0x437FFFFE, 0x437FFFFF], np.uint32).view(np.float32)


@pytest.mark.parametrize("r,c", [(16, 300), (5, 4096), (3, 7), (2, 70000)])
def test_fp8_rows_f32_bit_exact(cuda, r, c):
    v = synth.fp8_inputs(41, 1, r, c)
    c_ref, s_ref = O.quantize_fp8_rows(v)
    codes, scales = ops.quantize_fp8(torch.from_numpy(v).to(cuda))
    assert np.array_equal(codes.cpu().numpy(), c_ref)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_fp8_reference_quirk_inputs(cuda):
    # rows with amax 448 have scale exactly 1, so v/scale = v hits the 16 quirk magnitudes
    row = np.concatenate([[448.0], QUIRK, -QUIRK, [np.nan, 0.0, -0.0, 1e-3, 2.0 ** -10]]).astype(np.float32)
    v = np.stack([row, row[::-1].copy()])
    c_ref, s_ref = O.quantize_fp8_rows(v)
    codes, scales = ops.quantize_fp8(torch.from_numpy(v).to(cuda))
    assert np.array_equal(codes.cpu().numpy(), c_ref)
    assert s_ref[0] == 1.0


def test_fp8_rows_boundaries_many_scale_decades(cuda):
    # Per-row absmax 1e-10 .. 1e30 (scale = amax / 448 an arbitrary f32); values are
    # quotient * scale with quotients at E4M3 rounding midpoints, the log2 quirk thresholds and
    # the subnormal range, +-3 ulp, so a quotient one ulp off changes the code.  Rows 0..2
    # hold an infinity (infinite scale: finite values code +-0, infinities NaN).
    rows, cols = 256, 2048
    r = np.random.default_rng(19)
    amax = (10.0 ** r.uniform(-10, 30, rows)).astype(np.float32)
    scale = amax / np.float32(448.0)
    e = r.integers(0x75, 0x88, (rows, cols)).astype(np.uint32)
    m = (r.integers(0, 16, (rows, cols)).astype(np.uint32) << 19)
    m = np.where(r.random((rows, cols)) < 0.25, 0x7FFFF8, m).astype(np.int64)
    m = (m + r.integers(-3, 4, (rows, cols))) & 0x7FFFFF
    qd = ((e << 23) | m.astype(np.uint32)).view(np.float32)
    qd = np.minimum(qd, np.float32(447.0)) * np.where(r.random((rows, cols)) < 0.5, 1, -1).astype(np.float32)
    w = (qd * scale[:, None]).astype(np.float32)
    w = np.clip(w, -amax[:, None], amax[:, None])
    w[:, 0] = amax
    w[:3, 1:4] = [np.inf, np.nan, -1.0]
    w[3:8, 1:4] = [-0.0, 0.0, -1e-45]  # signed zeros and a denormal keep their sign bit
    c_ref, s_ref = O.quantize_fp8_rows(w)
    codes, scales = ops.quantize_fp8(torch.from_numpy(w).to(cuda))
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(codes.cpu().numpy(), c_ref)


@pytest.mark.parametrize("r,c", [(16, 512), (4096, 4096 // 8), (3, 11), (5, 4096), (7, 11008), (6, 520),
                                 (2, 12288), (3, 12296), (4097, 64), (2, 16384), (2, 16392)])
def test_fp8_rows_bf16_bit_exact(cuda, r, c):
    x = synth.activations_bf16(42, 1, r, c)
    c_ref, s_ref = O.quantize_fp8_rows(x)
    codes, scales = ops.quantize_fp8(torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(cuda))
    assert np.array_equal(codes.cpu().numpy(), c_ref)
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    d = ops.dequantize_fp8(codes, scales).cpu().numpy()
    dec = torch.from_numpy(c_ref).view(torch.float8_e4m3fn).float().numpy() * s_ref[:, None]
    assert np.array_equal(d, dec)


def test_fp8_rows_bf16_special_values(cuda):
    """bf16 rows with NaN, Inf, signed zeros, subnormals, values at the saturation edges and
    an all-zero row (cols % 8 == 0).  Rows 0 and 2 hold a NaN or an infinity (the kernel's
    general path); rows 4..7 stay finite (its fast path) with signed zeros, bf16 subnormals and,
    under an absmax of 3e38 or 1.7e38, negative values whose quotient underflows to -0 (code
    0x80) next to positive ones that underflow to +0."""
    x = synth.activations_bf16(43, 1, 8, 1024).copy()
    f = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0, 1e-40, -1e-40, 448.0, -464.0, 3e38], np.float32)
    x[0, :f.size] = O.f32_to_bf16_bits(f)
    x[1, :] = O.f32_to_bf16_bits(np.zeros(1024, np.float32))
    x[2, 5] = O.f32_to_bf16_bits(np.array([np.inf], np.float32))[0]
    x[3, 7] = O.f32_to_bf16_bits(np.array([1e-38], np.float32))[0]
    tiny = np.array([-0.0, 0.0, -1e-40, 1e-40, -1e-30, 1e-30, -1e-38, -3e-39, -2.0, 5.0], np.float32)
    x[4, :tiny.size] = O.f32_to_bf16_bits(tiny)
    x[5, :tiny.size] = O.f32_to_bf16_bits(tiny)
    x[5, 100] = O.f32_to_bf16_bits(np.array([3e38], np.float32))[0]
    x[6, :] = O.f32_to_bf16_bits(np.resize(tiny, 1024))
    x[6, 1023] = O.f32_to_bf16_bits(np.array([-1.7e38], np.float32))[0]
    x[7, :] = O.f32_to_bf16_bits(np.resize(tiny[:4], 1024))
    c_ref, s_ref = O.quantize_fp8_rows(x)
    codes, scales = ops.quantize_fp8(torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(cuda))
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(codes.cpu().numpy(), c_ref)


@pytest.mark.parametrize("c", [1024, 4096, 16384])
def test_fp8_rows_bf16_finite_rows_beside_special_ones(cuda, c):
    """Finite rows (the kernel's fast path) next to rows holding an infinity or a NaN (rows 4
    and 9, its general path) and an all-zero last row, 11 rows in all: every row's bytes and
    scale equal the oracle's, whichever path its neighbours take."""
    x = synth.activations_bf16(44, 1, 11, c).copy()
    x[4, 3] = O.f32_to_bf16_bits(np.array([np.inf], np.float32))[0]
    x[9, c - 1] = O.f32_to_bf16_bits(np.array([np.nan], np.float32))[0]
    x[10, :] = O.f32_to_bf16_bits(np.zeros(c, np.float32))
    c_ref, s_ref = O.quantize_fp8_rows(x)
    codes, scales = ops.quantize_fp8(torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(cuda))
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(codes.cpu().numpy(), c_ref)


# ------------------------------------------------------------- BASELINE block shapes ----
@pytest.mark.parametrize("name,n,k", synth.LLAMA7B_BLOCK)
def test_block_int8_channel_and_int4g128_full_size(cuda, name, n, k):
    tid = [b[0] for b in synth.LLAMA7B_BLOCK].index(name)
    w = synth.weight(0, tid, n, k)
    wd = torch.from_numpy(w).to(cuda)
    q_ref, s_ref = O.quantize_int8_rows(w, 8, 1)
    q, s = ops.quantize_int8(wd, 8, "channel", "half_even")
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref)
    c_ref, sc_ref, z_ref = O.quantize_int4g(w, 128)
    p = ops.quantize_int4g(wd, 128)
    assert np.array_equal(_u32(p.codes), c_ref)
    assert np.array_equal(p.scales.cpu().numpy().view(np.uint16), sc_ref)
    assert np.array_equal(_u32(p.zeros), z_ref)


# --------------------------------------------------------------- batched quantize ----
def _batch_inputs(cuda):
    shapes = [(37, 512), (100, 1024), (5, 512), (0, 512), (64, 2048), (3, 11008), (300, 1024)]
    ws = [torch.from_numpy(_w(200 + i, n, k, specials=(n * k >= 200))).to(cuda) for i, (n, k) in enumerate(shapes)]
    # one matrix that is not 16-byte aligned (a view one row and 4 columns in): quantized alone
    base = torch.from_numpy(_w(250, 9, 516)).to(cuda)
    ws.append(base.view(-1)[4:4 + 8 * 512].view(8, 512))
    return ws


def test_int4g_batched_matches_single(cuda):
    ws = _batch_inputs(cuda)
    batched = ops.quantize_int4g_batched(ws, 128)
    for w, b in zip(ws, batched):
        s = ops.quantize_int4g(w, 128)
        assert torch.equal(s.codes, b.codes) and torch.equal(s.zeros, b.zeros)
        assert torch.equal(s.scales.view(torch.int16), b.scales.view(torch.int16))
        if w.numel():
            codes, scales, zeros = O.quantize_int4g(w.cpu().numpy(), 128)
            assert np.array_equal(b.codes.cpu().numpy().view(np.uint32), codes)


def test_int4g_awq_batched_matches_single_and_oracle(cuda):
    """The batched AWQ form (one launch per column count) equals castforge_hip_quantize_int4g_awq
    per matrix bit for bit, and the oracle's quantization of f32(W * s); misaligned members take
    the single-matrix path inside the same call."""
    ws = _batch_inputs(cuda)
    ss = [torch.from_numpy(synth.awq_channel_scales(31, i, w.shape[1])).to(cuda) for i, w in enumerate(ws)]
    batched = ops.quantize_int4g_batched(ws, 128, ss)
    for w, sc, b in zip(ws, ss, batched):
        one = ops.quantize_int4g(w, 128, sc)
        assert torch.equal(one.codes, b.codes) and torch.equal(one.zeros, b.zeros)
        assert torch.equal(one.scales.view(torch.int16), b.scales.view(torch.int16))
        if w.numel():
            c_ref, s_ref, z_ref = O.quantize_int4g_awq(w.cpu().numpy(), sc.cpu().numpy(), 128)
            assert np.array_equal(b.codes.cpu().numpy().view(np.uint32), c_ref)
            assert np.array_equal(b.scales.cpu().numpy().view(np.uint16), s_ref)
            assert np.array_equal(b.zeros.cpu().numpy().view(np.uint32), z_ref)
    with pytest.raises(ValueError, match="in_scale"):
        ops.quantize_int4g_batched(ws[:1], 128, [ss[0][:-4]])


@pytest.mark.parametrize("mode", ["half_away", "half_even"])
def test_int8_batched_matches_single(cuda, mode):
    ws = _batch_inputs(cuda)
    batched = ops.quantize_int8_batched(ws, 8, mode)
    for w, (q, s) in zip(ws, batched):
        q1, s1 = ops.quantize_int8(w, 8, "channel", mode)
        assert torch.equal(q, q1)
        assert torch.equal(s.view(torch.int32), s1.view(torch.int32))
        if w.numel():
            q_ref, s_ref = O.quantize_int8_rows(w.cpu().numpy(), 8, 0 if mode == "half_away" else 1)
            assert np.array_equal(q.cpu().numpy(), q_ref)


def test_int4g_batched_block_rows_over_grid_limit(cuda):
    """The 7 block projections: the K = 4096 group has 38400 rows (one launch); splitting at
    65535 rows is exercised by five 16384-row matrices of the same K."""
    ws = [torch.from_numpy(synth.weight(300, i, 16384, 256)).to(cuda) for i in range(5)]
    for w, b in zip(ws, ops.quantize_int4g_batched(ws, 128)):
        s = ops.quantize_int4g(w, 128)
        assert torch.equal(s.codes, b.codes) and torch.equal(s.zeros, b.zeros)
        assert torch.equal(s.scales.view(torch.int16), b.scales.view(torch.int16))


def test_batched_quantize_rejects_bad_input(cuda):
    w = torch.zeros((4, 12), device=cuda)
    with pytest.raises(Exception, match="multiple of 8"):
        ops.quantize_int4g_batched([w], 128)
    with pytest.raises(Exception, match="at most"):
        ops.quantize_int8_batched([torch.zeros((2, 8), device=cuda)] * 9)
