"""GPU parity of the GGUF payload kernels (decode, encode, planes) and of the Q4_0 / Q8_0
dequant-GEMV against the oracle restatement of gguf.rs:486-550 / 283-296.

Decode, encode, repack and unpack are byte work plus exact products: bit-exact (NaN payloads
aside: both sides NaN).  The GEMV is checked as the reference evaluates it (decode to f32, then
the f32 matmul loop of eval.rs:1465-1507) within |y - ref| <= 1e-3 + 1e-2 |ref|, and at the full
LLaMA-7B block shapes against a torch fp32 matmul over the decoded weights.
"""
import struct

import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ffi, gguf, ops, synth
from castforge_amd.passes import PassManager, default_registry

pytestmark = pytest.mark.gpu

Q4_0, Q8_0, F32, F16, BF16 = 2, 8, 0, 1, 30
BB = {Q4_0: 18, Q8_0: 34}
RTOL, ATOL = 1e-2, 1e-3


def _same(got: np.ndarray, want: np.ndarray):
    """Bit-exact equality of f32 arrays; a NaN only has to meet a NaN."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert got.shape == want.shape
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"NaN positions differ at {np.argwhere(gn != wn)[:5].ravel()}"
    bad = (got.view(np.uint32) != want.view(np.uint32)) & ~gn
    assert not bad.any(), f"{bad.sum()} mismatches, first at {np.argwhere(bad)[0]}: {got[bad][:3]} vs {want[bad][:3]}"


def _blocks(ty, nblocks, seed, special=False):
    """Random blocks with finite f16 d of weight-like size (and, if special, the edge d values
    subnormal / zero / negative / max / Inf / NaN in the first blocks)."""
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, nblocks * BB[ty], dtype=np.uint8).reshape(nblocks, BB[ty])
    d = (rng.standard_normal(nblocks) * 0.01).astype(np.float16)
    if special:
        sp = np.array([0x0001, 0x03FF, 0x0000, 0x8000, 0xBC00, 0x7BFF, 0x7C00, 0x7E01, 0xFD00], np.uint16)
        sp = sp[:nblocks]
        d[:sp.size] = sp.view(np.float16)
    raw[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
    return raw.reshape(-1)


def _dev_u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.uint8)).to(dev)


def _x(seed, m, k, dev):
    xb = synth.activations_bf16(seed, 7, m, k)
    return xb, torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)


def _close(y, ref):
    y = y.float().cpu().numpy()
    err = np.abs(y - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}"


def _planes_expected(ty, raw, n, k):
    """The GGUF planes layout, written out with numpy reshapes (the C header's definition)."""
    G = k // 32
    blk = raw.reshape(n, G, BB[ty])
    d = blk[:, :, 0:2].copy().view(np.uint16).reshape(n, G)
    pay = blk[:, :, 2:]
    if ty == Q4_0:
        codes = pay.reshape(n, G // 4, 4, 4, 4).transpose(0, 1, 3, 2, 4).reshape(n, k // 2)
    else:
        codes = pay.reshape(n, G // 2, 2, 4, 8).transpose(0, 1, 3, 2, 4).reshape(n, k)
    gp = (G + 7) // 8 * 8
    sc = np.zeros((n, gp), np.uint16)
    sc[:, :G] = d
    return np.ascontiguousarray(codes), sc


# ---------------------------------------------------------------------------- payloads ----
@pytest.mark.parametrize("ty", [Q4_0, Q8_0])
@pytest.mark.parametrize("n", [1, 7, 32, 33, 1000, 3 * 4096 + 5])
def test_decode_blocks_match_oracle(cuda, ty, n):
    raw = _blocks(ty, (n + 31) // 32, 100 + n, special=True)
    got = ops.gguf_decode(ty, _dev_u8(raw, cuda), n)
    torch.cuda.synchronize()
    _same(got.cpu().numpy(), O.gguf_decode(ty, raw, n))


@pytest.mark.parametrize("ty", [F32, F16, BF16])
@pytest.mark.parametrize("n", [1, 9, 4096 + 3])
def test_decode_arrays_match_oracle(cuda, ty, n):
    rng = np.random.default_rng(200 + n)
    raw = rng.integers(0, 256, n * (4 if ty == F32 else 2), dtype=np.uint8)
    got = ops.gguf_decode(ty, _dev_u8(raw, cuda), n)
    torch.cuda.synchronize()
    _same(got.cpu().numpy(), O.gguf_decode(ty, raw, n))


def test_decode_into_unaligned_output(cuda):
    n = 1000
    raw = _blocks(Q4_0, (n + 31) // 32, 7)
    rd = _dev_u8(raw, cuda)
    buf = torch.zeros(n + 1, dtype=torch.float32, device=cuda)
    ffi.call("castforge_hip_gguf_decode", Q4_0, rd.data_ptr(), n, buf.data_ptr() + 4,
             torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    out = buf.cpu().numpy()
    assert out[0] == 0.0
    _same(out[1:], O.gguf_decode(Q4_0, raw, n))


@pytest.mark.parametrize("n", [0, 1, 31, 32, 40, 5000])
def test_encode_q8_0_matches_oracle(cuda, n):
    rng = np.random.default_rng(300 + n)
    codes = rng.integers(-128, 128, n).astype(np.int8)
    scale = float(np.float32(1.0 + 3 * 2.0 ** -12) if n % 2 else np.float32(0.0123))
    got = ops.gguf_encode(Q8_0, torch.from_numpy(codes).to(cuda), scale)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), O.gguf_encode_q8_0(codes, scale))


def test_encode_half_types_truncate_like_reference(cuda):
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 1e-8, -3e-5, 6.1e-5,
                                  np.inf, -np.inf, np.nan, 1.0 + 3 * 2.0 ** -12], np.float32)])
    vd = torch.from_numpy(v).to(cuda)
    f16 = ops.gguf_encode(F16, vd).cpu().numpy().view(np.uint16)
    bf = ops.gguf_encode(BF16, vd).cpu().numpy().view(np.uint16)
    f32 = ops.gguf_encode(F32, vd).cpu().numpy().view(np.float32)
    want16 = np.array([O.lib().orc_f32_to_f16_trunc(float(x)) for x in v], np.uint16)
    want_bf = np.array([O.lib().orc_f32_to_bf16_trunc(float(x)) for x in v], np.uint16)
    np.testing.assert_array_equal(f16, want16)
    np.testing.assert_array_equal(bf, want_bf)
    np.testing.assert_array_equal(f32.view(np.uint32), v.view(np.uint32))


# ------------------------------------------------------------------------------ planes ----
@pytest.mark.parametrize("ty,n,k", [(Q4_0, 3, 128), (Q4_0, 5, 384), (Q4_0, 16, 4096),
                                    (Q8_0, 3, 64), (Q8_0, 7, 192), (Q8_0, 16, 11008)])
def test_repack_layout_unpack_and_dequant(cuda, ty, n, k):
    raw = _blocks(ty, n * k // 32, 400 + k, special=True)
    p = ops.gguf_repack(ty, _dev_u8(raw, cuda), n, k)
    back = ops.gguf_unpack(p)
    deq = ops.dequantize_gguf(p)
    torch.cuda.synchronize()
    codes, sc = _planes_expected(ty, raw, n, k)
    np.testing.assert_array_equal(p.codes.cpu().numpy().view(np.uint8), codes)
    np.testing.assert_array_equal(p.scales.cpu().numpy().view(np.uint16), sc)
    np.testing.assert_array_equal(back.cpu().numpy(), raw)
    _same(deq.cpu().numpy().reshape(-1), O.gguf_decode(ty, raw, n * k))


@pytest.mark.parametrize("ty", [Q4_0, Q8_0])
def test_repack_unpack_identity_full_size(cuda, ty):
    n, k = 11008, 4096
    raw = torch.randint(0, 256, (n * k // 32 * BB[ty],), dtype=torch.uint8, device=cuda)
    p = ops.gguf_repack(ty, raw, n, k)
    assert torch.equal(ops.gguf_unpack(p), raw)


def test_planes_reject_bad_shapes(cuda):
    raw = _dev_u8(_blocks(Q4_0, 12, 1), cuda)
    with pytest.raises(ffi.CastForgeHipError, match="k % 128"):
        ops.gguf_repack(Q4_0, raw, 3, 96)
    with pytest.raises(ffi.CastForgeHipError, match="Q4_0 or"):
        ffi.call("castforge_hip_gguf_repack", F16, raw.data_ptr(), 1, 128, raw.data_ptr(), raw.data_ptr(), None)
    x = torch.zeros((1, 96), dtype=torch.bfloat16, device=cuda)
    y = torch.zeros((1, 3), dtype=torch.float32, device=cuda)
    with pytest.raises(ffi.CastForgeHipError, match="k % 64"):
        ffi.call("castforge_hip_gemv_gguf", Q8_0, x.data_ptr(), 1, 3, 96, raw.data_ptr(), raw.data_ptr(),
                 y.data_ptr(), ffi.DTYPE_F32, None)


# -------------------------------------------------------------------------------- GEMV ----
@pytest.mark.parametrize("ty", [Q4_0, Q8_0])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 9, 16, 17, 33, 64])
@pytest.mark.parametrize("n,k", [(48, 256), (100, 1024), (64, 11008), (4096, 4096)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_gemv_matches_oracle(cuda, ty, m, n, k, out):
    raw = _blocks(ty, n * k // 32, 500 + n + k)
    p = ops.gguf_repack(ty, _dev_u8(raw, cuda), n, k)
    xb, x = _x(501, m, k, cuda)
    y = ops.gemm_gguf(x, p, out)
    torch.cuda.synchronize()
    w = O.gguf_decode(ty, raw, n * k).reshape(n, k)
    ref = O.matmul_2d(O.bf16_bits_to_f32(xb.reshape(m, k)), w, packed_rhs=True)
    if out == torch.bfloat16:
        ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref))
    _close(y, ref)


@pytest.mark.parametrize("kernel", ["auto", "0", "1"])
@pytest.mark.parametrize("special", [False, True])
@pytest.mark.parametrize("m,n,k", [(64, 96, 1024), (300, 256, 4096), (17, 48, 256), (130, 1000, 2048), (129, 257, 640)])
def test_q4_0_prefill_and_int4g_form(cuda, monkeypatch, kernel, special, m, n, k):
    """Q4_0 at M > 16: the prefill MFMA kernel reading the planes matches the oracle's
    decode-then-matmul, and the INT4g form of the planes dequantizes to the same values bit
    for bit.  kernel: CASTFORGE_PREFILL_I4 ("1" forces the one-MFMA kernel, exact q - 8 with
    one f32 partial per 32-wide block scaled by its d; "0" the two-term kernel); special: d
    values that are subnormal, zero, -0, negative and the largest finite f16."""
    if kernel == "auto":
        monkeypatch.delenv("CASTFORGE_PREFILL_I4", raising=False)
    else:
        monkeypatch.setenv("CASTFORGE_PREFILL_I4", kernel)
    raw = _blocks(Q4_0, n * k // 32, 700 + m, special)
    p = ops.gguf_repack(Q4_0, _dev_u8(raw, cuda), n, k)
    i4 = ops.gguf_q4_0_to_int4g(p)
    _same(ops.dequantize_int4g(i4).cpu().numpy().reshape(-1), O.gguf_decode(Q4_0, raw, n * k))
    xb, x = _x(701, m, k, cuda)
    y = ops.gemm_gguf(x, p, torch.float32)
    torch.cuda.synchronize()
    w = O.gguf_decode(Q4_0, raw, n * k).reshape(n, k)
    _close(y, O.matmul_2d(O.bf16_bits_to_f32(xb.reshape(m, k)), w, packed_rhs=True))


@pytest.mark.parametrize("kernel", ["auto", "0", "1"])
@pytest.mark.parametrize("special", [False, True])
@pytest.mark.parametrize("m,n,k", [(64, 96, 1024), (300, 256, 4096), (17, 48, 256), (130, 1000, 2048), (129, 257, 640)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_q8_0_prefill_reads_planes(cuda, monkeypatch, kernel, special, m, n, k, out):
    """Q8_0 at M > 16: the prefill MFMA kernels read the planes directly and match the
    oracle's decode-then-matmul.  kernel: CASTFORGE_PREFILL_I4 ("1" forces the one-MFMA kernel,
    exact q with one f32 partial per 32-wide block scaled by its d, at K % 128 == 0; "0" the
    three-term kernel); special: subnormal, zero, -0, negative and largest finite d."""
    if kernel == "auto":
        monkeypatch.delenv("CASTFORGE_PREFILL_I4", raising=False)
    else:
        monkeypatch.setenv("CASTFORGE_PREFILL_I4", kernel)
    raw = _blocks(Q8_0, n * k // 32, 800 + m, special)
    p = ops.gguf_repack(Q8_0, _dev_u8(raw, cuda), n, k)
    xb, x = _x(801, m, k, cuda)
    y = ops.gemm_gguf(x, p, out)
    torch.cuda.synchronize()
    ref = O.matmul_2d(O.bf16_bits_to_f32(xb.reshape(m, k)), O.gguf_decode(Q8_0, raw, n * k).reshape(n, k), True)
    if out == torch.bfloat16:
        ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref))
    _close(y, ref)


@pytest.mark.parametrize("ty", [Q4_0, Q8_0])
def test_gemv_batched_block_matches_single_and_torch(cuda, ty):
    """The seven LLaMA-7B block projections in one launch: equal to one call per matrix, and
    within tolerance of a torch fp32 matmul over the decoded weights."""
    ps, xs, ys = [], [], []
    for tid, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK):
        raw = torch.randint(0, 256, (n * k // 32 * BB[ty],), dtype=torch.uint8, device=cuda)
        raw.view(-1, BB[ty])[:, 0:2] = (torch.randn(n * k // 32, device=cuda) * 0.003).half().view(torch.uint8).view(-1, 2)
        ps.append(ops.gguf_repack(ty, raw, n, k))
        xs.append(_x(600 + tid, 1, k, cuda)[1])
        ys.append(torch.empty((1, n), dtype=torch.float32, device=cuda))
    ops.gemv_gguf_batched(xs, ps, ys)
    for x, p, y in zip(xs, ps, ys):
        single = ops.gemm_gguf(x, p, torch.float32)
        assert torch.equal(single, y)
        ref = x.float() @ ops.dequantize_gguf(p).t()
        err = (y - ref).abs()
        assert bool((err <= ATOL + RTOL * ref.abs()).all()), f"max err {err.max().item():.3e}"


@pytest.mark.parametrize("ty", [Q4_0, Q8_0])
@pytest.mark.parametrize("m", [4, 16, 40, 64])
def test_gemv_batched_block_m_gt_1(cuda, ty, m):
    """The seven block projections at M > 1 in one launch equal one call per matrix and the
    oracle's decode-then-matmul (sampled rows of each matrix, to keep the CPU side short)."""
    ps, xs, ys, raws = [], [], [], []
    for tid, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK):
        raw = _blocks(ty, n * k // 32, 900 + 10 * tid + ty)
        raws.append(raw)
        ps.append(ops.gguf_repack(ty, _dev_u8(raw, cuda), n, k))
        xs.append(_x(900 + tid, m, k, cuda))
        ys.append(torch.empty((m, n), dtype=torch.float32, device=cuda))
    ops.gemv_gguf_batched([x for _, x in xs], ps, ys)
    rng = np.random.default_rng(ty + m)
    for (xb, x), p, y, raw in zip(xs, ps, ys, raws):
        if not (ty == Q4_0 and m > 32):  # single Q4_0 calls above M = 32 run the prefill kernel
            assert torch.equal(ops.gemm_gguf(x, p, torch.float32), y)
        rows = np.sort(rng.choice(p.n, 24, replace=False))
        sub = raw.reshape(p.n, -1)[rows].reshape(-1)  # whole rows of blocks (k % 32 == 0)
        w = O.gguf_decode(ty, sub, 24 * p.k).reshape(24, p.k)
        ref = O.matmul_2d(O.bf16_bits_to_f32(xb.reshape(m, p.k)), w, packed_rhs=True)
        _close(y[:, torch.from_numpy(rows).to(y.device)], ref)


@pytest.mark.parametrize("ty", [Q4_0, Q8_0])
def test_gemv_m1_beyond_split_lds_limit(cuda, ty):
    """K = 32768 needs more LDS per workgroup than the M = 1 split-K kernel takes, so M = 1
    runs the skinny kernel's one-row path; checked against the oracle."""
    n, k = 40, 32768
    raw = _blocks(ty, n * k // 32, 950 + ty)
    p = ops.gguf_repack(ty, _dev_u8(raw, cuda), n, k)
    xb, x = _x(951, 1, k, cuda)
    y = ops.gemm_gguf(x, p, torch.float32)
    torch.cuda.synchronize()
    ref = O.matmul_2d(O.bf16_bits_to_f32(xb.reshape(1, k)), O.gguf_decode(ty, raw, n * k).reshape(n, k), True)
    _close(y, ref)


def test_gemv_batched_rejects_mixed_types(cuda):
    raw = _dev_u8(_blocks(Q4_0, 16, 2), cuda)
    p4 = ops.gguf_repack(Q4_0, raw, 4, 128)
    p8 = ops.gguf_repack(Q8_0, _dev_u8(_blocks(Q8_0, 16, 3), cuda), 4, 128)
    x = torch.zeros((1, 128), dtype=torch.bfloat16, device=cuda)
    y = [torch.empty((1, 4), device=cuda) for _ in range(2)]
    with pytest.raises(ValueError, match="share the GGML type"):
        ops.gemv_gguf_batched([x, x], [p4, p8], y)


# --------------------------------------------------------------------------- container ----
def _gguf_file(seed):
    rng = np.random.default_rng(seed)
    f32 = rng.standard_normal((256, 128)).astype(np.float32)
    f16 = rng.standard_normal(128).astype(np.float16)
    bf = rng.integers(0, 1 << 16, (2, 64), dtype=np.uint16)
    q4 = _blocks(Q4_0, 128 * 256 // 32, seed + 1)
    q8 = _blocks(Q8_0, 256 * 64 // 32, seed + 2)
    odd = _blocks(Q4_0, 3, seed + 3)  # [1, 80]: not a planes shape, decoded
    tensors = [("blk.0.w", (256, 128), F32, f32.view(np.uint8).reshape(-1)),
               ("blk.0.norm", (128,), F16, f16.view(np.uint8)),
               ("blk.0.q4", (128, 256), Q4_0, q4),
               ("blk.0.q8", (256, 64), Q8_0, q8),
               ("blk.0.bf", (2, 64), BF16, bf.view(np.uint8).reshape(-1)),
               ("blk.0.odd", (1, 80), Q4_0, odd)]
    return tensors, gguf.write_gguf_tensors(tensors, name="t.model")


def test_import_decodes_like_oracle_and_builds_graph(cuda):
    tensors, raw = _gguf_file(11)
    mod = gguf.import_gguf_bytes(raw, cuda)
    assert mod.name == "t_model" and len(mod.tensor_store) == len(tensors)
    for name, shape, ty, payload in tensors:
        e = mod.tensor_store.get(name)
        n = int(np.prod(shape))
        assert tuple(e.ty.shape) == shape
        _same(e.backing.data.reshape(-1).cpu().numpy(), O.gguf_decode(ty, payload, n))
    printed = mod.print_mlir()
    assert "stablehlo.dot_general" in printed and "stablehlo.multiply" in printed


def test_import_keep_packed_and_export_roundtrip(cuda):
    tensors, raw = _gguf_file(12)
    mod = gguf.import_gguf_bytes(raw, cuda, keep_packed=True)
    q4 = mod.tensor_store.get("blk.0.q4").backing
    assert q4.format == "gguf_q4_0" and q4.shape == (128, 256)
    assert mod.tensor_store.get("blk.0.q8").backing.format == "gguf_q8_0"
    assert hasattr(mod.tensor_store.get("blk.0.odd").backing, "data")  # k = 80: decoded
    out = gguf.export_gguf_bytes(mod)
    _, infos, base = gguf.read_gguf_header(out)
    by_name = {t[0]: t for t in tensors}
    for name, shape, ty, off in infos:
        want = by_name[name]
        if name in ("blk.0.q4", "blk.0.q8", "blk.0.w"):
            assert ty == want[2]
            np.testing.assert_array_equal(np.frombuffer(out, np.uint8, want[3].size, base + off), want[3])
    # the packed weight feeds the GEMV through the evaluator's fused path
    p = ops.GgufPacked(Q4_0, q4.codes, q4.scales, 128, 256)
    xb, x = _x(13, 1, 256, cuda)
    ref = O.matmul_2d(O.bf16_bits_to_f32(xb.reshape(1, 256)),
                      O.gguf_decode(Q4_0, by_name["blk.0.q4"][3], 128 * 256).reshape(128, 256), True)
    _close(ops.gemm_gguf(x, p, torch.float32), ref)


def test_reference_quantized_gguf_roundtrip(cuda):
    """frontend_tests.rs:167-219: x[2,4] . w (0.5) + b (0.1); quantize-weights, export (Q8_0),
    import: two tensors come back, each the codes times the f16-truncated scale."""
    from castforge_amd.ir import Module, TensorType

    mod = Module("frontend")
    x = mod.add_argument(TensorType((2, 4), "f32"), "x")
    w = mod.constant("w", torch.full((4, 4), 0.5, device=cuda), inline=True)
    b = mod.constant("b", torch.full((2, 4), 0.1, device=cuda), inline=True)
    mm = mod.dot_general(x, w, name="mm")
    mod.set_results(mod.add_op("stablehlo.add", [mm, b], [TensorType((2, 4), "f32")], {}, ["y"]).results[0])
    PassManager.from_pipeline_str(default_registry(), "quantize-weights").run(mod)
    raw = gguf.export_gguf_bytes(mod)
    back = gguf.import_gguf_bytes(raw, cuda)
    assert len(back.tensor_store) == 2
    for name in ("w", "b"):
        q = mod.tensor_store.get(name).backing
        d = np.float32(O.lib().orc_f16_to_f32(O.lib().orc_f32_to_f16_trunc(q.scale)))
        want = q.data.cpu().numpy().astype(np.float32).reshape(-1) * d
        _same(back.tensor_store.get(name).backing.data.reshape(-1).cpu().numpy(), want)
    assert "stablehlo.dot_general" in back.print_mlir()
