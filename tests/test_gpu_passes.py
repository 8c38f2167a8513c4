"""GPU tests of the reference's pass / evaluator interface on the HIP kernels, modelled on the
reference's own tests of this path:
  tests/ai_opt_tests.rs:656, 740-775   quantize(bits=8) fixture, quantize + fuse-gemm(kind=dequant)
                                       equals the unfused module within 1e-5
  tests/pipeline_tests.rs:140-147      `!quant.uniform<i8:f32,` and uniform_dequantize appear;
                                       safetensors round trip (350-372)
  tests/frontend_tests.rs:747-756      AWQ salient count on a 2x2 weight
  tests/frontend_tests.rs:811-817      quantize(scheme=fp8) tags fp8_e4m3
  tests/loop_ir_tests.rs:495-507       quantize(dtype=bf16) within 1e-5 (the converts are copies)
Values are checked against the CPU oracle bit for bit where the reference is exact."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ops, synth
from castforge_amd.evaluate import evaluate_module, generate_synthetic_inputs, verify_module_numerics
from castforge_amd.ir import Module, QuantPacked, QuantUniform, TensorType
from castforge_amd.passes import PassManager, default_registry

pytestmark = pytest.mark.gpu

GOLD = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _mlp_module(dev, w, m=2, packed=False, name="w"):
    """forward(%x: tensor<m x K>) = dot_general(%x, %w) with %w a dense_resource constant."""
    mod = Module("qmatmul")
    x = mod.add_argument(TensorType((m, w.shape[1] if packed else w.shape[0]), "f32"), "x")
    wv = mod.constant(name, _t(w, dev))
    mod.set_results(mod.dot_general(x, wv, packed_rhs=packed, name="out"))
    return mod


def test_quantize_bits8_reference_fixture(cuda):
    """ai_opt_tests.rs:656: w = [[0.5,-0.25],[0.75,0.5]] -> codes [85,-42,127,85], scale bits
    0x3bc18306, `!quant.uniform<i8:f32,0.005906:0>`; the evaluator dequantizes through the
    string scale."""
    g = GOLD["int8_per_tensor"]
    w = np.array(g["weights"], np.float32).reshape(2, 2)
    mod = _mlp_module(cuda, w)
    res = PassManager.from_pipeline_str(default_registry(), "quantize(bits=8)").run(mod)
    assert res[0].changed and res[0].ops_modified == 1 and res[0].ops_created == 1
    e = mod.tensor_store.get("w")
    assert e.backing.data.cpu().numpy().ravel().tolist() == g["codes"]
    assert np.float32(e.backing.scale).view(np.uint32) == g["scale_bits"]
    assert str(e.ty.dtype) == g["type_string"]
    printed = mod.print_mlir()
    assert "!quant.uniform<i8:f32," in printed and "stablehlo.uniform_dequantize" in printed
    # the constant's value as the evaluator sees it
    wid = [v for v in mod.values.values() if v.ssa_name == "w"][0].id
    from castforge_amd.evaluate import _Evaluator

    ev = _Evaluator(mod, "f32")
    ev.run(generate_synthetic_inputs(mod, cuda))
    np.testing.assert_allclose(ev.env[wid].cpu().numpy().ravel(), g["dequant_with_string_scale"], rtol=0, atol=5e-7)


def test_quantize_fuse_equals_unfused(cuda):
    """ai_opt_tests.rs:740-775: quantize(bits=8,min_elements=4) then fuse-gemm(kind=dequant)
    removes every uniform_dequantize and matches the quantize-only module within 1e-5, with
    the interpreter's f32 activations and with the bf16 activations of the fused kernels."""
    w = synth.weight(3, 1, 64, 48)
    base = _mlp_module(cuda, w, m=5)
    reg = default_registry()
    q_only = base.clone()
    PassManager.from_pipeline_str(reg, "quantize(bits=8,min_elements=4)").run(q_only)
    fused = base.clone()
    res = PassManager.from_pipeline_str(reg, "quantize(bits=8,min_elements=4),fuse-gemm(kind=dequant)").run(fused)
    assert res[0].changed and res[1].changed
    printed = fused.print_mlir()
    assert "castforge.fused_qmatmul" in printed and "stablehlo.uniform_dequantize" not in printed
    for act in ("f32", "bf16"):
        rep = verify_module_numerics(q_only, fused, 1e-5, cuda, act)
        assert rep.passed, (act, rep.max_abs_diff)
    # the f32 evaluator is bit-identical to the oracle's eval_matmul_2d on dequantized weights
    x = generate_synthetic_inputs(base, cuda)
    out = evaluate_module(fused, x, "f32")[0].cpu().numpy()
    e = q_only.tensor_store.get("w")
    q = e.backing.data.cpu().numpy().astype(np.float32)
    s = np.float32(float(e.ty.dtype.scale))  # the evaluator's string scale
    ref = O.matmul_2d(x[0].cpu().numpy(), (q * s).astype(np.float32), False)
    assert np.array_equal(out, ref)


def test_bits4_group128_keeps_reference_scheme_inference(cuda):
    """families.rs:93-116: `group` is not `group_size`, so quantize(bits=4,group=128) is the
    per-tensor i4 scheme with a `!quant.uniform<i4:f32,...>` type."""
    w = synth.weight(4, 1, 16, 256)
    mod = _mlp_module(cuda, w.T.copy())
    PassManager.from_pipeline_str(default_registry(), "quantize(bits=4,group=128)").run(mod)
    e = mod.tensor_store.get("w")
    assert isinstance(e.ty.dtype, QuantUniform) and e.ty.dtype.storage == "i4"
    q_ref, s_ref = O.quantize_symmetric(w.T.copy(), 4, 0)
    assert np.array_equal(e.backing.data.cpu().numpy().ravel(), q_ref.ravel())
    assert np.float32(e.backing.scale) == s_ref


def test_awq_salient_reference_case_and_values(cuda):
    """frontend_tests.rs:747-756: scheme=awq,bits=4,group_size=2,salient_ratio=0.25 on a 2x2
    weight tags awq_groupwise with 1 salient channel; values bit-exact with the oracle."""
    w = np.array([[0.5, -0.25], [0.75, 0.5]], np.float32)
    mod = _mlp_module(cuda, w)
    PassManager.from_pipeline_str(default_registry(), "quantize(scheme=awq,bits=4,group_size=2,salient_ratio=0.25)").run(mod)
    cop = [o for o in mod.ops.values() if o.is_op("stablehlo", "constant")][0]
    assert cop.attributes["castforge.quant_scheme"] == "awq_groupwise"
    assert cop.attributes["castforge.awq_salient_channels"] == GOLD["awq_salient_count"]["count"]
    deq, _, cnt, _ = O.quantize_groupwise(w, 4, 2, True, 0.25, 0)
    got = mod.tensor_store.get("w").backing.data.cpu().numpy().ravel()
    assert cnt == 1 and np.array_equal(got.view(np.uint32), deq.view(np.uint32))
    # running again leaves the tagged constant alone
    r = PassManager.from_pipeline_str(default_registry(), "quantize(scheme=awq,bits=4,group_size=2,salient_ratio=0.25)").run(mod)
    assert not r[0].changed


@pytest.mark.parametrize("shape,bits,gs,ratio,awq", [((4096, 4096), 4, 32, 0.01, True),
                                                     ((333, 129), 8, 100, 0.3, True),
                                                     ((64, 64), 4, 7, 0.001, False),
                                                     ((1, 5), 4, 2, 0.5, True)])
def test_groupwise_kernel_bit_exact(cuda, shape, bits, gs, ratio, awq):
    print(f"[groupwise] shape={shape} bits={bits} gs={gs}", flush=True)
    w = synth.weight(5, 2, *shape)
    deq, scales, cnt = ops.quantize_groupwise(_t(w, cuda), bits, gs, awq, ratio)
    d_ref, s_ref, c_ref, _ = O.quantize_groupwise(w, bits, gs, awq, ratio, 0)
    assert cnt == c_ref
    assert np.array_equal(deq.cpu().numpy().ravel().view(np.uint32), d_ref.view(np.uint32))
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_groupwise_special_values(cuda):
    """NaN / inf / ties in the salient ranking and the group max (total_cmp order, NaN-ignoring
    max, NaN-propagating clamp) match the oracle bit for bit (NaN payloads compared as NaN)."""
    rng = np.random.default_rng(11)
    w = rng.standard_normal(4096).astype(np.float32) * 0.05
    w[[3, 700, 701]] = np.nan
    w[[5, 9]] = np.inf
    w[[10]] = -np.inf
    w[100:140] = 0.25  # many equal values at the threshold
    w[2000:2032] = 0.0  # an all-zero group
    for ratio in (0.001, 0.01, 0.2):
        deq, _, cnt = ops.quantize_groupwise(_t(w, cuda), 4, 32, True, ratio)
        d_ref, _, c_ref, _ = O.quantize_groupwise(w, 4, 32, True, ratio, 0)
        got = deq.cpu().numpy()
        assert cnt == c_ref
        nan = np.isnan(d_ref)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), d_ref[~nan].view(np.uint32))


def test_fp8_pass_reference_tag_and_values(cuda):
    """frontend_tests.rs:811-817 (the attribute) and the values of schemes.rs:681-713 against
    the oracle (which calls glibc log2f / powf), e4m3 and e5m2, MX and plain scales."""
    w = synth.fp8_inputs(6, 1, 96, 200) * np.float32(0.02)
    mod = _mlp_module(cuda, w)
    PassManager.from_pipeline_str(default_registry(), "quantize(scheme=fp8)").run(mod)
    cop = [o for o in mod.ops.values() if o.is_op("stablehlo", "constant")][0]
    assert cop.attributes["castforge.fp8_format"] == "fp8_e4m3"
    dot = [o for o in mod.ops.values() if o.is_op("stablehlo", "dot_general")][0]
    assert dot.attributes["castforge.fp8_format"] == "fp8_e4m3" and dot.attributes["castforge.mxfp8"] is True
    got = mod.tensor_store.get("w").backing.data.cpu().numpy().ravel()
    assert np.array_equal(got.view(np.uint32), O.quantize_fp8_grid(w, False, True, 32).view(np.uint32))
    for e5m2 in (False, True):
        for mx in (False, True):
            for bs in (3, 32, 100):
                d = ops.quantize_fp8_grid(_t(w, cuda), "e5m2" if e5m2 else "e4m3", mx, bs).cpu().numpy().ravel()
                assert np.array_equal(d.view(np.uint32), O.quantize_fp8_grid(w, e5m2, mx, bs).view(np.uint32))


def test_fp8_mx_scale_near_powers_of_two(cuda):
    """Blocks whose amax / 448 lands just above a power of two: the reference's log2f rounds to
    the integer there and keeps the smaller MX scale; the kernel's closed form agrees."""
    cases = []
    for e in range(-20, 20):
        for mbits in (0, 1, 2, 3, 5, 9, 17, 40, 1000):
            raw = np.array([(127 + e) << 23 | mbits], np.uint32).view(np.float32)[0]
            amax = np.float32(raw * np.float32(448.0))
            for cand in (np.nextafter(amax, np.float32(0)), amax, np.nextafter(amax, np.float32(np.inf))):
                if np.float32(cand) / np.float32(448.0) == raw:
                    cases.append(np.float32(cand))
                    break
    blocks = np.zeros((len(cases), 32), np.float32)
    rng = np.random.default_rng(7)
    for i, a in enumerate(cases):
        blocks[i] = rng.uniform(-1, 1, 32).astype(np.float32) * a
        blocks[i, i % 32] = a
    got = ops.quantize_fp8_grid(_t(blocks, cuda), "e4m3", True, 32).cpu().numpy().ravel()
    ref = O.quantize_fp8_grid(blocks, False, True, 32)
    assert len(cases) > 300
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_lower_mixed_precision_bf16_is_numerically_a_copy(cuda):
    """loop_ir_tests.rs:495-507: quantize(dtype=bf16) inserts the amp converts and keeps the
    interpreter's values within 1e-5."""
    w = synth.weight(8, 1, 32, 24)
    before = _mlp_module(cuda, w, m=3)
    after = before.clone()
    r = PassManager.from_pipeline_str(default_registry(), "quantize(dtype=bf16)").run(after)
    assert r[0].changed and r[0].ops_created == 4
    dot = [o for o in after.ops.values() if o.is_op("stablehlo", "dot_general")][0]
    assert dot.attributes["compute_precision"] == "bf16"
    assert sum(o.is_op("stablehlo", "convert") for o in after.ops.values()) == 4
    assert verify_module_numerics(before, after, 1e-5, cuda).passed


def test_pack_weights_transposes_on_gpu(cuda):
    w = synth.weight(9, 1, 40, 72)  # [K, N]
    mod = _mlp_module(cuda, w, m=3)
    before = mod.clone()
    r = PassManager.from_pipeline_str(default_registry(), "pack-weights").run(mod)
    assert r[0].changed
    dot = [o for o in mod.ops.values() if o.is_op("stablehlo", "dot_general")][0]
    assert dot.attributes["packed_rhs"] is True and dot.attributes["rhs_contracting_dimensions"] == [1]
    e = mod.tensor_store.get("w")
    assert e.ty.shape == (72, 40) and np.array_equal(e.backing.data.cpu().numpy(), w.T)
    rep = verify_module_numerics(before, mod, 0.0, cuda)
    assert rep.passed, rep.max_abs_diff  # same products, same k order


@pytest.mark.parametrize("scheme,opts", [("int4_asym", "group=128"), ("nf4", "block_size=64"),
                                         ("int8_channel", ""), ("fp8_row", "")])
def test_packed_schemes_fuse_and_match_oracle(cuda, scheme, opts):
    """pack-weights, then a packed scheme, then fuse-gemm: the fused module runs the HIP
    GEMV / GEMM (bf16 activations) and matches the oracle on the same codes."""
    k, n, m = 512, 96, 3
    w = synth.weight(10, 1, k, n)  # [K, N] as a frontend would hand it over
    mod = _mlp_module(cuda, w, m=m)
    spec = f"pack-weights,quantize(scheme={scheme}{',' + opts if opts else ''}),fuse-gemm(kind=dequant)"
    res = PassManager.from_pipeline_str(default_registry(), spec).run(mod)
    assert all(r.changed for r in res)
    e = mod.tensor_store.get("w")
    assert isinstance(e.ty.dtype, QuantPacked) and e.ty.dtype.format == scheme
    x = generate_synthetic_inputs(mod, cuda)
    y = evaluate_module(mod, x, "bf16")[0].cpu().numpy()
    xb = synth.f32_to_bf16_bits(x[0].cpu().numpy())
    b = e.backing
    wt = np.ascontiguousarray(w.T)
    if scheme == "int4_asym":
        c, s, z = O.quantize_int4g(wt, 128)
        assert np.array_equal(b.codes.cpu().numpy().view(np.uint32), c)
        ref = O.gemm_w4a16(xb, c, s, z, n, k, 128)
    elif scheme == "nf4":
        c, a = O.quantize_nf4(wt, 64)
        assert np.array_equal(b.codes.cpu().numpy().view(np.uint32), c)
        ref = O.gemm_nf4(xb, c, a, n, k, 64)
    elif scheme == "int8_channel":
        q, s = O.quantize_int8_rows(wt, 8, 1)
        assert np.array_equal(b.codes.cpu().numpy(), q)
        ref = O.gemm_w8a16(xb, q, s)
    else:
        qw, sw = O.quantize_fp8_rows(wt)
        assert np.array_equal(b.codes.cpu().numpy(), qw)
        qa, sa = O.quantize_fp8_rows(xb)
        ref = O.gemm_fp8(qa, sa, qw, sw)
    err = np.abs(y - ref)
    assert np.all(err <= 1e-3 + 1e-2 * np.abs(ref)), err.max()


@pytest.mark.parametrize("epi", ["bias", "bias_relu", "bias_tanh", "bias_silu", "bias_gelu", "bias_scale"])
def test_fused_qmatmul_epilogues(cuda, epi):
    """eval.rs:1151-1176: a fused_matmul_epilogue composite over a quantized weight becomes a
    fused_qmatmul; its epilogue runs on the GPU and matches the oracle's restatement (tanh /
    exp are the device's: within a few ulp)."""
    k, n, m = 64, 40, 4
    w = synth.weight(12, 1, n, k)
    mod = Module("epi")
    x = mod.add_argument(TensorType((m, k), "f32"), "x")
    wv = mod.constant("w", _t(w, cuda))
    bias = mod.constant("b", _t(np.linspace(-1, 1, n).astype(np.float32), cuda))
    z = mod.constant("z", _t(np.linspace(0.5, -0.5, m * n).astype(np.float32), cuda))
    y = mod.add_op("stablehlo.composite", [x, wv, bias, z], [TensorType((m, n), "f32")],
                   {"name": "castforge.fused_matmul_epilogue", "epilogue": epi, "packed_rhs": True}).results[0]
    mod.set_results(y)
    PassManager.from_pipeline_str(default_registry(), "quantize(scheme=int8_channel),fuse-gemm(kind=dequant)").run(mod)
    comp = [o for o in mod.ops.values() if o.is_op("stablehlo", "composite")][0]
    assert comp.attributes["name"] == "castforge.fused_qmatmul"
    xs = generate_synthetic_inputs(mod, cuda)
    got = evaluate_module(mod, xs, "bf16")[0].cpu().numpy()
    q = mod.tensor_store.get("w").backing
    xb = synth.f32_to_bf16_bits(xs[0].cpu().numpy())
    mm = O.gemm_w8a16(xb, q.codes.cpu().numpy(), q.scales.cpu().numpy()).ravel()
    mode = {"bias": 1, "bias_relu": 2, "bias_tanh": 3, "bias_silu": 4, "bias_gelu": 5, "bias_scale": 6}[epi]
    ref = mm.copy()
    O.lib().orc_epilogue(O._p(ref), ref.size, O._p(np.linspace(-1, 1, n).astype(np.float32)), n,
                         O._p(np.linspace(0.5, -0.5, m * n).astype(np.float32)), m * n, mode)
    np.testing.assert_allclose(got.ravel(), ref, rtol=1e-5, atol=1e-5)


def test_safetensors_round_trip_quantized_and_packed(cuda):
    """pipeline_tests.rs:350-372: quantized weights survive a safetensors round trip (I8 with
    scale / zero_point header keys; packed formats as component tensors)."""
    from castforge_amd.tensor_store import TensorStore

    w = synth.weight(13, 1, 32, 256)
    m1 = _mlp_module(cuda, w.T.copy(), name="a")
    PassManager.from_pipeline_str(default_registry(), "quantize(bits=8)").run(m1)
    m2 = _mlp_module(cuda, w, packed=True, name="b")
    PassManager.from_pipeline_str(default_registry(), "quantize(scheme=int4_asym)").run(m2)
    st = TensorStore()
    st.insert(m1.tensor_store.get("a"))
    st.insert(m2.tensor_store.get("b"))
    raw = st.to_safetensors_bytes()
    back = TensorStore()
    assert back.load_safetensors_bytes(raw, cuda) == 2
    a0, a1 = st.get("a"), back.get("a")
    assert a1.ty == a0.ty and a1.backing.scale == np.float32(a0.backing.scale)
    assert torch.equal(a1.backing.data, a0.backing.data)
    b0, b1 = st.get("b"), back.get("b")
    assert b1.ty == b0.ty
    for part in ("codes", "scales", "zeros"):
        assert torch.equal(getattr(b1.backing, part), getattr(b0.backing, part))


def test_quantize_channel_granularity_option(cuda):
    """quantize(bits=8,granularity=channel): this build's per-output-channel scheme (BASELINE
    config 1), round half-even by default."""
    w = synth.weight(14, 1, 48, 128)
    mod = _mlp_module(cuda, w, packed=True)
    PassManager.from_pipeline_str(default_registry(), "quantize(bits=8,granularity=channel)").run(mod)
    b = mod.tensor_store.get("w").backing
    q, s = O.quantize_int8_rows(w, 8, 1)
    assert np.array_equal(b.codes.cpu().numpy(), q)
    assert np.array_equal(b.scales.cpu().numpy().view(np.uint32), s.view(np.uint32))


# ------------------------------------------------------------ static W8A8 (calibrate) ----
@pytest.mark.parametrize("bits", [8, 4])
def test_static_quantize_kernel_matches_oracle(cuda, bits):
    r = np.random.default_rng(bits)
    for sc in (np.float32(1.25 / 127), np.float32(0.5), np.float32(3.0e-6), np.float32(7.0)):
        x = (r.standard_normal(5000) * float(sc) * r.choice([1, 10, 200], 5000)).astype(np.float32)
        x[:12] = [np.nan, np.inf, -np.inf, 0.0, -0.0, 0.5 * sc, -0.5 * sc, 1.5 * sc, -2.5 * sc,
                  127.5 * sc, -127.5 * sc, 1e30]
        y = ops.static_quantize(_t(x, cuda), float(sc), bits).cpu().numpy()
        ref = O.static_quantize(x, sc, bits)
        assert np.array_equal(np.isnan(y), np.isnan(ref))
        ok = ~np.isnan(ref)
        assert np.array_equal(y[ok].view(np.uint32), ref[ok].view(np.uint32))


def test_absmax_kernel(cuda):
    r = np.random.default_rng(3)
    for n in (0, 1, 7, 4096, 100003):
        x = r.standard_normal(n).astype(np.float32)
        if n > 10:
            x[5] = np.nan
            x[9] = -37.5
        got = ops.absmax(_t(x, cuda))
        want = float(np.nanmax(np.abs(x))) if n else 0.0
        assert got == want
    x = np.array([1.0, -np.inf, np.nan], np.float32)
    assert ops.absmax(_t(x, cuda)) == np.inf
    # an unaligned start (scalar path of the reduction)
    x = _t(r.standard_normal(1001).astype(np.float32), cuda)
    assert ops.absmax(x[1:]) == float(x[1:].abs().max().item())


def test_calibrate_w8a8_reference_case(cuda):
    """codegen_tests.rs:252-285 (the quantize part): quantize(scheme=w8a8,bits=8,samples=4) on two
    matmuls of one activation inserts castforge.static_quantize and the module stays within 2e-2
    of the original.  Here the two matmul results are the outputs (the reference adds them; this
    evaluator covers the quantized-weight path's ops only)."""
    mod = Module("parallel_branches")
    x = mod.add_argument(TensorType((2, 4), "f32"), "x")
    w0 = mod.add_argument(TensorType((4, 4), "f32"), "w0")
    w1 = mod.add_argument(TensorType((4, 4), "f32"), "w1")
    mod.set_results(mod.dot_general(x, w0, name="b0"), mod.dot_general(x, w1, name="b1"))
    before = mod.clone()
    res = PassManager.from_pipeline_str(default_registry(), "quantize(scheme=w8a8,bits=8,samples=4)").run(mod)
    assert res[0].changed
    assert "castforge.static_quantize" in mod.print_mlir()
    rep = verify_module_numerics(before, mod, 2e-2, cuda)
    assert rep.passed, rep.max_abs_diff
    assert rep.max_abs_diff > 0  # the activations really were quantized


def test_calibrate_constant_weight_range(cuda):
    """A constant rhs's bound is its max |w| (at least 1e-5), read on the device."""
    w = synth.weight(77, 1, 64, 32, 0.5)
    w[3, 4] = -2.75
    mod = _mlp_module(cuda, w)
    before = mod.clone()
    PassManager.from_pipeline_str(default_registry(), "calibrate-quantize").run(mod)
    d = [mod.ops[o] for o in mod.block_ops() if mod.ops[o].is_op("stablehlo", "dot_general")][0]
    assert d.attributes["rhs_scale"] == 2.75 / 127.0 and d.attributes["lhs_scale"] == 1.25 / 127.0
    assert verify_module_numerics(before, mod, 0.2, cuda).passed
