"""CPU tests of the host-side mirror of the reference's pass interface: option parsing and
scheme inference (registry/families.rs:93-183), pipeline strings (registry/manager.rs:410-459),
option validation (manager.rs:512-540), the `!quant.uniform` type string (ir/mlir.rs:82-91,
ir/parser.rs:1336-1351; formats.rs:680-688) and the graph-only passes (lower-mixed-precision,
the dequant fusion rewrite).  No kernel runs here."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd.ir import (Module, QuantPacked, QuantUniform, TensorRef, TensorType, format_scale,
                              parse_dtype, parse_tensor_type)
from castforge_amd.passes import (FuseDequantMatmulPass, LowerMixedPrecisionPass, PackWeightsPass, PassManager,
                                  QuantizeFp8Pass, QuantizeGroupwisePass, QuantizePass, default_registry,
                                  parse_pass_spec_item, split_pipeline_spec)
from castforge_amd.tensor_store import QuantizedI8, TensorEntry


def _q(spec):
    return PassManager.from_pipeline_str(default_registry(), spec).passes[0]


@pytest.mark.parametrize("spec,scheme,bits", [
    ("quantize", "weight", 8),
    ("quantize(bits=8)", "weight", 8),
    ("quantize(bits=4,group=128)", "weight", 4),          # `group` does not select groupwise
    ("quantize(group_size=128)", "groupwise", 4),
    ("quantize(awq_salient=false)", "groupwise", 4),
    ("quantize(salient_ratio=0.02)", "awq", 4),
    ("quantize(format=e5m2)", "fp8", 8),
    ("quantize(mxfp8=false)", "fp8", 8),
    ("quantize(alpha=0.5)", "smoothquant", 8),
    ("quantize(samples=8)", "w8a8", 8),
    ("quantize(block_size=16)", "hadamard", 8),
    ("quantize(block_size=16,bits=8)", "weight", 8),
    ("quantize(mode=fp8)", "fp8", 8),
    ("quantize(dtype=bf16)", "bf16", 8),
    ("quantize(scheme=nf4)", "nf4", 4),
    ("quantize(scheme=int4_asym,group=64)", "int4_asym", 4),
    ("quantize(bits=300)", "weight", 8),                   # not a u8: default
])
def test_quantize_scheme_inference(spec, scheme, bits):
    p = _q(spec)
    assert isinstance(p, QuantizePass)
    assert p.scheme == scheme and p.bits == bits


def test_quantize_option_defaults_and_aliases():
    p = _q("quantize(scheme=groupwise,group=64,size=8,salient_ratio=abc)")
    assert p.group_size == 64 and p.block_size == 8 and p.salient_ratio == pytest.approx(0.01)
    p = _q("quantize(scheme=fp8,dtype=e5m2)")
    assert p.scheme == "fp8" and p.format == "e5m2"
    p = _q("quantize(scheme=int4_asym)")
    assert not p.group_given  # int4_asym then uses group 128
    p = _q('quantize(scheme="awq", bits=\'4\')')
    assert p.scheme == "awq" and p.bits == 4


def test_pipeline_string_parsing():
    assert split_pipeline_spec("a(x=1,y=2),b|c") == ["a(x=1,y=2)", "b", "c"]
    assert parse_pass_spec_item(" quantize ( bits = 8 , min_elements=4 ) ") == (
        "quantize", {"bits": "8", "min_elements": "4"})
    with pytest.raises(ValueError, match="Unclosed"):
        parse_pass_spec_item("quantize(bits=8")
    with pytest.raises(ValueError, match="trailing"):
        parse_pass_spec_item("quantize(bits=8)x")
    with pytest.raises(ValueError, match="key=value"):
        parse_pass_spec_item("quantize(bits)")


def test_registry_validation_errors():
    reg = default_registry()
    with pytest.raises(ValueError, match="Unknown pass `nope`"):
        reg.create_pass("nope", {})
    with pytest.raises(ValueError, match="does not accept options"):
        reg.create_pass("pack-weights", {"bits": "8"})
    with pytest.raises(ValueError, match="unrecognized option `bogus`"):
        reg.create_pass("quantize", {"bogus": "1"})
    with pytest.raises(ValueError, match="kind"):
        reg.create_pass("fuse-gemm", {"kind": "horizontal"})
    with pytest.raises(ValueError, match="round"):
        reg.create_pass("quantize", {"round": "up"})
    assert isinstance(reg.create_pass("quantize-groupwise", {"group": "16"}), QuantizeGroupwisePass)
    assert reg.create_pass("quantize-groupwise", {"group": "16"}).group_size == 16
    assert isinstance(reg.create_pass("quantize-fp8", {}), QuantizeFp8Pass)
    assert isinstance(reg.create_pass("pack-weights", {}), PackWeightsPass)
    assert reg.create_pass("lower-mixed-precision", {"dtype": "BF16"}).low == "bf16"


def test_quant_uniform_type_string_round_trip():
    dt = QuantUniform("i8", "f32", "0.005906", 0)
    assert str(dt) == "!quant.uniform<i8:f32,0.005906:0>"
    assert parse_dtype(str(dt)) == dt
    ty = TensorType((2, 2), dt)
    assert str(ty) == "tensor<2x2x!quant.uniform<i8:f32,0.005906:0>>"
    assert parse_tensor_type(str(ty)) == ty
    p = QuantPacked("int4_asym", "f32", 128)
    assert parse_dtype(str(p)) == p
    assert parse_dtype("mystery") == "f32"  # parser.rs: unknown -> f32
    assert parse_tensor_type("tensor<f32>") == TensorType((), "f32")


@pytest.mark.parametrize("scale", [0.0059055118, 1.0, 2.5, 1e-7, 123.4567891, 0.0000005, 7.0 / 3.0])
def test_scale_string_matches_oracle(scale):
    s = float(np.float32(scale))
    assert format_scale(s) == O.scale_string(s)


def test_scale_string_known_answer():
    assert format_scale(float(np.float32(0.75) / np.float32(127))) == "0.005906"
    assert format_scale(1.0) == "1.0"
    assert format_scale(2.5) == "2.5"


def _cpu_module():
    m = Module("t")
    x = m.add_argument(TensorType((2, 3), "f32"), "x")
    w = m.constant("w", torch.zeros(3, 4))
    y = m.dot_general(x, w, name="y")
    m.set_results(y)
    return m, x, w, y


def test_module_verify_print_clone():
    m, x, w, y = _cpu_module()
    m.verify()
    txt = m.print_mlir()
    assert "stablehlo.dot_general %x, %w" in txt and "dense_resource<w>" in txt
    c = m.clone()
    c.tensor_store.insert(TensorEntry("w", TensorType((3, 4), "f32"), None))
    assert m.tensor_store.get("w").backing is not None  # copy-on-write store
    m.ops[m.order[-1]].operands[0] = 999
    with pytest.raises(ValueError, match="undefined"):
        m.verify()


def test_lower_mixed_precision_graph_rewrite():
    m, x, w, y = _cpu_module()
    r = LowerMixedPrecisionPass("bf16").run(m)
    assert r.changed and r.ops_created == 4 and r.ops_modified == 1
    dot = m.ops[m.values[y].op]
    assert dot.attributes["compute_precision"] == "bf16"
    convs = [m.ops[o] for o in m.order if m.ops[o].is_op("stablehlo", "convert")]
    assert len(convs) == 4 and all(c.attributes["amp_cast"] for c in convs)
    assert [str(m.values[c.results[0]].ty.dtype) for c in convs] == ["bf16", "f32", "bf16", "f32"]
    m.verify()
    assert not LowerMixedPrecisionPass("bf16").run(m).changed  # already tagged


def test_fuse_dequant_rewrite_and_dce():
    """epilogue.rs:10-45 on a hand-built quantized constant (no kernel): the dot_general
    becomes the fused_qmatmul composite with the type's scale, and the dequantize is removed."""
    m = Module("f")
    x = m.add_argument(TensorType((1, 4), "f32"), "x")
    qty = TensorType((3, 4), QuantUniform("i8", "f32", "0.25", 0))
    m.tensor_store.insert(TensorEntry("w", qty, QuantizedI8(torch.zeros(3, 4, dtype=torch.int8), 0.25, 0)))
    c = m.add_op("stablehlo.constant", [], [qty], {"value": TensorRef("w")}, ["w"])
    d = m.add_op("stablehlo.uniform_dequantize", [c.results[0]], [TensorType((3, 4), "f32")], {}, ["w_deq"])
    y = m.dot_general(x, d.results[0], packed_rhs=True, name="y")
    m.set_results(y)
    r = FuseDequantMatmulPass().run(m)
    assert r.changed and r.ops_created == 1 and r.ops_removed == 1
    op = m.ops[m.values[y].op]
    assert op.name == "stablehlo.composite" and op.attributes["name"] == "castforge.fused_qmatmul"
    assert op.attributes["scale"] == 0.25 and op.attributes["zero_point"] == 0 and op.attributes["packed_rhs"]
    assert op.operands == [x, c.results[0]]
    assert not any(o.is_op("stablehlo", "uniform_dequantize") for o in m.ops.values())
    m.verify()


# ------------------------------------------------------------ safetensors dtypes (CPU) ----
def _st_bytes(entries):
    """A safetensors file from (name, dtype, shape, raw bytes, extra header keys)."""
    import json as _json
    import struct as _struct

    header, blobs, off = {}, [], 0
    for name, dt, shape, data, extra in entries:
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(data)], **extra}
        blobs.append(data)
        off += len(data)
    hb = _json.dumps(header).encode()
    return _struct.pack("<Q", len(hb)) + hb + b"".join(blobs)


def test_safetensors_loader_dtypes_follow_the_reference():
    """tensor_store.rs:656-752: F16 / BF16 load as f32 values that keep their dtype (exact
    decode, f16 subnormals and NaN payloads included), I8 with an integral scale gets the
    trimmed string "1" (no ".0"), and an unknown dtype is kept as raw U8 bytes."""
    import numpy as np

    from castforge_amd.tensor_store import F32Data, InMemory, QuantizedI8, TensorStore

    f16 = np.array([1.0, -0.5, 6.1e-5, 3e-7, 65504.0, -np.inf], np.float16).view(np.uint16)
    f16 = np.concatenate([f16, np.array([0x7C01, 0xFE00], np.uint16)])  # signalling / quiet NaN
    bf = np.array([0x3F80, 0xC2F7, 0x0001, 0x7F80], np.uint16)
    raw = _st_bytes([("h", "F16", (8,), f16.tobytes(), {}),
                     ("b", "BF16", (2, 2), bf.tobytes(), {}),
                     ("q", "I8", (3,), np.array([1, -2, 127], np.int8).tobytes(), {"scale": 1.0, "zero_point": 0}),
                     ("q2", "I8", (1,), b"\x05", {"scale": 0.0059055118, "zero_point": 0}),
                     ("i", "I64", (1,), np.array([7], np.int64).tobytes(), {})])
    st = TensorStore()
    assert st.load_safetensors_bytes(raw, "cpu") == 5
    h = st.get("h")
    assert h.ty.dtype == "f16" and isinstance(h.backing, F32Data)
    got = h.backing.data.numpy().view(np.uint32)
    want = np.array([0x3F800000, 0xBF000000, f2u(float(np.float16(6.1e-5))), f2u(float(np.float16(3e-7))),
                     0x477FE000, 0xFF800000, 0x7F802000, 0xFFC00000], np.uint32)
    assert got.tolist() == want.tolist()
    b = st.get("b")
    assert b.ty.dtype == "bf16" and tuple(b.ty.shape) == (2, 2)
    assert b.backing.data.numpy().view(np.uint32).tolist() == [0x3F800000, 0xC2F70000, 0x00010000, 0x7F800000]
    q = st.get("q")
    assert isinstance(q.backing, QuantizedI8) and str(q.ty.dtype) == "!quant.uniform<i8:f32,1:0>"
    assert str(st.get("q2").ty.dtype) == "!quant.uniform<i8:f32,0.005906:0>"
    i = st.get("i")
    assert isinstance(i.backing, InMemory) and i.ty.dtype == "u8"
    assert i.backing.data.numpy().tobytes() == np.array([7], np.int64).tobytes()
    # writing back: F16 / BF16 through the truncating converters, unknown bytes as U8
    back = TensorStore()
    assert back.load_safetensors_bytes(st.to_safetensors_bytes(), "cpu") == 5
    # the writer's converter has no subnormals: the two f16 subnormals come back as +0
    assert back.get("h").backing.data.numpy().view(np.uint32)[:6].tolist() == [0x3F800000, 0xBF000000, 0, 0,
                                                                               0x477FE000, 0xFF800000]
    assert back.get("b").backing.data.numpy().view(np.uint32).tolist() == [0x3F800000, 0xC2F70000, 0x00010000,
                                                                            0x7F800000]
    assert back.get("i").backing.data.numpy().tobytes() == np.array([7], np.int64).tobytes()
    with pytest.raises(ValueError, match="not a multiple of 2"):
        TensorStore().load_safetensors_bytes(_st_bytes([("x", "BF16", (1,), b"\x00\x00\x00", {})]), "cpu")


def test_f16_truncating_writer_matches_reference_rules():
    """f32_to_f16_bits (tensor_store.rs:84-102): truncation, not rounding; exponent overflow
    to inf; no subnormals (flush to signed zero); the KAT translator.rs:295-296."""
    import numpy as np

    from castforge_amd.tensor_store import f32_to_f16_bits_trunc

    v = np.array([-1e-10, 1.0 + 3 * 2 ** -12, 65520.0, 65536.0, 1e-5, -0.0, np.nan, -np.inf, 2.0 ** -14],
                 np.float32)
    # 65520 truncates to 65504 (0x7bff) where round-to-nearest-even would give inf
    assert f32_to_f16_bits_trunc(v).tolist() == [0x8000, 0x3C00, 0x7BFF, 0x7C00, 0x0000, 0x8000, 0x7E00, 0xFC00,
                                                 0x0400]


def f2u(x: float) -> int:
    import struct as _struct

    return _struct.unpack("<I", _struct.pack("<f", x))[0]


@pytest.mark.parametrize("scheme", ["fp4", "nvfp4", "qat"])
def test_quantize_unsupported_scheme_leaves_module_unchanged(scheme):
    """quantize(scheme=fp4|..., hadamard=true) raises before the rotation step runs, so the
    caller's module is not left half transformed (the reference runs QuantizeFp4Pass /
    InsertQatStePass there, schemes.rs:128-145; this path does not build them)."""
    m = Module()
    w = torch.arange(16, dtype=torch.float32).reshape(4, 4)
    m.constant("w", w.clone())
    before = m.tensor_store.get("w").backing.data.clone()
    with pytest.raises(ValueError, match="not part of the HIP"):
        QuantizePass(scheme=scheme, hadamard=True, block_size=4).run(m)
    assert torch.equal(m.tensor_store.get("w").backing.data, before)
