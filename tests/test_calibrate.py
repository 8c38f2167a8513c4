"""CPU tests of static W8A8 calibration (`calibrate-quantize`, `quantize(scheme=w8a8)`;
passes/quantize/formats.rs:15-241) on modules without constants, so no kernel runs, and of
the oracle's restatement of `castforge.static_quantize` (codegen/eval.rs:1369-1382) against
closed forms: grid points are fixed points, exact ties round away from zero, values past the
grid clamp to +-qmax * scale, NaN passes, and bits == 4 clamps at 7."""
import math

import numpy as np
import pytest

import oracle_lib as O
from castforge_amd.ir import Module, TensorType
from castforge_amd.passes import CalibrateQuantizePass, PassManager, calibrate_value_ranges, default_registry


def test_static_quantize_oracle_closed_forms():
    for sc in (np.float32(0.25), np.float32(0.0078125), np.float32(3.0)):
        k = np.arange(-127, 128, dtype=np.float32)
        assert np.array_equal(O.static_quantize(k * sc, sc, 8), k * sc)           # grid points
        ties = (np.arange(-5, 5, dtype=np.float32) + np.float32(0.5)) * sc          # exact when sc is 2^e
        if sc in (np.float32(0.25), np.float32(0.0078125)):
            away = np.where(ties > 0, np.ceil(ties / sc), np.floor(ties / sc)) * sc
            assert np.array_equal(O.static_quantize(ties, sc, 8), away.astype(np.float32))
        big = np.array([1e6, -1e6, np.inf, -np.inf], np.float32)
        assert np.array_equal(O.static_quantize(big, sc, 8), np.array([127, -127, 127, -127], np.float32) * sc)
        assert np.array_equal(O.static_quantize(big, sc, 4), np.array([7, -7, 7, -7], np.float32) * sc)
    y = O.static_quantize(np.array([np.nan, -0.0, 0.0], np.float32), np.float32(0.5), 8)
    assert np.isnan(y[0]) and np.signbit(y[1]) and not np.signbit(y[2])


def _two_matmuls(k=4):
    m = Module("parallel_branches")
    x = m.add_argument(TensorType((2, k), "f32"), "x")
    w0 = m.add_argument(TensorType((k, k), "f32"), "w0")
    w1 = m.add_argument(TensorType((k, k), "f32"), "w1")
    b0 = m.dot_general(x, w0, name="b0")
    b1 = m.dot_general(b0, w1, name="b1")
    m.set_results(b1)
    return m, x, b0


def test_calibrate_ranges_and_scales():
    m, x, b0 = _two_matmuls(4)
    # 4 samples: scales 0.5, 0.75, 1.0, 1.25 -> every argument's bound is 1.25
    r = calibrate_value_ranges(m, 4)
    assert r[x] == 1.25 and r[b0] == 1.25 * 1.25 * math.sqrt(4.0)
    res = CalibrateQuantizePass(8, 4).run(m)
    assert res.changed and res.ops_created == 2 and res.ops_modified == 2
    dots = [m.ops[o] for o in m.block_ops() if m.ops[o].is_op("stablehlo", "dot_general")]
    sq = [m.ops[o] for o in m.block_ops() if m.ops[o].attributes.get("name") == "castforge.static_quantize"]
    assert len(dots) == 2 and len(sq) == 2
    assert dots[0].attributes["quant_mode"] == "w8a8_static"
    assert dots[0].attributes["lhs_scale"] == 1.25 / 127.0 and dots[0].attributes["rhs_scale"] == 1.25 / 127.0
    assert dots[1].attributes["lhs_scale"] == 1.25 * 1.25 * 2.0 / 127.0
    assert dots[0].attributes["calibration_samples"] == 4
    # each static_quantize sits right before its matmul and feeds its lhs
    order = m.block_ops()
    for q, d in zip(sq, dots):
        assert order.index(q.id) == order.index(d.id) - 1 and d.operands[0] == q.results[0]
        assert q.attributes["scale"] == d.attributes["lhs_scale"] and q.attributes["bits"] == 8
    assert "castforge.static_quantize" in m.print_mlir()
    m.verify()
    # already tagged: a second run changes nothing
    assert not CalibrateQuantizePass(8, 4).run(m).changed


def test_calibrate_bits4_and_pipeline_options():
    m, x, _ = _two_matmuls(4)
    res = PassManager.from_pipeline_str(default_registry(), "quantize(scheme=w8a8,bits=4,samples=2)").run(m)
    assert res[0].changed
    d = [m.ops[o] for o in m.block_ops() if m.ops[o].is_op("stablehlo", "dot_general")][0]
    # 2 samples: scales 0.5, 1.0 -> bound 1.0; bits 4 -> qmax 7
    assert d.attributes["quant_mode"] == "w4a4_static" and d.attributes["lhs_scale"] == 1.0 / 7.0
    m2, _, _ = _two_matmuls(4)
    # scheme inferred from `samples` (families.rs:93-183); the leaf pass by name
    PassManager.from_pipeline_str(default_registry(), "quantize(samples=1)").run(m2)
    d2 = [m2.ops[o] for o in m2.block_ops() if m2.ops[o].is_op("stablehlo", "dot_general")][0]
    assert d2.attributes["lhs_scale"] == 0.8 / 127.0  # one sample (0.5): the 0.8 floor
    m3, _, _ = _two_matmuls(4)
    assert PassManager.from_pipeline_str(default_registry(), "calibrate-quantize(bits=8,samples=3)").run(m3)[0].changed


def test_calibrate_skips_non_float_lhs():
    m = Module("t")
    x = m.add_argument(TensorType((2, 4), "i8"), "x")
    w = m.add_argument(TensorType((4, 4), "f32"), "w")
    m.set_results(m.dot_general(x, w))
    assert not CalibrateQuantizePass().run(m).changed
