"""GPU parity of the outlier-suppression passes: Walsh-Hadamard rotation (formats.rs:230-343)
and SmoothQuant (schemes.rs:155-298), bit-exact against the oracle restatements; the
one-pass rotate+INT4g quantizer against the two-pass composition; and the passes' graph
effects as the reference's tests check them (frontend_tests.rs:820-860)."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ffi, ops, synth
from castforge_amd.ir import Module, TensorType
from castforge_amd.passes import PassManager, calibrate_value_ranges, default_registry

pytestmark = pytest.mark.gpu


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


@pytest.mark.parametrize("k,n,b", [(8, 3, 2), (64, 33, 4), (64, 33, 64), (4096, 100, 128), (2048, 64, 1024),
                                   (8192, 16, 4096), (128, 4096, 32)])
def test_rotate_columns_bit_exact(cuda, k, n, b):
    w = synth.weight(70, k, k, n)
    got = ops.rotate_hadamard(_t(w, cuda), b, 0)
    torch.cuda.synchronize()
    want, rb = O.rotate_hadamard(w, b)
    assert rb == b
    np.testing.assert_array_equal(_bits(got.cpu().numpy()), _bits(want))


@pytest.mark.parametrize("d0,d1,b", [(3, 16, 2), (5, 4096, 8), (7, 4096, 512), (4, 4096, 1024), (2, 8192, 4096),
                                     (33, 11008, 256), (1, 64, 64), (9, 4096, 16), (6, 4096, 32),
                                     (40, 4096, 128), (3, 128, 128), (5, 11008, 64)])
def test_rotate_rows_bit_exact(cuda, d0, d1, b):
    w = synth.weight(71, d1, d0, d1)
    got = ops.rotate_hadamard(_t(w, cuda), b, 1)
    torch.cuda.synchronize()
    want, _ = O.rotate_hadamard(np.ascontiguousarray(w.T), b)
    np.testing.assert_array_equal(_bits(got.cpu().numpy()), _bits(np.ascontiguousarray(want.T)))


@pytest.mark.parametrize("b", [16, 32, 64, 128])
def test_rotate_rows_special_values(cuda, b):
    """Exact zeros, -0 (whole rows and half rows: one 512-value wave with and one without),
    +-inf, NaN, values whose butterflies overflow, values just below the kernel's 2^117
    overflow guard, and blocks that cancel to exact zeros: every non-NaN output has the
    oracle's bits, -0 and +0 included, and NaN outputs are where the oracle's are."""
    d0, d1 = 12, 1024
    rng = np.random.default_rng(76)
    w = rng.standard_normal((d0, d1)).astype(np.float32)
    w[0] = 0.0
    w[1] = -0.0
    w[2, :512] = -0.0
    w[3, ::5] = np.inf
    w[4, 3::7] = np.nan
    w[5, ::3] = 3e38
    w[6] = 1.0                              # every difference of the first stage is exactly 0
    w[7, 0::2], w[7, 1::2] = 0.5, -0.5
    w[8] = np.float32(2.0 ** 117)           # at the guard: the exact path
    w[9] = np.float32(2.0 ** 116)           # below it: the one-fma path, no overflow
    w[10, ::2] = -w[10, 1::2]
    got = ops.rotate_hadamard(_t(w, cuda), b, 1).cpu().numpy()
    want, _ = O.rotate_hadamard(np.ascontiguousarray(w.T), b)
    want = np.ascontiguousarray(want.T)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(_bits(got)[~nan], _bits(want)[~nan])


def test_rotate_in_place_and_unaligned(cuda):
    w = synth.weight(72, 1, 6, 1024)
    buf = torch.zeros(6 * 1024 + 1, dtype=torch.float32, device=cuda)
    buf[1:] = _t(w, cuda).reshape(-1)
    p = buf.data_ptr() + 4
    ffi.call("castforge_hip_rotate_hadamard", p, 6, 1024, 256, 1, p, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want, _ = O.rotate_hadamard(np.ascontiguousarray(w.T), 256)
    np.testing.assert_array_equal(_bits(buf[1:].cpu().numpy()), _bits(np.ascontiguousarray(want.T).reshape(-1)))
    assert buf[0].item() == 0.0
    with pytest.raises(ffi.CastForgeHipError, match="multiple of block"):
        ops.rotate_hadamard(_t(w, cuda), 64, 0)


@pytest.mark.parametrize("group", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("b", [2, 16, 32, 64, 128, 256, 1024])
def test_fused_hadamard_int4g_equals_two_pass(cuda, group, b):
    w = _t(synth.weight(73, group, 96, 4096), cuda)
    fused = ops.quantize_int4g_hadamard(w, group, b)
    two = ops.quantize_int4g(ops.rotate_hadamard(w, b, 1), group)
    for a, c in ((fused.codes, two.codes), (fused.scales, two.scales), (fused.zeros, two.zeros)):
        assert torch.equal(a, c)


@pytest.mark.parametrize("b", [32, 128, 256])
def test_fused_hadamard_int4g_special_values(cuda, b):
    """Exact zeros, -0, +-inf, NaN, values whose butterflies overflow, and blocks that cancel to
    exact zeros: the fused quantizer's codes, scales and zero points equal the two-pass ones
    (its Hadamard stages may give a zero or a NaN the other sign, which no code depends on)."""
    rng = np.random.default_rng(75)
    w = (rng.standard_normal((24, 2048)) * 0.02).astype(np.float32)
    w[0, :] = 0.0
    w[1, :] = -0.0
    w[2, ::7] = np.inf
    w[3, 5::11] = -np.inf
    w[4, 3::13] = np.nan
    w[5, ::3] = 3e38
    w[6, :] = 1.0                        # every block sums to b, every difference to exactly 0
    w[7, 0::2], w[7, 1::2] = 0.5, -0.5   # cancellations at h = 1
    w[8, :1024] = -0.0
    w = _t(w, cuda)
    for group in (32, 128):
        fused = ops.quantize_int4g_hadamard(w, group, b)
        two = ops.quantize_int4g(ops.rotate_hadamard(w, b, 1), group)
        for a, c in ((fused.codes, two.codes), (fused.scales, two.scales), (fused.zeros, two.zeros)):
            assert torch.equal(a, c), (group, b)


def test_fused_hadamard_int4g_many_rows(cuda):
    w = _t(synth.weight(74, 1, 70000, 64), cuda)
    fused = ops.quantize_int4g_hadamard(w, 32, 64)
    two = ops.quantize_int4g(ops.rotate_hadamard(w, 64, 1), 32)
    assert torch.equal(fused.codes, two.codes) and torch.equal(fused.scales, two.scales)
    assert torch.equal(fused.zeros, two.zeros)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("act,alpha", [(4.0, 0.5), (30.0, 0.8), (0.01, 0.3), (1e-7, 0.05)])
def test_smoothquant_kernel_bit_exact(cuda, bits, act, alpha):
    w = synth.weight(75, 1, 64, 1000)
    w[0, :3] = [np.nan, -0.0, 1e-30]
    want, s, e = O.smoothquant(w, act, alpha, bits)
    w_max = max(float(np.float32(ops.absmax(_t(w, cuda)))), float(np.float32(1e-5)))
    s2, e2 = ops.smoothquant_scales(act, w_max, float(np.float32(min(max(alpha, 0.05), 0.95))), bits)
    assert (np.float32(s2), np.float32(e2)) == (s, e)
    got = ops.smoothquant(_t(w, cuda), s2, e2, bits)
    torch.cuda.synchronize()
    g = got.cpu().numpy()
    assert np.array_equal(np.isnan(g), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_array_equal(_bits(g)[ok], _bits(want)[ok])


# ------------------------------------------------------------------------------ passes ----
def _frontend_module(dev, w=None, b=None):
    """frontend_tests.rs:167-179: x[2,4] . w + b with w = 0.5, b = 0.1 (inline constants)."""
    m = Module("frontend")
    x = m.add_argument(TensorType((2, 4), "f32"), "x")
    wv = m.constant("w", _t(np.full((4, 4), 0.5) if w is None else w, dev), inline=True)
    bv = m.constant("b", _t(np.full((2, 4), 0.1) if b is None else b, dev), inline=True)
    mm = m.dot_general(x, wv, name="mm")
    m.set_results(m.add_op("stablehlo.add", [mm, bv], [TensorType((2, 4), "f32")], {}, ["y"]).results[0])
    return m


def _const(m, name):
    op = [o for o in m.ops.values() if o.results and m.values[o.results[0]].ssa_name == name][0]
    return op


def test_quantize_scheme_hadamard_reference_case(cuda):
    """frontend_tests.rs:820-839: quantize(scheme=hadamard,block_size=64) changes the module
    and prints castforge.hadamard_rotated = true."""
    w = synth.weight(76, 1, 4, 4)
    m = _frontend_module(cuda, w)
    res = PassManager.from_pipeline_str(default_registry(), "quantize(scheme=hadamard,block_size=64)").run(m)
    assert res[0].changed and res[0].pass_name == "quantize"
    assert "castforge.hadamard_rotated = true" in m.print_mlir()
    want, b = O.rotate_hadamard(w, 64)  # b = min(64, k = 4) = 4
    assert b == 4
    np.testing.assert_array_equal(_bits(_const(m, "w").attributes["value"].data.cpu().numpy()), _bits(want))
    mm = [o for o in m.ops.values() if o.name == "stablehlo.dot_general"][0]
    assert mm.attributes["castforge.hadamard_block"] == 4
    # b [2, 4]: b = 2, rotated along its 2 rows; a second run skips both constants
    bo = _const(m, "b")
    assert bo.attributes["castforge.hadamard_rotated"] is True
    r2 = PassManager.from_pipeline_str(default_registry(), "rotate-hadamard").run(m)
    assert not r2[0].changed


def test_rotate_hadamard_tags_without_rotating_when_not_divisible(cuda):
    m = Module("odd")
    x = m.add_argument(TensorType((1, 6), "f32"), "x")
    w = synth.weight(77, 1, 6, 3)
    wv = m.constant("w", _t(w, cuda))
    m.set_results(m.dot_general(x, wv, name="y"))
    res = PassManager.from_pipeline_str(default_registry(), "rotate-hadamard(block_size=4)").run(m)
    assert res[0].changed and res[0].ops_modified == 1
    np.testing.assert_array_equal(m.tensor_store.get("w").backing.data.reshape(6, 3).cpu().numpy(), w)
    m3 = Module("bad")
    x = m3.add_argument(TensorType((1, 3), "f32"), "x")
    m3.set_results(m3.dot_general(x, m3.constant("w", _t(synth.weight(78, 1, 3, 2), cuda)), name="y"))
    with pytest.raises(ValueError, match="not a power of two"):
        PassManager.from_pipeline_str(default_registry(), "rotate-hadamard(block_size=4)").run(m3)


def test_quantize_hadamard_then_per_tensor(cuda):
    """quantize(bits=8,hadamard=true,block_size=8): rotation first, then quantize-weights on
    the rotated values (schemes.rs:105-112).  (Without bits, block_size alone makes the option
    inference pick scheme=hadamard: rotation only, families.rs:93-116.)"""
    w = synth.weight(79, 1, 32, 16)
    m = Module("h8")
    x = m.add_argument(TensorType((1, 32), "f32"), "x")
    m.set_results(m.dot_general(x, m.constant("w", _t(w, cuda)), name="y"))
    res = PassManager.from_pipeline_str(default_registry(), "quantize(bits=8,hadamard=true,block_size=8)").run(m)
    assert res[0].changed and res[0].ops_modified == 2
    rot, _ = O.rotate_hadamard(w, 8)
    q, s = O.quantize_symmetric(rot, 8, 0)
    e = m.tensor_store.get("w").backing
    np.testing.assert_array_equal(e.data.cpu().numpy().reshape(-1), q.reshape(-1))
    assert np.float32(e.scale) == s


def test_fused_k_axis_int4_equals_reference_order(cuda):
    """pack-weights, quantize(scheme=int4_asym, hadamard=true, hadamard_axis=k): the same
    codes as rotate-hadamard on the [K, N] weight, then pack-weights and int4_asym."""
    w = synth.weight(80, 1, 1024, 96)  # [K, N]
    reg = default_registry()

    def mod():
        m = Module("kq")
        x = m.add_argument(TensorType((1, 1024), "f32"), "x")
        m.set_results(m.dot_general(x, m.constant("w", _t(w, cuda)), name="y"))
        return m
    a, b = mod(), mod()
    ra = PassManager.from_pipeline_str(reg, "pack-weights,quantize(scheme=int4_asym,hadamard=true,hadamard_axis=k,block_size=128)").run(a)
    PassManager.from_pipeline_str(reg, "rotate-hadamard(block_size=128),pack-weights,quantize(scheme=int4_asym)").run(b)
    assert ra[1].changed and ra[1].ops_modified == 2
    pa, pb = a.tensor_store.get("w").backing, b.tensor_store.get("w").backing
    for part in ("codes", "scales", "zeros"):
        assert torch.equal(getattr(pa, part), getattr(pb, part))
    assert "castforge.hadamard_rotated = true" in a.print_mlir()


def test_smoothquant_pass_reference_case_and_values(cuda):
    """frontend_tests.rs:847-860: quantize(scheme=smoothquant,alpha=0.5) tags
    castforge.quant_scheme = "smoothquant"; values equal the oracle with act_max the
    constant's calibrated bound."""
    w = synth.weight(81, 1, 4, 4) * 10
    bias = synth.weight(82, 1, 2, 4)
    m = _frontend_module(cuda, w, bias)
    ranges = calibrate_value_ranges(m, 4)
    acts = {n: float(np.float32(ranges[_const(m, n).results[0]])) for n in ("w", "b")}
    res = PassManager.from_pipeline_str(default_registry(), "quantize(scheme=smoothquant,alpha=0.5)").run(m)
    assert res[0].changed and res[0].ops_modified == 2
    assert 'castforge.quant_scheme = "smoothquant"' in m.print_mlir()
    for name, src in (("w", w), ("b", bias)):
        want, _, _ = O.smoothquant(src, acts[name], 0.5, 8)
        got = _const(m, name).attributes["value"].data.cpu().numpy()
        np.testing.assert_array_equal(_bits(got), _bits(want))
    mm = [o for o in m.ops.values() if o.name == "stablehlo.dot_general"][0]
    assert mm.attributes["castforge.quant_bits"] == 8 and mm.attributes["castforge.smoothquant_alpha"] == 0.5
