"""Oracle of rotate-hadamard (formats.rs:301-327) and smooth-quantize (schemes.rs:188-238) on
the CPU, pinned by mathematics: the Sylvester Hadamard matrix (scipy.linalg.hadamard) on
integer data, exact where 1/sqrt(b) is a power of two; the block-size rule on its edge cases;
the rotation's orthogonality (applied twice it returns the input); SmoothQuant's closed form
when s = 1 (act_max = w_max, alpha = 0.5) and its fixed points.  Also the pass registry."""
import numpy as np
import pytest
from scipy.linalg import hadamard

import oracle_lib as O
from castforge_amd.passes import PassManager, RotateHadamardPass, SmoothQuantizePass, default_registry


@pytest.mark.parametrize("b", [4, 16, 64, 256])
def test_rotation_equals_sylvester_matrix_exactly(b):
    rng = np.random.default_rng(b)
    k, n = 2 * b, 5
    w = rng.integers(-50, 50, (k, n)).astype(np.float32)
    r, got_b = O.rotate_hadamard(w, b)
    assert got_b == b
    H = np.kron(np.eye(k // b), hadamard(b)).astype(np.float64)
    want = (H @ w.astype(np.float64)) / np.sqrt(b)  # 1/sqrt(b) is a power of two here: exact
    np.testing.assert_array_equal(r, want.astype(np.float32))


@pytest.mark.parametrize("b", [2, 8, 32, 128])
def test_rotation_close_to_sylvester_and_involutive(b):
    rng = np.random.default_rng(b)
    w = rng.standard_normal((b * 3, 7)).astype(np.float32)
    r, _ = O.rotate_hadamard(w, b)
    H = np.kron(np.eye(3), hadamard(b)) / np.sqrt(b)
    np.testing.assert_allclose(r, H @ w.astype(np.float64), rtol=0, atol=1e-5 * np.abs(w).max() * np.sqrt(b))
    rr, _ = O.rotate_hadamard(r, b)
    np.testing.assert_allclose(rr, w, rtol=0, atol=1e-5 * np.abs(w).max())


@pytest.mark.parametrize("block,k,want_b,rotated", [
    (4, 8, 4, True), (5, 16, 8, True), (64, 16, 16, True), (0, 4, 2, True),
    (1, 3, 2, False),   # 3 % 2 != 0: unchanged
    (4, 6, 4, False),   # 6 % 4 != 0: unchanged
    (4, 3, -1, False),  # b = 3: not a power of two (the reference panics)
])
def test_block_rule(block, k, want_b, rotated):
    w = np.arange(k * 2, dtype=np.float32).reshape(k, 2) + 1
    r, b = O.rotate_hadamard(w, block)
    assert b == want_b
    assert (not np.array_equal(r, w)) == rotated


def test_smoothquant_closed_form_when_scale_is_one():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal(1000) * 2).astype(np.float32)
    w[0] = 4.0
    w = np.clip(w, -4, 4)
    out, s, e = O.smoothquant(w, 4.0, 0.5, 8)  # act_max = w_max = 4: s = 4^0.5 / 4^0.5 = 1
    assert s == np.float32(1.0)
    assert e == np.float32(np.float32(4.0) / np.float32(127.0))
    q = np.clip(np.sign(w / e) * np.floor(np.abs(w / e) + np.float32(0.5)), -128, 127).astype(np.float32)
    np.testing.assert_array_equal(out, (q * e).astype(np.float32))
    again, _, _ = O.smoothquant(out, 4.0, 0.5, 8)
    np.testing.assert_array_equal(again, out)  # grid values are fixed points


def test_smoothquant_alpha_clamp_bits4_and_nan():
    w = np.array([1.0, -2.0, 0.3, np.nan], np.float32)
    out, s, e = O.smoothquant(w, 8.0, 1.0, 4)
    a = np.float32(0.95)
    s_want = max(np.float32(np.float32(8.0) ** a / np.float32(2.0) ** (np.float32(1) - a)), np.float32(1e-4))
    assert abs(float(s) - float(s_want)) <= 2 * np.spacing(np.float32(s_want))
    assert np.isnan(out[3])
    assert np.all(np.abs(out[:3] * s / e) <= 8.0 + 1e-3)
    q = np.rint(out[:3] * s / e)
    assert q.min() >= -8 and q.max() <= 7


def test_registry_builds_outlier_passes():
    reg = default_registry()
    pm = PassManager.from_pipeline_str(reg, "rotate-hadamard(block_size=8),smooth-quantize(alpha=0.7,bits=4,samples=2)")
    rot, sq = pm.passes
    assert isinstance(rot, RotateHadamardPass) and rot.block_size == 8
    assert isinstance(sq, SmoothQuantizePass) and sq.bits == 4 and sq.num_samples == 2
    assert abs(sq.alpha - 0.7) < 1e-7
    q = PassManager.from_pipeline_str(reg, "quantize(scheme=hadamard,block_size=64)").passes[0]
    assert q.scheme == "hadamard" and q.block_size == 64
    q = PassManager.from_pipeline_str(reg, "quantize(scheme=int4_asym,hadamard=true,hadamard_axis=k)").passes[0]
    assert q.hadamard and q.hadamard_axis == "k"
