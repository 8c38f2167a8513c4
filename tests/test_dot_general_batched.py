"""Batched / rank-3 `stablehlo.dot_general` in the evaluator: eval_dot_general's flat form
(eval.rs:1509-1604) past its 2-D case.  GPU: bit-identical to the oracle's restatement
(oracle_lib.dot_general_flat, one orc_matmul_2d per batch) for both rhs layouts, and a rank-3
activation against a 2-D weight.  CPU: operands that do not factor as [batch, m, k] x
[batch, k, n] are refused with a message, before any kernel runs."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd.evaluate import evaluate_module
from castforge_amd.ir import Module, TensorType


def _module(ls, rs, out, lb, rb, lc, rc):
    mod = Module()
    a = mod.add_argument(TensorType(ls, "f32"), "a")
    b = mod.add_argument(TensorType(rs, "f32"), "b")
    attrs = {"lhs_batching_dimensions": lb, "rhs_batching_dimensions": rb,
             "lhs_contracting_dimensions": lc, "rhs_contracting_dimensions": rc}
    y = mod.add_op("stablehlo.dot_general", [a, b], [TensorType(out, "f32")], attrs, ["y"]).results[0]
    mod.set_results(y)
    return mod


@pytest.mark.gpu
@pytest.mark.parametrize("contract_last", [False, True])
def test_batched_dot_general_vs_oracle(cuda, contract_last):
    bt, m, k, n = 4, 9, 70, 13
    rng = np.random.default_rng(40 + contract_last)
    a = rng.standard_normal((bt, m, k)).astype(np.float32)
    b = rng.standard_normal((bt, n, k) if contract_last else (bt, k, n)).astype(np.float32)
    mod = _module((bt, m, k), b.shape, (bt, m, n), [0], [0], [2], [2 if contract_last else 1])
    y = evaluate_module(mod, [torch.from_numpy(a).to(cuda), torch.from_numpy(b).to(cuda)], "f32")[0]
    assert tuple(y.shape) == (bt, m, n)
    assert np.array_equal(y.cpu().numpy(), O.dot_general_flat(a, b, bt, k, contract_last))


@pytest.mark.gpu
def test_rank3_activation_dot_general_vs_oracle(cuda):
    """A [2, 6, 64] activation against a [64, 24] weight, no batching dimensions: the reference
    reads it flat as [1, 12, 64] (batch 1, m = |lhs| / k)."""
    rng = np.random.default_rng(42)
    a = rng.standard_normal((2, 6, 64)).astype(np.float32)
    w = rng.standard_normal((64, 24)).astype(np.float32)
    mod = _module((2, 6, 64), (64, 24), (2, 6, 24), [], [], [2], [0])
    y = evaluate_module(mod, [torch.from_numpy(a).to(cuda), torch.from_numpy(w).to(cuda)], "f32")[0]
    ref = O.dot_general_flat(a, w, 1, 64, False).reshape(2, 6, 24)
    assert np.array_equal(y.cpu().numpy(), ref)
    assert np.array_equal(ref.reshape(12, 24), O.matmul_2d(a.reshape(12, 64), w, False))


def test_dot_general_that_does_not_factor_is_refused():
    # k = 6 from the lhs, but |rhs| = 35 is not a multiple of batch * k
    mod = _module((2, 3, 6), (5, 7), (2, 3, 5), [], [], [2], [1])
    with pytest.raises(ValueError, match="do not factor"):
        evaluate_module(mod, [torch.zeros((2, 3, 6)), torch.zeros((5, 7))], "f32")
    mod = _module((2, 3, 6), (2, 6, 4), (2, 3, 4), [3], [0], [2], [1])
    with pytest.raises(ValueError, match="outside an operand of rank 3"):
        evaluate_module(mod, [torch.zeros((2, 3, 6)), torch.zeros((2, 6, 4))], "f32")
