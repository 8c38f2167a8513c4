"""GPU parity at the shapes and launch forms bench.py times, against the oracle's evaluator
semantics (dequantize to f32, then the f32 m,n,k loop of eval_matmul_2d, eval.rs:1465-1507):
every sampled output within |y - ref| <= 1e-3 + 1e-2 * |ref|.

- NF4 block 64 at M = 64: W_gate, W_up and W_down (K = 11008) in ONE batched launch, as the
  nf4_gemm_m64 component runs it;
- NF4 block 64 at M = 512 on W_down (4096 x 11008), the prefill kernel's 64 x 64-tile instance;
- W4A16 INT4 g128 at M = 16 over the whole 7-matrix block in one batched launch (config 2);
- W4A16 INT4 g128 prefill at M = 4096 on the W_gate and W_down shapes, 64 rows x 128 columns.

y[m, n] depends only on x[m] and W[n], so the oracle runs on sampled rows and columns.  The
weights are drawn on the GPU (N(0, 0.02), seeded) and quantized there; the quantizers are
bit-exact with the oracle (tests/test_gpu_quantize.py), and the oracle here reads the codes
back.  Activations carry 1% of channels x20."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ops, synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _close(y, ref, what):
    err = np.abs(y - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}"


def _w(seed, n, k, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randn((n, k), generator=g, device=dev, dtype=torch.float32) * 0.02


def _x(seed, m, k, dev):
    xb = synth.activations_bf16(seed, 11, m, k)
    return xb, torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)


def _sample(rng, m, n, rows, cols):
    return np.sort(rng.choice(m, min(rows, m), replace=False)), np.sort(rng.choice(n, min(cols, n), replace=False))


def _nf4_ref(xb, p, rows, cols):
    codes = p.codes.cpu().numpy().view(np.uint32)[cols]
    am = p.absmax.cpu().numpy()[cols]
    return O.gemm_nf4(np.ascontiguousarray(xb[rows]), np.ascontiguousarray(codes), np.ascontiguousarray(am),
                      len(cols), p.k, p.block)


def _int4_ref(xb, p, rows, cols):
    c = p.codes.cpu().numpy().view(np.uint32)[cols]
    s = p.scales.cpu().numpy().view(np.uint16)[cols]
    z = p.zeros.cpu().numpy().view(np.uint32)[cols]
    return O.gemm_w4a16(np.ascontiguousarray(xb[rows]), np.ascontiguousarray(c), np.ascontiguousarray(s),
                        np.ascontiguousarray(z), len(cols), p.k, p.group)


def test_nf4_m64_batched_mlp(cuda):
    """nf4_gemm_m64: W_gate / W_up / W_down in one launch (skinny kernel, K up to 11008)."""
    m = 64
    mlp = synth.LLAMA7B_BLOCK[4:]
    ps = [ops.quantize_nf4(_w(300 + i, n, k, cuda), 64) for i, (_, n, k) in enumerate(mlp)]
    xbs, xs = zip(*[_x(310 + i, m, k, cuda) for i, (_, n, k) in enumerate(mlp)])
    ys = [torch.empty((m, n), dtype=torch.bfloat16, device=cuda) for (_, n, k) in mlp]
    print("[bench shapes] NF4 M=64 batched W_gate/W_up/W_down", flush=True)
    ops.gemv_nf4_batched(list(xs), ps, ys)
    torch.cuda.synchronize()
    rng = np.random.default_rng(31)
    for (name, n, k), xb, p, y in zip(mlp, xbs, ps, ys):
        rows, cols = _sample(rng, m, n, 64, 160)
        _close(y.float().cpu().numpy()[np.ix_(rows, cols)], _nf4_ref(xb, p, rows, cols), f"nf4 m64 {name}")


def test_nf4_m512_w_down(cuda):
    """nf4_gemm_m512 on W_down (4096 x 11008): the prefill kernel's 64 x 64-tile instance."""
    m, n, k = 512, 4096, 11008
    p = ops.quantize_nf4(_w(320, n, k, cuda), 64)
    xb, x = _x(321, m, k, cuda)
    print("[bench shapes] NF4 M=512 W_down", flush=True)
    y = ops.gemm_nf4(x, p, torch.bfloat16)
    torch.cuda.synchronize()
    rows, cols = _sample(np.random.default_rng(32), m, n, 48, 96)
    _close(y.float().cpu().numpy()[np.ix_(rows, cols)], _nf4_ref(xb, p, rows, cols), "nf4 m512 w_down")


def test_w4a16_m16_block_batched(cuda):
    """w4a16_gemv_m16: the 7 projections at M = 16 in one batched launch (config 2)."""
    m = 16
    ps = [ops.quantize_int4g(_w(330 + i, n, k, cuda), 128) for i, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK)]
    xbs, xs = zip(*[_x(340 + i, m, k, cuda) for i, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK)])
    ys = [torch.empty((m, n), dtype=torch.bfloat16, device=cuda) for (_, n, k) in synth.LLAMA7B_BLOCK]
    print("[bench shapes] W4A16 M=16 batched block", flush=True)
    ops.gemv_w4a16_batched(list(xs), ps, ys)
    torch.cuda.synchronize()
    rng = np.random.default_rng(33)
    for (name, n, k), xb, p, y in zip(synth.LLAMA7B_BLOCK, xbs, ps, ys):
        rows, cols = _sample(rng, m, n, 16, 256)
        _close(y.float().cpu().numpy()[np.ix_(rows, cols)], _int4_ref(xb, p, rows, cols), f"w4a16 m16 {name}")


@pytest.mark.parametrize("name,n,k", [("w_gate", 11008, 4096), ("w_down", 4096, 11008)])
def test_w4a16_prefill_m4096_64x128(cuda, name, n, k):
    """w4a16_prefill_m4096: 64 rows x 128 columns of each shape."""
    m = 4096
    p = ops.quantize_int4g(_w(350 + n, n, k, cuda), 128)
    xb, x = _x(351, m, k, cuda)
    print(f"[bench shapes] W4A16 prefill M=4096 {name}", flush=True)
    y = ops.gemm_w4a16(x, p, torch.bfloat16)
    torch.cuda.synchronize()
    rows, cols = _sample(np.random.default_rng(34), m, n, 64, 128)
    _close(y.float().cpu().numpy()[np.ix_(rows, cols)], _int4_ref(xb, p, rows, cols), f"w4a16 m4096 {name}")
