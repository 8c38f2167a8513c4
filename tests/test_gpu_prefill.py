"""GPU parity of the prefill (M > 16) dequant-fused GEMM on MFMA against the oracle's evaluator
semantics (dequantize to f32, then the f32 m,n,k loop of eval_matmul_2d): every output within
|y - ref| <= 1e-3 + 1e-2 * |ref|, the north-star tolerance.  Activations carry 1% of channels
scaled x20, the case where a weight rounded to 16 bits would fail the
absolute bound on near-zero outputs.  Full BASELINE shapes are checked on sampled rows and
columns: y[m, n] depends only on x[m] and W[n], so the oracle runs on the sampled slices."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from castforge_amd import ops, synth

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 1e-3


def _close(y, ref, what=""):
    y = y.float().cpu().numpy() if isinstance(y, torch.Tensor) else y
    err = np.abs(y - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{what}: {bad.sum()} / {bad.size} outside tol; max err {err.max():.3e}"


def _x(seed, m, k, dev):
    xb = synth.activations_bf16(seed, 7, m, k)
    return xb, torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)


def _int4(w, group, dev):
    codes, scales, zeros = O.quantize_int4g(w, group)
    n, k = w.shape
    p = ops.Int4Packed(torch.from_numpy(codes.view(np.int32)).to(dev),
                       torch.from_numpy(scales.view(np.float16)).to(dev),
                       torch.from_numpy(zeros.view(np.int32)).to(dev), n, k, group)
    return p, (codes, scales, zeros)


# INT4 prefill kernel: "auto" picks by shape (the one-MFMA kernel once its tiles fill the chip),
# "0" keeps the generic two-term kernel, "1" forces the one-MFMA kernel wherever the groups
# are whole 128-wide K blocks (CASTFORGE_PREFILL_I4).
I4_KERNELS = ["auto", "0", "1"]


def _i4_kernel(monkeypatch, kernel):
    if kernel == "auto":
        monkeypatch.delenv("CASTFORGE_PREFILL_I4", raising=False)
    else:
        monkeypatch.setenv("CASTFORGE_PREFILL_I4", kernel)


@pytest.mark.parametrize("kernel", I4_KERNELS)
@pytest.mark.parametrize("m", [17, 64, 130, 256, 300])
@pytest.mark.parametrize("n,k", [(256, 1024), (300, 512), (520, 2048)])
@pytest.mark.parametrize("out", [torch.float32, torch.bfloat16])
def test_w4a16_prefill(cuda, monkeypatch, kernel, m, n, k, out):
    _i4_kernel(monkeypatch, kernel)
    print(f"[prefill w4a16] kernel={kernel} m={m} n={n} k={k} out={out}", flush=True)
    w = synth.weight(81, 1, n, k)
    p, (c, s, z) = _int4(w, 128, cuda)
    xb, x = _x(82, m, k, cuda)
    y = ops.gemm_w4a16(x, p, out)
    torch.cuda.synchronize()
    _close(y, O.gemm_w4a16(xb, c, s, z, n, k, 128), "w4a16")


@pytest.mark.parametrize("kernel", I4_KERNELS)
@pytest.mark.parametrize("group", [32, 64, 256, 1024])
def test_w4a16_prefill_groups(cuda, monkeypatch, kernel, group):
    _i4_kernel(monkeypatch, kernel)
    m, n, k = 96, 264, 2048
    print(f"[prefill w4a16 group] kernel={kernel} group={group}", flush=True)
    w = synth.weight(83, 1, n, k)
    p, (c, s, z) = _int4(w, group, cuda)
    xb, x = _x(84, m, k, cuda)
    y = ops.gemm_w4a16(x, p, torch.float32)
    torch.cuda.synchronize()
    _close(y, O.gemm_w4a16(xb, c, s, z, n, k, group), f"group {group}")


@pytest.mark.parametrize("m", [40, 64, 512])
@pytest.mark.parametrize("block", [32, 64, 128])
def test_nf4_prefill(cuda, m, block):
    n, k = 384, 1024
    print(f"[prefill nf4] m={m} block={block}", flush=True)
    w = synth.weight(85, 1, n, k)
    xb, x = _x(86, m, k, cuda)
    p = ops.quantize_nf4(torch.from_numpy(w).to(cuda), block)
    y = ops.gemm_nf4(x, p, torch.bfloat16)
    torch.cuda.synchronize()
    ref = O.gemm_nf4(xb, p.codes.cpu().numpy().view(np.uint32), p.absmax.cpu().numpy(), n, k, block)
    _close(y, ref, "nf4")


@pytest.mark.parametrize("tile", ["256x256", "128x256", "128x128", "64x128", "64x64"])
@pytest.mark.parametrize("fmt", ["int4", "nf4", "int8"])
def test_prefill_every_tile_shape(cuda, monkeypatch, tile, fmt):
    """Each tile shape forced through CASTFORGE_PREFILL_TILE, with partial tiles in m and n
    (300 x 328 is not a multiple of any tile) and K over several slices."""
    m, n, k = 300, 328, 768
    print(f"[prefill tile] {fmt} {tile}", flush=True)
    monkeypatch.setenv("CASTFORGE_PREFILL_TILE", tile)
    w = synth.weight(91, 1, n, k)
    xb, x = _x(92, m, k, cuda)
    if fmt == "int4":
        p, (c, s, z) = _int4(w, 128, cuda)
        y = ops.gemm_w4a16(x, p, torch.float32)
        ref = O.gemm_w4a16(xb, c, s, z, n, k, 128)
    elif fmt == "nf4":
        p = ops.quantize_nf4(torch.from_numpy(w).to(cuda), 64)
        y = ops.gemm_nf4(x, p, torch.bfloat16)
        ref = O.gemm_nf4(xb, p.codes.cpu().numpy().view(np.uint32), p.absmax.cpu().numpy(), n, k, 64)
    else:
        q, sc = ops.quantize_int8(torch.from_numpy(w).to(cuda), 8, "channel")
        y = ops.gemm_w8a16(x, q, sc, "channel", torch.float32)
        ref = O.gemm_w8a16(xb, q.cpu().numpy(), sc.cpu().numpy())
    torch.cuda.synchronize()
    _close(y, ref, f"{fmt} {tile}")


@pytest.mark.parametrize("kernel", I4_KERNELS)
@pytest.mark.parametrize("m,n,k", [(17, 300, 1024), (200, 300, 1024), (300, 520, 2048), (129, 257, 640)])
@pytest.mark.parametrize("gran", ["channel", "tensor"])
def test_w8a16_prefill(cuda, monkeypatch, kernel, m, n, k, gran):
    """INT8 at M > 16; kernel "1" forces the one-MFMA kernel (K % 128 == 0: exact q, the row or
    tensor scale applied once to the f32 sum), "0" the generic kernel."""
    _i4_kernel(monkeypatch, kernel)
    print(f"[prefill w8a16] kernel={kernel} m={m} n={n} k={k} gran={gran}", flush=True)
    w = synth.weight(87, 1, n, k)
    xb, x = _x(88, m, k, cuda)
    q, s = ops.quantize_int8(torch.from_numpy(w).to(cuda), 8, gran, "half_even")
    y = ops.gemm_w8a16(x, q, s, gran, torch.float32)
    torch.cuda.synchronize()
    sc = s.cpu().numpy()
    sc = sc if gran == "channel" else np.full(n, sc[0], np.float32)
    _close(y, O.gemm_w8a16(xb, q.cpu().numpy(), sc), "w8a16")


@pytest.mark.parametrize("kernel", I4_KERNELS)
def test_prefill_unaligned_output(cuda, monkeypatch, kernel):
    """N % 4 != 0 and an output view that is not 16-byte aligned take the checked stores."""
    _i4_kernel(monkeypatch, kernel)
    m, n, k = 70, 262, 512
    w = synth.weight(89, 1, n, k)
    p, (c, s, z) = _int4(w, 128, cuda)
    xb, x = _x(90, m, k, cuda)
    ref = O.gemm_w4a16(xb, c, s, z, n, k, 128)
    buf = torch.full((m * n + 1,), -7.0, dtype=torch.float32, device=cuda)
    y = buf[1:].view(m, n)
    from castforge_amd import ffi
    ffi.call("castforge_hip_gemv_w4a16", x.data_ptr(), m, n, k, 128, p.codes.data_ptr(), p.scales.data_ptr(),
             p.zeros.data_ptr(), y.data_ptr(), ffi.DTYPE_F32, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    _close(y, ref, "unaligned")
    assert buf[0].item() == -7.0, "wrote before the output"


@pytest.mark.parametrize("kernel", ["0", "1"])
@pytest.mark.parametrize("fmt", ["int4", "int8", "q4_0", "q8_0"])
@pytest.mark.parametrize("m,n,k", [(130, 300, 128), (129, 64, 28672)])
def test_prefill_k_extremes(cuda, monkeypatch, kernel, fmt, m, n, k):
    """K of one 128-wide block (every step of the one-MFMA kernel is a tail step) and K =
    28672 (224 blocks: many unrolled steady groups, then the tail), INT4 g128 / INT8 / GGUF
    Q4_0 / Q8_0 on both prefill kernels, against the oracle at the north-star bound."""
    _i4_kernel(monkeypatch, kernel)
    print(f"[prefill k extremes] kernel={kernel} {fmt} m={m} n={n} k={k}", flush=True)
    xb, x = _x(97, m, k, cuda)
    xf = O.bf16_bits_to_f32(xb.reshape(m, k))
    if fmt == "int4":
        w = synth.weight(98, 1, n, k)
        p, (c, s, z) = _int4(w, 128, cuda)
        y = ops.gemm_w4a16(x, p, torch.float32)
        ref = O.gemm_w4a16(xb, c, s, z, n, k, 128)
    elif fmt == "int8":
        w = synth.weight(98, 1, n, k)
        q, sc = ops.quantize_int8(torch.from_numpy(w).to(cuda), 8, "channel", "half_even")
        y = ops.gemm_w8a16(x, q, sc, "channel", torch.float32)
        ref = O.gemm_w8a16(xb, q.cpu().numpy(), sc.cpu().numpy())
    else:
        ty, bb = (2, 18) if fmt == "q4_0" else (8, 34)
        rng = np.random.default_rng(99)
        raw = rng.integers(0, 256, (n * k // 32, bb), dtype=np.uint8)
        raw[:, 0:2] = (rng.standard_normal(n * k // 32) * 0.003).astype(np.float16).view(np.uint8).reshape(-1, 2)
        raw = raw.reshape(-1)
        p = ops.gguf_repack(ty, torch.from_numpy(raw).to(cuda), n, k)
        y = ops.gemm_gguf(x, p, torch.float32)
        ref = O.matmul_2d(xf, O.gguf_decode(ty, raw, n * k).reshape(n, k), packed_rhs=True)
    torch.cuda.synchronize()
    _close(y, ref, f"{fmt} k={k}")


@pytest.mark.parametrize("kernel", ["0", "1"])
def test_w4a16_prefill_special_scales(cuda, monkeypatch, kernel):
    """Group scales that are f16 subnormals, zero and the largest finite f16 give the
    oracle's outputs (each is exact in f32 and multiplies an exact partial); a row with one
    +Inf scale gives non-finite outputs in its column, as the evaluator's Inf weights do."""
    _i4_kernel(monkeypatch, kernel)
    m, n, k = 150, 300, 1024
    w = synth.weight(95, 1, n, k)
    codes, scales, zeros = O.quantize_int4g(w, 128)
    sv = scales.view(np.uint16).copy()
    sv[3, :4] = [0x0001, 0x03FF, 0x0000, 0x7BFF]  # subnormals, zero, 65504
    sv[7, 2] = 0x7C00                               # +Inf
    p = ops.Int4Packed(torch.from_numpy(codes.view(np.int32)).to(cuda), torch.from_numpy(sv.view(np.float16)).to(cuda),
                       torch.from_numpy(zeros.view(np.int32)).to(cuda), n, k, 128)
    xb, x = _x(96, m, k, cuda)
    y = ops.gemm_w4a16(x, p, torch.float32).cpu().numpy()
    assert not np.isfinite(y[:, 7]).any()
    ok = np.ones(n, bool)
    ok[7] = False
    ref = O.gemm_w4a16(xb, codes, sv, zeros, n, k, 128)
    _close(y[:, ok], ref[:, ok], "special scales")


def test_prefill_k_not_multiple_of_32_uses_exact_fallback(cuda):
    m, n, k = 33, 40, 1000
    w = synth.weight(91, 1, n, k)
    p = ops.quantize_int4g(torch.from_numpy(w).to(cuda), 8)
    xb, x = _x(92, m, k, cuda)
    y = ops.gemm_w4a16(x, p, torch.float32)
    ref = O.gemm_w4a16(xb, p.codes.cpu().numpy().view(np.uint32), p.scales.cpu().numpy().view(np.uint16),
                       p.zeros.cpu().numpy().view(np.uint32), n, k, 8)
    _close(y, ref, "fallback")


@pytest.mark.parametrize("name,n,k", [("w_gate", 11008, 4096), ("w_down", 4096, 11008)])
def test_w4a16_prefill_baseline_m4096_sampled(cuda, name, n, k):
    """BASELINE config 5 follow-on: W4A16 prefill at M = 4096 on 7B shapes, outputs sampled."""
    m = 4096
    print(f"[prefill w4a16 M=4096] {name}", flush=True)
    w = synth.weight(0, 4 if name == "w_gate" else 6, n, k)
    p, (c, s, z) = _int4(w, 128, cuda)
    xb, x = _x(93, m, k, cuda)
    y = ops.gemm_w4a16(x, p, torch.bfloat16)
    torch.cuda.synchronize()
    rng = np.random.default_rng(5)
    rows = np.sort(rng.choice(m, 24, replace=False))
    cols = np.sort(rng.choice(n, 48, replace=False))
    ref = O.gemm_w4a16(np.ascontiguousarray(xb[rows]), np.ascontiguousarray(c[cols]),
                       np.ascontiguousarray(s[cols]), np.ascontiguousarray(z[cols]), len(cols), k, 128)
    _close(y.float().cpu().numpy()[np.ix_(rows, cols)], ref, name)


def test_nf4_prefill_baseline_m512_sampled(cuda):
    """NF4 b64 GEMM at M = 512 on W_gate's shape, outputs sampled."""
    m, n, k = 512, 11008, 4096
    w = synth.weight(0, 4, n, k)
    xb, x = _x(94, m, k, cuda)
    p = ops.quantize_nf4(torch.from_numpy(w).to(cuda), 64)
    y = ops.gemm_nf4(x, p, torch.bfloat16)
    torch.cuda.synchronize()
    rng = np.random.default_rng(6)
    rows = np.sort(rng.choice(m, 32, replace=False))
    cols = np.sort(rng.choice(n, 64, replace=False))
    codes = p.codes.cpu().numpy().view(np.uint32)[cols]
    am = p.absmax.cpu().numpy()[cols]
    ref = O.gemm_nf4(np.ascontiguousarray(xb[rows]), np.ascontiguousarray(codes), np.ascontiguousarray(am),
                     len(cols), k, 64)
    _close(y.float().cpu().numpy()[np.ix_(rows, cols)], ref, "nf4 m512")
