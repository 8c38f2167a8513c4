"""Benchmark of the quantized-weight hot path on one MI355X.

Headline (`value`): W4A16 dequant-fused GEMV at M=1 over one LLaMA-7B decoder block quantized
INT4 asymmetric g128.  One step = one launch that multiplies the block's 7
projections (Wq/Wk/Wv/Wo 4096x4096, W_gate/W_up 11008x4096, W_down 4096x11008) by bf16
activations.  Steps rotate over `--copies` distinct copies of the packed block so the working
set (16 x 105 MB) exceeds the 256 MB MALL and every step streams from HBM.

Also reported (`components`): quantize GB/s (INT4 g128 and INT8 per-channel over the f32
block), W4A16 GEMV at M=4/8 over the GEMV planes and at M=8/16 over the canonical layout,
W8A16 GEMV at M=1 (config 1), NF4 GEMV at M=1 and NF4 GEMM at M=64/512 (config 3), W4A16 prefill GEMM at M=4096 (config 5), FP8 W8A8 GEMM (config 4), and
the 32-layer AWQ-style INT4 model (config 5): quantize, decode GEMV and prefill GEMM over all
layers; also W8A16 and GGUF Q4_0 / Q8_0 prefill at M=4096 on the W_gate / W_down shapes.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E
METRIC = "quantize GB/s; W4A16 GEMV GB/s (%HBM peak) at M=1; FP8 GEMM TFLOPS at M=4096"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-model", action="store_true",
                    help="skip the 32-layer (25.9 GB f32) AWQ quantize / decode / prefill components")
    ap.add_argument("--only-headline", action="store_true",
                    help="time only the headline kernel (for profiler runs)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain elementwise copy (torch.neg, 1 GiB in, 1 GiB out) so that "
                         "FETCH_SIZE / WRITE_SIZE counter readings can be scaled to bytes")
    return ap.parse_args()


def model_32_layers(args, dev, gen, torch, synth, ops, log, time_steps, ev):
    """BASELINE config 5 over all 32 layers; returns the component figures."""
    out = {}
    layers = 32
    t0 = time.time()
    f32_layers, scales = [], []
    for li in range(layers):
        ws = []
        for tid, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK):
            ws.append(torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32) * 0.02)
        f32_layers.append(ws)
        scales.append([torch.from_numpy(synth.awq_channel_scales(0, 1000 + li * 7 + tid, k)).to(dev)
                       for tid, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK)])
    torch.cuda.synchronize()
    log(f"[bench] 32-layer f32 weight set generated in {time.time() - t0:.1f}s")

    packed = [[None] * 7 for _ in range(layers)]

    def quantize_all():
        # one batched AWQ launch per layer and column count (6 matrices of K = 4096, W_down)
        for li in range(layers):
            packed[li] = ops.quantize_int4g_batched(f32_layers[li], 128, scales[li])

    quantize_all()  # warm-up (and the packed set the GEMMs below use)
    torch.cuda.synchronize()
    s, e = ev(), ev()
    s.record()
    quantize_all()
    e.record()
    e.synchronize()
    ms_q = s.elapsed_time(e)
    q_bytes = 0
    for (_, n, k) in synth.LLAMA7B_BLOCK:
        g = (k + 127) // 128
        q_bytes += n * k * 4 + k * 4 + n * k // 2 + n * ((g + 7) // 8 * 8) * 2 + n * ((g + 7) // 8) * 4
    q_bytes *= layers
    out["model32_awq_int4g128_quantize_GBps"] = round(q_bytes / (ms_q * 1e-3) / 1e9, 1)
    out["model32_awq_int4g128_quantize_ms"] = round(ms_q, 3)
    log(f"[bench] 32-layer AWQ INT4 quantize: {ms_q:.2f} ms, {out['model32_awq_int4g128_quantize_GBps']} GB/s")
    del f32_layers
    torch.cuda.empty_cache()

    # decode: one batched 7-projection launch per layer, 32 launches in one graph, over the
    # GEMV planes (converted once at load time) and, for comparison, the canonical layout
    xs1 = {k: torch.randn((1, k), generator=gen, device=dev).to(torch.bfloat16) for k in (4096, 11008)}
    ys1 = [torch.empty((1, n), dtype=torch.bfloat16, device=dev) for (_, n, k) in synth.LLAMA7B_BLOCK]
    planes = [[ops.int4g_to_planes(p) for p in layer] for layer in packed]
    xs_l = [xs1[k] for (_, n, k) in synth.LLAMA7B_BLOCK]

    def decode(i):
        for li in range(layers):
            ops.gemv_w4a16_planes_batched(xs_l, planes[li], ys1)

    def decode_canonical(i):
        for li in range(layers):
            ops.gemv_w4a16_batched(xs_l, packed[li], ys1)

    ms_d = time_steps(decode, 20, 3, min_ms=50.0, replays=5)
    # compulsory bytes over the planes: codes, one f16 scale and one u4 zero point per row and
    # group, x and y (bf16)
    pb = sum(n * k // 2 + n * (k // 128) * 2 + n * (k // 128) // 2 + 2 * k + 2 * n
             for (_, n, k) in synth.LLAMA7B_BLOCK) * layers
    out["model32_decode_m1_GBps"] = round(pb / (ms_d * 1e-3) / 1e9, 1)
    out["model32_decode_m1_ms"] = round(ms_d, 4)
    log(f"[bench] 32-layer decode M=1 (planes): {ms_d * 1e3:.1f} us, {out['model32_decode_m1_GBps']} GB/s")
    ms_c = time_steps(decode_canonical, 20, 3, min_ms=50.0, replays=5)
    d_bytes = 0
    for (_, n, k) in synth.LLAMA7B_BLOCK:
        g = (k + 127) // 128
        d_bytes += n * k // 2 + n * ((g + 7) // 8 * 8) * 2 + n * ((g + 7) // 8) * 4 + 2 * k + 2 * n
    d_bytes *= layers
    out["model32_decode_m1_canonical_GBps"] = round(d_bytes / (ms_c * 1e-3) / 1e9, 1)
    log(f"[bench] 32-layer decode M=1 (canonical layout): {ms_c * 1e3:.1f} us, "
        f"{out['model32_decode_m1_canonical_GBps']} GB/s")
    del planes

    # prefill M=4096 over every projection of every layer
    m = 4096
    xs = {k: torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16) for k in (4096, 11008)}
    ys = {n: torch.empty((m, n), dtype=torch.bfloat16, device=dev) for n in (4096, 11008)}

    def prefill():
        for li in range(layers):
            for j, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK):
                p = packed[li][j]
                ops.ffi.call("castforge_hip_gemv_w4a16", xs[k].data_ptr(), m, n, k, 128, p.codes.data_ptr(),
                             p.scales.data_ptr(), p.zeros.data_ptr(), ys[n].data_ptr(), ops.ffi.DTYPE_BF16,
                             torch.cuda.current_stream().cuda_stream)

    prefill()
    torch.cuda.synchronize()
    s, e = ev(), ev()
    s.record()
    prefill()
    e.record()
    e.synchronize()
    ms_p = s.elapsed_time(e)
    flops = 2.0 * m * sum(n * k for (_, n, k) in synth.LLAMA7B_BLOCK) * layers
    out["model32_prefill_m4096_TFLOPs"] = round(flops / (ms_p * 1e-3) / 1e12, 1)
    out["model32_prefill_m4096_ms"] = round(ms_p, 2)
    log(f"[bench] 32-layer prefill M=4096: {ms_p:.1f} ms, {out['model32_prefill_m4096_TFLOPs']} TFLOP/s")
    del packed, xs, ys
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the quantized "
              "GEMV/GEMM would shard by output rows, each GPU holding its rows' codes and "
              "scales, with no collective at M = 1). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from castforge_amd import ffi, ops, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ffi.lib()
    log(f"[bench] {ffi.version()} on {torch.cuda.get_device_name(dev)}")

    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    def ev():
        return torch.cuda.Event(enable_timing=True)

    def time_steps(fn, steps, warmup, min_ms=20.0, replays=3, stream=None):
        """Milliseconds per step.  `warmup` eager calls of fn(i), then `steps` calls captured
        into one HIP graph (fn enqueues on torch's current stream, which is the capture stream
        during capture), replayed once untimed (graph upload), then replayed at least
        `replays` times and for at least `min_ms` in total, each replay between two events
        on the capture stream; the median replay gives the time per step.  The graph keeps
        Python/ctypes launch cost off the clock, so the time is the GPU's: kernel durations
        plus the gaps between back-to-back launches."""
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, capture_error_mode="thread_local"):
            for i in range(steps):
                fn(i)
        g.replay()
        torch.cuda.synchronize()
        times, total = [], 0.0
        while len(times) < replays or total < min_ms:
            s, e = ev(), ev()
            s.record()
            g.replay()
            e.record()
            e.synchronize()
            t = s.elapsed_time(e)
            times.append(t)
            total += t
        torch.cuda.synchronize()
        del g
        times.sort()
        time_steps.last = {"replays": len(times), "timed_ms": round(total, 2),
                           "min_us": round(times[0] / steps * 1e3, 2), "max_us": round(times[-1] / steps * 1e3, 2)}
        return times[len(times) // 2] / steps

    # ---------------------------------------------------------------- block weights ----
    t0 = time.time()
    block_f32 = []
    for tid, (name, n, k) in enumerate(synth.LLAMA7B_BLOCK):
        block_f32.append(torch.randn((n, k), generator=gen, device=dev, dtype=torch.float32) * 0.02)
    packed0 = [ops.quantize_int4g(w, 128) for w in block_f32]
    torch.cuda.synchronize()
    log(f"[bench] generated + quantized block in {time.time() - t0:.1f}s")

    # activations: bf16 N(0,1) with 1% of K channels x20 (host-generated, seeded)
    def x_for(m, k, tid):
        xb = synth.activations_bf16(0, 100 + tid, m, k)
        return torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(dev)

    def w4_bytes(m):
        tot = 0
        for (_, n, k) in synth.LLAMA7B_BLOCK:
            g = (k + 127) // 128
            tot += n * k // 2 + n * ((g + 7) // 8 * 8) * 2 + n * ((g + 7) // 8) * 4 + 2 * m * k + 2 * m * n
        return tot

    def planes_bytes(m=1):
        """Compulsory bytes of one step over GEMV planes: codes, one f16 scale and one u4 zero
        point per row and group (once, whatever M), x and y (bf16, M rows)."""
        return sum(n * k // 2 + n * (k // 128) * 2 + n * (k // 128) // 2 + 2 * m * k + 2 * m * n
                   for (_, n, k) in synth.LLAMA7B_BLOCK)

    copies = [packed0] + [[ops.Int4Packed(p.codes.clone(), p.scales.clone(), p.zeros.clone(),
                                          p.n, p.k, p.group) for p in packed0]
                          for _ in range(args.copies - 1)]
    # the GEMV planes of every copy, built once as a loader would
    planes = [[ops.int4g_to_planes(p) for p in c] for c in copies]
    torch.cuda.synchronize()

    def gemv_case(m):
        xs = [x_for(m, k, tid) for tid, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK)]
        ys = [torch.empty((m, n), dtype=torch.bfloat16, device=dev) for (_, n, k) in synth.LLAMA7B_BLOCK]
        return lambda i: ops.gemv_w4a16_batched(xs, copies[i % len(copies)], ys)

    def planes_case(m=1):
        # a decoder's activations: q/k/v share one x, gate/up another
        xk = {tid: x_for(m, k, tid) for tid, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK)}
        xs = [xk[0], xk[0], xk[0], xk[3], xk[4], xk[4], xk[6]]
        ys = [torch.empty((m, n), dtype=torch.bfloat16, device=dev) for (_, n, k) in synth.LLAMA7B_BLOCK]
        return lambda i: ops.gemv_w4a16_planes_batched(xs, planes[i % len(planes)], ys)

    components = {}
    ms_step = time_steps(planes_case(), args.steps, args.warmup, min_ms=50.0, replays=5)
    timing = dict(time_steps.last)
    bytes_m1 = planes_bytes()
    value = bytes_m1 / (ms_step * 1e-3) / 1e9
    # one step is one launch, so the average launch duration over the timed region (kernel
    # plus the inter-launch gap) is ms_step and roofline.achieved equals value
    achieved = value
    log(f"[bench] W4A16 GEMV M=1 (planes): {ms_step * 1e3:.2f} us/step (one launch), {value:.0f} GB/s; "
        f"median of {timing['replays']} replays ({timing['timed_ms']} ms), "
        f"{timing['min_us']}..{timing['max_us']} us")
    st = time_steps(gemv_case(1), args.steps, 5, min_ms=20.0, replays=3)
    components["w4a16_gemv_m1_canonical_GBps"] = round(w4_bytes(1) / (st * 1e-3) / 1e9, 1)
    log(f"[bench] W4A16 GEMV M=1 (canonical layout): {st * 1e3:.2f} us/step, "
        f"{components['w4a16_gemv_m1_canonical_GBps']} GB/s")

    if args.copy_calibration:
        # a copy of known size: 2^28 f32 read + 2^28 f32 written per launch
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        log("[bench] copy calibration: 5 launches of neg over 1 GiB")
        del src, dst

    if not args.only_headline:
        # small-batch decode over the planes (M = 2..16, every matrix's planes streamed once)
        for m in (4, 8, 16):
            st = time_steps(planes_case(m), max(20, args.steps // 4), 5, min_ms=20.0, replays=3)
            components[f"w4a16_planes_gemv_m{m}_GBps"] = round(planes_bytes(m) / (st * 1e-3) / 1e9, 1)
            components[f"w4a16_planes_gemv_m{m}_us"] = round(st * 1e3, 2)
            log(f"[bench] W4A16 GEMV M={m} (planes): {st * 1e3:.1f} us/step "
                f"{components[f'w4a16_planes_gemv_m{m}_GBps']} GB/s")
        for m in (8, 16):
            st = time_steps(gemv_case(m), max(20, args.steps // 4), 5, min_ms=20.0, replays=3)
            components[f"w4a16_gemv_m{m}_GBps"] = round(w4_bytes(m) / (st * 1e-3) / 1e9, 1)
            log(f"[bench] W4A16 GEMV M={m} (canonical layout): {st * 1e3:.1f} us/step "
                f"{components[f'w4a16_gemv_m{m}_GBps']} GB/s")

        # quantize over the f32 block (809 MB in, > MALL)
        nel = sum(n * k for (_, n, k) in synth.LLAMA7B_BLOCK)
        nrows = sum(n for (_, n, k) in synth.LLAMA7B_BLOCK)
        # the batched entry points: one launch per column count over the block (the same codes
        # as one call per matrix)
        st = time_steps(lambda i: ops.quantize_int4g_batched(block_f32, 128), 10, 2)
        q4_bytes = nel * 4 + nel // 2 + sum(n * (((k + 127) // 128 + 7) // 8) * (16 + 4)
                                            for (_, n, k) in synth.LLAMA7B_BLOCK)
        components["quantize_int4g128_GBps"] = round(q4_bytes / (st * 1e-3) / 1e9, 1)
        st = time_steps(lambda i: ops.quantize_int8_batched(block_f32, 8, "half_even"), 10, 2)
        components["quantize_int8_channel_GBps"] = round((nel * 5 + nrows * 4) / (st * 1e-3) / 1e9, 1)
        log(f"[bench] quantize int4g {components['quantize_int4g128_GBps']} GB/s, "
            f"int8 {components['quantize_int8_channel_GBps']} GB/s")
        # QuaRot-style K-axis Hadamard (block 128) fused into the INT4 g128 quantizer (same
        # bytes as plain quantize: the rotated f32 tensor is never written), and the rotation
        # alone along K (f32 read + write)
        st = time_steps(lambda i: [ops.quantize_int4g_hadamard(w, 128, 128) for w in block_f32], 10, 2)
        components["quantize_int4g128_hadamard128_GBps"] = round(q4_bytes / (st * 1e-3) / 1e9, 1)
        st = time_steps(lambda i: [ops.rotate_hadamard(w, 128, 1) for w in block_f32], 10, 2)
        components["rotate_hadamard128_GBps"] = round(8 * nel / (st * 1e-3) / 1e9, 1)
        log(f"[bench] hadamard128+int4g {components['quantize_int4g128_hadamard128_GBps']} GB/s, "
            f"rotation {components['rotate_hadamard128_GBps']} GB/s")

        # W8A16 GEMV M=1 over rotating copies of the INT8 block (config 1)
        q8 = [ops.quantize_int8(w, 8, "channel", "half_even") for w in block_f32]
        q8c = [q8] + [[(q.clone(), s.clone()) for q, s in q8] for _ in range(7)]
        xs8 = [x_for(1, k, tid) for tid, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK)]
        ys8 = [torch.empty((1, n), dtype=torch.bfloat16, device=dev) for (_, n, k) in synth.LLAMA7B_BLOCK]

        def w8_step(i):  # the 7 projections in one launch, like the W4A16 headline
            ops.gemv_w8a16_batched(xs8, q8c[i % len(q8c)], ys8, "channel")
        st = time_steps(w8_step, 50, 5)
        w8_bytes = nel + nrows * 4 + sum(2 * k + 2 * n for (_, n, k) in synth.LLAMA7B_BLOCK)
        components["w8a16_gemv_m1_GBps"] = round(w8_bytes / (st * 1e-3) / 1e9, 1)
        # INT8 prefill at M = 4096 on W_gate / W_down (one-MFMA kernel at these shapes)
        for idx in (4, 6):
            _, n, k = synth.LLAMA7B_BLOCK[idx]
            m = 4096
            xp = torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
            qi, si = q8[idx]
            st = time_steps(lambda i: ops.gemm_w8a16(xp, qi, si, "channel", torch.bfloat16), 10, 2, min_ms=30.0,
                            replays=3)
            components[f"w8a16_prefill_m{m}_n{n}_k{k}_TFLOPs"] = round(2.0 * m * n * k / (st * 1e-3) / 1e12, 1)
            log(f"[bench] W8A16 prefill M={m} n={n} k={k}: {st * 1e3:.1f} us, "
                f"{components[f'w8a16_prefill_m{m}_n{n}_k{k}_TFLOPs']} TFLOP/s")
            del xp
        del q8, q8c

        # NF4 b64 GEMV M=1 over W_gate/W_up/W_down (config 3)
        nf = [ops.quantize_nf4(w, 64) for w in block_f32[4:]]
        nfc = [nf] + [[ops.Nf4Packed(p.codes.clone(), p.absmax.clone(), p.n, p.k, p.block) for p in nf]
                      for _ in range(15)]
        xsn = [x_for(1, p.k, 4 + j) for j, p in enumerate(nf)]
        ysn = [torch.empty((1, p.n), dtype=torch.bfloat16, device=dev) for p in nf]

        def nf_step(i):  # W_gate / W_up / W_down in one launch
            ops.gemv_nf4_batched(xsn, nfc[i % len(nfc)], ysn)
        st = time_steps(nf_step, 50, 5)
        nf_bytes = sum(p.nbytes() + 2 * p.k + 2 * p.n for p in nf)
        components["nf4_gemv_m1_GBps"] = round(nf_bytes / (st * 1e-3) / 1e9, 1)
        # the same launch over NF4 planes (castforge_hip_gemv_nf4_planes_batched); the same
        # algorithmic bytes (the canonical codes, absmax, x and y)
        nfp = [[ops.nf4_to_planes(p) for p in c] for c in nfc]
        st = time_steps(lambda i: ops.gemv_nf4_planes_batched(xsn, nfp[i % len(nfp)], ysn), 50, 5)
        components["nf4_planes_gemv_m1_GBps"] = round(nf_bytes / (st * 1e-3) / 1e9, 1)
        log(f"[bench] W8A16 M=1 {components['w8a16_gemv_m1_GBps']} GB/s, NF4 M=1 {components['nf4_gemv_m1_GBps']} GB/s "
            f"(planes {components['nf4_planes_gemv_m1_GBps']} GB/s)")
        del nf, nfc, nfp

        # GGUF Q4_0 / Q8_0 GEMV M=1 over the block (gguf.rs block formats, GEMV planes), seeded
        # random blocks with f16 d ~ N(0, 0.003); rotating copies keep the set above the MALL
        for ty, bb, tag, ncopy in ((2, 18, "q4_0", 8), (8, 34, "q8_0", 4)):
            gc = []
            for c in range(ncopy):
                gg = torch.Generator(device=dev)
                gg.manual_seed(1000 * ty + c)
                row = []
                for (_, n, k) in synth.LLAMA7B_BLOCK:
                    raw = torch.randint(0, 256, (n * k // 32 * bb,), dtype=torch.uint8, device=dev, generator=gg)
                    d = (torch.randn(n * k // 32, device=dev, generator=gg) * 0.003).half()
                    raw.view(-1, bb)[:, 0:2] = d.view(torch.uint8).view(-1, 2)
                    row.append(ops.gguf_repack(ty, raw, n, k))
                    del raw, d
                gc.append(row)
            ysg = [torch.empty((1, n), dtype=torch.bfloat16, device=dev) for (_, n, k) in synth.LLAMA7B_BLOCK]
            st = time_steps(lambda i: ops.gemv_gguf_batched(xs8, gc[i % len(gc)], ysg), 50, 5)
            gb = sum(p.nbytes() + 2 * p.k + 2 * p.n for p in gc[0])
            components[f"gguf_{tag}_gemv_m1_GBps"] = round(gb / (st * 1e-3) / 1e9, 1)
            log(f"[bench] GGUF {tag} GEMV M=1: {st * 1e3:.1f} us, {components[f'gguf_{tag}_gemv_m1_GBps']} GB/s")
            if ty == 2:  # the same launch over Q4_0 GEMV planes (same algorithmic bytes)
                gpl = [[ops.gguf_q4_0_to_gemv_planes(p) for p in row] for row in gc]
                st = time_steps(lambda i: ops.gemv_gguf_q4_0_planes_batched(xs8, gpl[i % len(gpl)], ysg), 50, 5)
                components["gguf_q4_0_planes_gemv_m1_GBps"] = round(gb / (st * 1e-3) / 1e9, 1)
                log(f"[bench] GGUF q4_0 GEMV M=1 over Q4_0 GEMV planes: {st * 1e3:.1f} us, "
                    f"{components['gguf_q4_0_planes_gemv_m1_GBps']} GB/s")
                del gpl
            # prefill at M = 4096 on W_gate / W_down over the same planes
            for idx in (4, 6):
                _, n, k = synth.LLAMA7B_BLOCK[idx]
                m = 4096
                xp = torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
                pg = gc[0][idx]
                st = time_steps(lambda i: ops.gemm_gguf(xp, pg, torch.bfloat16), 10, 2, min_ms=30.0, replays=3)
                components[f"gguf_{tag}_prefill_m{m}_n{n}_k{k}_TFLOPs"] = round(2.0 * m * n * k / (st * 1e-3) / 1e12, 1)
                log(f"[bench] GGUF {tag} prefill M={m} n={n} k={k}: {st * 1e3:.1f} us, "
                    f"{components[f'gguf_{tag}_prefill_m{m}_n{n}_k{k}_TFLOPs']} TFLOP/s")
                del xp
            del gc, ysg

        # prefill GEMMs on MFMA: W4A16 INT4 g128 at M=4096 (config 5 follow-on) and NF4 b64 at
        # M=64 / 512 over W_gate / W_up / W_down (config 3)
        for (name, n, k) in (synth.LLAMA7B_BLOCK[4], synth.LLAMA7B_BLOCK[6]):
            m = 4096
            xp = torch.randn((m, k), generator=gen, device=dev).to(torch.bfloat16)
            pp = packed0[4 if name == "w_gate" else 6]
            yp = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
            st = time_steps(lambda i: ops.gemm_w4a16(xp, pp, torch.bfloat16), 10, 2, min_ms=30.0, replays=3)
            components[f"w4a16_prefill_m{m}_n{n}_k{k}_TFLOPs"] = round(2.0 * m * n * k / (st * 1e-3) / 1e12, 1)
            log(f"[bench] W4A16 prefill M={m} {name}: {st * 1e3:.1f} us, "
                f"{components[f'w4a16_prefill_m{m}_n{n}_k{k}_TFLOPs']} TFLOP/s")
            del xp, yp
        nf3 = [ops.quantize_nf4(w, 64) for w in block_f32[4:]]
        # M = 64: one launch over the three matrices on the skinny kernel, rotating over 4 copies
        # of the weights (270 MB, beyond the 256 MB MALL); M = 512: one prefill GEMM per matrix
        nf3c = [nf3] + [[ops.Nf4Packed(p.codes.clone(), p.absmax.clone(), p.n, p.k, p.block) for p in nf3]
                        for _ in range(3)]
        for m in (64, 512):
            xs3 = [torch.randn((m, p.k), generator=gen, device=dev).to(torch.bfloat16) for p in nf3]
            if m == 64:
                ys3 = [torch.empty((m, p.n), dtype=torch.bfloat16, device=dev) for p in nf3]
                st = time_steps(lambda i: ops.gemv_nf4_batched(xs3, nf3c[i % len(nf3c)], ys3), 20, 3)
            else:
                st = time_steps(lambda i: [ops.gemm_nf4(x, p, torch.bfloat16) for x, p in zip(xs3, nf3)], 10, 2)
            fl = sum(2.0 * m * p.n * p.k for p in nf3)
            by = sum(p.nbytes() + 2 * m * p.k + 2 * m * p.n for p in nf3)
            components[f"nf4_gemm_m{m}_TFLOPs"] = round(fl / (st * 1e-3) / 1e12, 1)
            components[f"nf4_gemm_m{m}_GBps"] = round(by / (st * 1e-3) / 1e9, 1)
            log(f"[bench] NF4 GEMM M={m} (Wg, Wu, Wd): {st * 1e3:.1f} us, "
                f"{components[f'nf4_gemm_m{m}_TFLOPs']} TFLOP/s, {components[f'nf4_gemm_m{m}_GBps']} GB/s")
        del nf3, nf3c

        # Config 5: a 32-layer LLaMA-7B-shaped f32 weight set (6.476 B linear params, 25.9 GB),
        # quantized end to end INT4 g128 with the AWQ-style per-input-channel pre-scale
        # s = a^0.5 fused into the quantize pass; then a W4A16 decode GEMV (M = 1) and a prefill
        # GEMM (M = 4096) over every layer.  3.4 GB of packed weights: no cache holds them.
        if not args.skip_model:
            components.update(model_32_layers(args, dev, gen, torch, synth, ops, log, time_steps, ev))

        # FP8 E4M3 W8A8 GEMM at M=4096 (config 4): N(0,1) inputs with 0.5% outliers x30
        for (m, n, k) in ((4096, 11008, 4096), (4096, 4096, 11008)):
            a = torch.randn((m, k), generator=gen, device=dev)
            a[torch.rand((m, k), generator=gen, device=dev) < 0.005] *= 30
            w = torch.randn((n, k), generator=gen, device=dev)
            w[torch.rand((n, k), generator=gen, device=dev) < 0.005] *= 30
            a16 = a.to(torch.bfloat16)
            del a
            qw, sw = ops.quantize_fp8(w)
            qa, sa = ops.quantize_fp8(a16)
            y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
            la = time_steps(lambda i: ops.gemm_fp8(qa, sa, qw, sw, y), 30, 3)
            tag = f"m{m}_n{n}_k{k}"
            components[f"fp8_gemm_{tag}_TFLOPs"] = round(2.0 * m * n * k / (la * 1e-3) / 1e12, 1)
            components[f"fp8_gemm_{tag}_pct_fp8_peak"] = round(100 * 2.0 * m * n * k / (la * 1e-3) / 5.0e15, 1)
            # the exact form (E4M3 widened to f16, f16 MFMA) that the evaluator dispatches to
            le = time_steps(lambda i: ops.gemm_fp8(qa, sa, qw, sw, y, exact=True), 20, 3)
            components[f"fp8_gemm_exact_{tag}_TFLOPs"] = round(2.0 * m * n * k / (le * 1e-3) / 1e12, 1)
            components[f"fp8_gemm_exact_{tag}_pct_f16_peak"] = round(100 * 2.0 * m * n * k / (le * 1e-3) / 2.5e15, 1)
            lq = time_steps(lambda i: ops.quantize_fp8(a16), 20, 3)
            components[f"fp8_act_quant_{tag}_GBps"] = round((m * k * 3 + m * 4) / (lq * 1e-3) / 1e9, 1)

            # the W8A8 step end to end: per-token E4M3 quantize of the bf16 activations, then
            # the GEMM on the fresh codes (weights quantized once, outside the step)
            def w8a8(i):
                qx, sx = ops.quantize_fp8(a16)
                ops.gemm_fp8(qx, sx, qw, sw, y)

            lw = time_steps(w8a8, 20, 3)
            components[f"fp8_w8a8_step_{tag}_us"] = round(lw * 1e3, 2)
            components[f"fp8_w8a8_step_{tag}_TFLOPs"] = round(2.0 * m * n * k / (lw * 1e-3) / 1e12, 1)
            log(f"[bench] FP8 GEMM {tag}: {la * 1e3:.1f} us, {components[f'fp8_gemm_{tag}_TFLOPs']} TFLOP/s "
                f"(exact form {le * 1e3:.1f} us, {components[f'fp8_gemm_exact_{tag}_TFLOPs']} TFLOP/s); "
                f"act quant {components[f'fp8_act_quant_{tag}_GBps']} GB/s; W8A8 step (quantize + GEMM) "
                f"{lw * 1e3:.1f} us, {components[f'fp8_w8a8_step_{tag}_TFLOPs']} TFLOP/s")
            del w, a16, qw, sw, qa, sa, y

    components["w4a16_gemv_m1_GBps"] = round(value, 1)
    components["w4a16_gemv_m1_pct_hbm_peak"] = round(100.0 * value / HBM_PEAK_GBPS, 1)

    # ---------------------------------------------------------------- CPU baseline ----
    cpu = None
    if not args.no_cpu_baseline:
        sys.path.insert(0, str(ROOT / "tests"))
        import oracle_lib as O

        host = [(p.codes.cpu().numpy().view(np.uint32), p.scales.cpu().numpy().view(np.uint16),
                 p.zeros.cpu().numpy().view(np.uint32), p.n, p.k) for p in packed0]
        xh = [synth.activations_bf16(0, 100 + tid, 1, k) for tid, (_, n, k) in enumerate(synth.LLAMA7B_BLOCK)]
        passes, t_cpu = 0, 0.0
        while t_cpu < 10.0 and passes < 8:
            t1 = time.perf_counter()
            for (c, s, z, n, k), x in zip(host, xh):
                O.gemm_w4a16(x, c, s, z, n, k, 128)
            t_cpu += time.perf_counter() - t1
            passes += 1
        cpu_model = "unknown"
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
        cpu = {"value": round(w4_bytes(1) * passes / t_cpu / 1e9, 3), "unit": "GB/s", "cores": 1,
               "kind": "port", "cpu_model": cpu_model, "host_cpus": os.cpu_count(),
               "sample": f"{passes} pass(es) of the full block W4A16 GEMV at M=1 with the oracle's "
                         f"evaluator semantics (dequantize to f32, then the m,n,k f32 loop of "
                         f"eval.rs:1465-1507), single thread, {t_cpu:.1f} s"}
        log(f"[bench] cpu baseline {cpu['value']} GB/s over {passes} passes ({t_cpu:.1f}s)")
        import ctypes
        cp = ctypes.c_void_p
        ptr = lambda a: a.ctypes.data_as(cp)
        xf = [np.ascontiguousarray(O.bf16_bits_to_f32(x).reshape(-1), dtype=np.float32) for x in xh]
        yf = [np.zeros(n, np.float32) for (_, n, k) in synth.LLAMA7B_BLOCK]
        # CPU-B, codegen-faithful: the loop nest the reference's Rust emitter writes for
        # fused_qmatmul (dequant inline in the k loop), built like its JIT (-O3, no -march,
        # no contraction), one thread (oracle/cpu_codegen.c)
        cpg = ctypes.CDLL(str(ROOT / "oracle" / "_build" / "libcf_cpucodegen.so"))
        cpg.cpcg_gemv_w4a16.argtypes = [cp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, cp, cp, cp, cp]
        passes_b, t_b = 0, 0.0
        while t_b < 6.0 and passes_b < 8:
            t1 = time.perf_counter()
            for (c, s_, z, n, k), x, y in zip(host, xf, yf):
                cpg.cpcg_gemv_w4a16(ptr(x), 1, n, k, ptr(c), ptr(s_), ptr(z), ptr(y))
            t_b += time.perf_counter() - t1
            passes_b += 1
        cpu["codegen_faithful"] = {
            "value": round(w4_bytes(1) * passes_b / t_b / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "CPU-B codegen-faithful (oracle/cpu_codegen.c)",
            "sample": f"{passes_b} pass(es) of the full block W4A16 GEMV at M=1 through the emitted "
                      f"loop nest of rust_composites.rs:176-244 (dequant inline, f32 accumulator, no "
                      f"FMA), gcc -O3 without -march, single thread, {t_b:.1f} s"}
        log(f"[bench] cpu codegen-faithful {cpu['codegen_faithful']['value']} GB/s over {passes_b} passes "
            f"({t_b:.1f}s)")
        # CPU-C, the best-effort host figure (blocked, SIMD, all visible cores; oracle/cpu_best.c):
        # reported beside the port, which stays the baseline
        cpub = ctypes.CDLL(str(ROOT / "oracle" / "_build" / "libcf_cpubest.so"))
        cpub.cpub_gemv_w4a16.argtypes = [cp, ctypes.c_int64, ctypes.c_int64, cp, cp, cp, cp, ctypes.c_int]
        ncpu = len(os.sched_getaffinity(0))
        # 6 rotating copies of the block (630 MB), more than a host's last-level cache, as the GPU
        # side rotates copies past the MALL
        hosts = [host] + [[(c.copy(), s_.copy(), z.copy(), n, k) for (c, s_, z, n, k) in host] for _ in range(5)]
        passes_c, t_c = 0, 0.0
        while t_c < 2.0 and passes_c < 5000:
            t1 = time.perf_counter()
            for (c, s_, z, n, k), x, y in zip(hosts[passes_c % len(hosts)], xf, yf):
                cpub.cpub_gemv_w4a16(ptr(x), n, k, ptr(c), ptr(s_), ptr(z), ptr(y), ncpu)
            t_c += time.perf_counter() - t1
            passes_c += 1
        del hosts
        cpu["best_effort"] = {"value": round(w4_bytes(1) * passes_c / t_c / 1e9, 2), "unit": "GB/s",
                              "cores": ncpu, "kind": "CPU-C best-effort (oracle/cpu_best.c)",
                              "sample": f"{passes_c} passes of the full block W4A16 GEMV at M=1 over 6 rotating "
                                        f"copies (630 MB), OpenMP over "
                                        f"{ncpu} threads, AVX2/FMA, group products in f32 lanes with the "
                                        f"zero point folded out, {t_c:.1f} s"}
        log(f"[bench] cpu best-effort {cpu['best_effort']['value']} GB/s on {ncpu} threads "
            f"over {passes_c} passes ({t_c:.1f}s)")

    traffic = None
    tfile = ROOT / "profiles" / "traffic_w4a16_planes_gemv_m1.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4xbf16",
        "data": "synthetic (N(0,0.02) weights, bf16 N(0,1) activations with 1% x20 channels)",
        "config": {"workload": "llama7b_block_int4g128_w4a16_gemv_m1", "m": 1, "group": 128,
                   "matrices": 7, "rotating_copies": len(copies),
                   "layout": "GEMV planes (built once at load)", "x_shared": "q/k/v and gate/up",
                   "value_is": "W4A16 GEMV GB/s at M=1 (algorithmic bytes / whole-job time per step)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": "planes_i8_kernel<16, 2>", "bytes_per_launch": bytes_m1,
                     "us_per_launch": round(ms_step * 1e3, 2), "timing": timing},
        "cpu_baseline": cpu,
        "components": components,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
