"""Seeded synthetic inputs for the BASELINE workloads (no checkpoints or datasets exist here).

Host-side generation (numpy PCG64 keyed by (seed, tensor id)) gives identical bytes to the
CPU oracle and the GPU; device-side generation (torch on the GPU) is used only where the
bytes need not match a CPU run (bench timing at full size).
"""
from __future__ import annotations

import numpy as np

# One LLaMA-7B decoder block, weights stored [N, K] (out_features, in_features).
LLAMA7B_BLOCK = (
    ("wq", 4096, 4096),
    ("wk", 4096, 4096),
    ("wv", 4096, 4096),
    ("wo", 4096, 4096),
    ("w_gate", 11008, 4096),
    ("w_up", 11008, 4096),
    ("w_down", 4096, 11008),
)


def rng(seed: int, tensor_id: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([seed, tensor_id]))


def weight(seed: int, tensor_id: int, n: int, k: int, std: float = 0.02) -> np.ndarray:
    """f32 [n, k] ~ N(0, std^2)."""
    w = rng(seed, tensor_id).standard_normal((n, k), dtype=np.float32)
    w *= np.float32(std)
    return w


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def activations_bf16(seed: int, tensor_id: int, m: int, k: int, outlier_frac: float = 0.01,
                     outlier_scale: float = 20.0) -> np.ndarray:
    """bf16 bit patterns [m, k] ~ N(0, 1) with `outlier_frac` of the K channels scaled."""
    g = rng(seed, tensor_id)
    x = g.standard_normal((m, k), dtype=np.float32)
    n_out = int(round(outlier_frac * k))
    if n_out:
        ch = g.choice(k, size=n_out, replace=False)
        x[:, ch] *= np.float32(outlier_scale)
    return f32_to_bf16_bits(x)


def fp8_inputs(seed: int, tensor_id: int, rows: int, cols: int, outlier_frac: float = 0.005,
               outlier_scale: float = 30.0) -> np.ndarray:
    """f32 [rows, cols] ~ N(0, 1) with `outlier_frac` of the elements scaled (FP8 W8A8 config)."""
    g = rng(seed, tensor_id)
    x = g.standard_normal((rows, cols), dtype=np.float32)
    n_out = int(round(outlier_frac * x.size))
    if n_out:
        idx = g.choice(x.size, size=n_out, replace=False)
        x.reshape(-1)[idx] *= np.float32(outlier_scale)
    return x


def awq_channel_scales(seed: int, tensor_id: int, k: int) -> np.ndarray:
    """s = a^0.5 per input channel with a ~ LogNormal(0, 1), computed on the
    host in f64 and rounded once to f32 (the device never recomputes the transcendental)."""
    a = rng(seed, tensor_id).lognormal(0.0, 1.0, size=k)
    return np.sqrt(a).astype(np.float32)
