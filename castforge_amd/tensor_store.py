"""TensorStore: the weight plane beside the SSA graph (ir/tensor_store.rs:13-56, 214-348).

Entries map a name (the `dense_resource` key or the constant's SSA name) to a typed backing:
  F32Data          f32 values (tensor_store.rs:41)
  QuantizedI8      i8 codes + one f32 scale + i64 zero point (tensor_store.rs:44-48)
  QuantizedPacked  this library's packed low-bit weights (codes / scales / zeros of one of
                   the formats of include/castforge_hip.h) -- the reference has no slot for them
All data are device tensors.  `resolve_f32_attr` dequantizes on the GPU through the C ABI.
The store is shared copy-on-write between module clones (tensor_store.rs:214-233): entries
are replaced, never mutated, so a clone keeps seeing its own values.

Safetensors I/O keeps the reference's header convention (I8 + `scale` / `zero_point` keys,
tensor_store.rs:300-309, 478-497, 716-744) and stores packed formats as their component
tensors `<name>.codes / .scales / .zeros` plus a `castforge_packed` header entry.
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass
from typing import Any

import numpy as np
import torch

from .ir import Dense, QuantPacked, QuantUniform, TensorRef, TensorType


@dataclass
class F32Data:
    data: Any  # device f32 tensor


@dataclass
class QuantizedI8:
    data: Any  # device int8 tensor
    scale: float
    zero_point: int


@dataclass
class InMemory:
    """Raw bytes of a tensor whose dtype the loader does not decode (tensor_store.rs:22, kept
    as DType::U8 by load_safetensors, tensor_store.rs:736-744)."""
    data: Any  # uint8 tensor


@dataclass
class QuantizedPacked:
    """format: int8_channel | int4_asym | nf4 | fp8_row | gguf_q4_0 | gguf_q8_0; shape [N, K]
    (gguf_*: GGUF planes, codes + f16 scales, no zeros)."""
    format: str
    codes: Any
    scales: Any
    zeros: Any
    group: int
    shape: tuple


@dataclass
class TensorEntry:
    name: str
    ty: TensorType
    backing: Any


class TensorStore:
    def __init__(self):
        self._entries: dict[str, TensorEntry] = {}

    def clone(self) -> "TensorStore":
        s = TensorStore()
        s._entries = dict(self._entries)  # entries are replaced on write: shallow copy is CoW
        return s

    def insert(self, entry: TensorEntry) -> None:
        self._entries[entry.name] = entry

    def get(self, key: str) -> TensorEntry | None:
        return self._entries.get(key)

    def __len__(self) -> int:
        return len(self._entries)

    def items(self):
        return self._entries.items()

    # -- resolution (tensor_store.rs:314-348, 406-424) --------------------------------------
    def resolve_f32_attr(self, attr, expected_len: int):
        """Flat f32 device tensor of a constant's value, dequantizing quantized backings with
        the backing's own (exact) scale: (q - zero_point) * scale (tensor_store.rs:323-331)."""
        if isinstance(attr, Dense):
            t = attr.data
            return t.reshape(-1).float() if t.dtype != torch.float32 else t.reshape(-1)
        if not isinstance(attr, TensorRef):
            return None
        e = self.get(attr.key)
        if e is None:
            return None
        b = e.backing
        if isinstance(b, F32Data):
            return b.data.reshape(-1)
        if isinstance(b, QuantizedI8):
            from . import ops

            if b.zero_point != 0:
                raise NotImplementedError("QuantizedI8 with a non-zero zero_point has no HIP dequant path")
            scales = torch.tensor([b.scale], dtype=torch.float32, device=b.data.device)
            return ops.dequantize_int8(b.data.reshape(1, -1), scales, "tensor").reshape(-1)
        if isinstance(b, QuantizedPacked):
            return dequantize_packed(b).reshape(-1)
        return None

    def resolve_i8_attr(self, attr, expected_len: int):
        if isinstance(attr, TensorRef):
            e = self.get(attr.key)
            if e is not None and isinstance(e.backing, QuantizedI8):
                return e.backing.data
            return None
        if isinstance(attr, Dense):
            return attr.data if attr.data.dtype == torch.int8 else attr.data.to(torch.int8)
        return None

    def update_f32_constant(self, ssa_name: str | None, old_attr, new_ty: TensorType, new_vals):
        """tensor_store.rs:253-285: a TensorRef keeps its key and gets f32 data; an inline
        constant gets a new inline value (and a same-named store entry, if any, is updated)."""
        if isinstance(old_attr, TensorRef):
            if old_attr.key in self._entries:
                self.insert(TensorEntry(old_attr.key, new_ty, F32Data(new_vals)))
            return TensorRef(old_attr.key)
        if ssa_name is not None and ssa_name in self._entries:
            self.insert(TensorEntry(ssa_name, new_ty, F32Data(new_vals)))
        return Dense(new_vals.reshape(new_ty.shape))

    # -- safetensors --------------------------------------------------------------------------
    def to_safetensors_bytes(self) -> bytes:
        header: dict[str, Any] = {}
        blobs: list[bytes] = []
        off = 0

        def put(name, dtype, shape, data: bytes, extra=None):
            nonlocal off
            h = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(data)]}
            if extra:
                h.update(extra)
            header[name] = h
            blobs.append(data)
            off += len(data)

        packed_meta = {}
        for name, e in self._entries.items():
            b = e.backing
            shape = tuple(e.ty.shape)
            if isinstance(b, F32Data):
                vals = b.data.detach().contiguous().cpu().numpy().astype(np.float32, copy=False).ravel()
                if e.ty.dtype == "f16":  # tensor_store.rs:446-451: truncating f32_to_f16_bits
                    put(name, "F16", shape, f32_to_f16_bits_trunc(vals).tobytes())
                elif e.ty.dtype == "bf16":  # tensor_store.rs:452-457: bits >> 16
                    put(name, "BF16", shape, (vals.view(np.uint32) >> 16).astype(np.uint16).tobytes())
                else:
                    put(name, "F32", shape, vals.tobytes())
            elif isinstance(b, InMemory):
                put(name, "U8", shape, b.data.detach().contiguous().cpu().numpy().tobytes())
            elif isinstance(b, QuantizedI8):
                put(name, "I8", shape, b.data.detach().contiguous().cpu().numpy().tobytes(),
                    {"scale": float(b.scale), "zero_point": int(b.zero_point)})
            elif isinstance(b, QuantizedPacked):
                for part in ("codes", "scales", "zeros"):
                    t = getattr(b, part)
                    if t is None:
                        continue
                    dt = {torch.int32: "I32", torch.float16: "F16", torch.float32: "F32",
                          torch.int8: "I8", torch.uint8: "U8"}[t.dtype]
                    put(f"{name}.{part}", dt, tuple(t.shape), t.detach().contiguous().cpu().numpy().tobytes())
                packed_meta[name] = {"format": b.format, "group": b.group, "shape": list(b.shape),
                                     "expressed": "f32"}
        meta = {"castforge_packed": json.dumps(packed_meta, sort_keys=True)} if packed_meta else {}
        if meta:
            header["__metadata__"] = meta
        hb = json.dumps(header).encode()
        hb += b" " * ((8 - len(hb) % 8) % 8)
        return struct.pack("<Q", len(hb)) + hb + b"".join(blobs)

    def load_safetensors_bytes(self, raw: bytes, device) -> int:
        """tensor_store.rs:656-752: F32; F16 / BF16 decoded exactly to f32 values that keep
        their dtype; I8 with the `scale` / `zero_point` keys as QuantizedI8 (the type's scale
        string `{:.6}` with trailing zeros and dot trimmed); every other dtype kept as raw U8
        bytes.  Packed formats of this library come back from their component tensors."""
        (hlen,) = struct.unpack("<Q", raw[:8])
        header = json.loads(raw[8:8 + hlen].decode())
        base = 8 + hlen
        meta = json.loads(header.pop("__metadata__", {}).get("castforge_packed", "{}"))
        npd = {"F32": np.float32, "F16": np.uint16, "BF16": np.uint16, "I8": np.int8, "I32": np.int32,
               "U8": np.uint8}
        width = {"F32": 4, "F16": 2, "BF16": 2}
        parts: dict[str, Any] = {}
        loaded = 0
        for name, h in header.items():
            a, b = h["data_offsets"]
            blob = raw[base + a:base + b]
            shape = tuple(h["shape"])
            stem, _, part = name.rpartition(".")
            if stem in meta and part in ("codes", "scales", "zeros"):
                dt = np.float16 if h["dtype"] == "F16" else npd[h["dtype"]]
                parts.setdefault(stem, {})[part] = torch.from_numpy(
                    np.frombuffer(blob, dtype=dt).reshape(shape).copy()).to(device)
                continue
            dtype = h["dtype"]
            if dtype in width and len(blob) % width[dtype]:
                raise ValueError(f"{dtype} tensor `{name}` byte length {len(blob)} is not a multiple of "
                                 f"{width[dtype]}")
            if dtype == "F32":
                vals = np.frombuffer(blob, np.float32).copy()
                self.insert(TensorEntry(name, TensorType(shape, "f32"), F32Data(torch.from_numpy(vals).to(device))))
            elif dtype in ("F16", "BF16"):
                bits = np.frombuffer(blob, np.uint16)
                vals = f16_bits_to_f32(bits) if dtype == "F16" else (bits.astype(np.uint32) << 16).view(np.float32)
                self.insert(TensorEntry(name, TensorType(shape, dtype.lower()),
                                        F32Data(torch.from_numpy(vals.copy()).to(device))))
            elif dtype == "I8":
                t = torch.from_numpy(np.frombuffer(blob, np.int8).reshape(shape).copy()).to(device)
                scale = float(np.float32(h["scale"])) if h.get("scale") is not None else 1.0
                zp = int(h["zero_point"]) if h.get("zero_point") is not None else 0
                dt = QuantUniform("i8", "f32", loader_scale_string(scale), zp) if h.get("scale") is not None else "i8"
                self.insert(TensorEntry(name, TensorType(shape, dt), QuantizedI8(t, scale, zp)))
            else:
                t = torch.from_numpy(np.frombuffer(blob, np.uint8).copy()).to(device)
                self.insert(TensorEntry(name, TensorType(shape, "u8"), InMemory(t)))
            loaded += 1
        for stem, m in meta.items():
            p = parts.get(stem, {})
            ty = TensorType(tuple(m["shape"]), QuantPacked(m["format"], m.get("expressed", "f32"), m["group"]))
            self.insert(TensorEntry(stem, ty, QuantizedPacked(m["format"], p.get("codes"), p.get("scales"),
                                                              p.get("zeros"), m["group"], tuple(m["shape"]))))
            loaded += 1
        return loaded


def loader_scale_string(scale: float) -> str:
    """The scale string load_safetensors gives an I8 tensor (tensor_store.rs:716-724):
    `{:.6}` of the f32 scale with trailing zeros, then a trailing dot, trimmed ("1", "0.5")."""
    return f"{float(np.float32(scale)):.6f}".rstrip("0").rstrip(".")


def f16_bits_to_f32(bits):
    """tensor_store.rs:59-82 on an array of f16 bit patterns: exact, subnormals included, a NaN
    keeps its payload (mantissa << 13) without the quiet bit being forced."""
    bits = np.asarray(bits, np.uint16)
    out = bits.view(np.float16).astype(np.float32).view(np.uint32).copy()
    u = bits.astype(np.uint32)
    nan = ((u >> 10) & 0x1F == 0x1F) & (u & 0x3FF != 0)
    out[nan] = ((u[nan] >> 15) << 31) | 0x7F800000 | ((u[nan] & 0x3FF) << 13)
    return out.view(np.float32)


def f32_to_f16_bits_trunc(vals):
    """tensor_store.rs:84-102 on an f32 array: mantissa truncated, exponent overflow to +-inf,
    new exponent <= 0 to signed zero (no subnormals), NaN -> 0x7e00 | sign."""
    b = np.asarray(vals, np.float32).view(np.uint32)
    sign = ((b >> 16) & 0x8000).astype(np.uint32)
    exp = ((b >> 23) & 0xFF).astype(np.int64)
    mant = b & 0x7FFFFF
    new_exp = exp - 112
    res = np.where(new_exp >= 31, sign | 0x7C00,
                   np.where(new_exp <= 0, sign, sign | (np.clip(new_exp, 0, 31).astype(np.uint32) << 10) | (mant >> 13)))
    res = np.where(exp == 255, sign | 0x7C00 | np.where(mant != 0, 0x200, 0), res)
    return res.astype(np.uint16)


def dequantize_packed(b: QuantizedPacked):
    """f32 [N, K] of a packed backing, on the GPU."""
    from . import ops

    n, k = b.shape
    if b.format == "int4_asym":
        return ops.dequantize_int4g(ops.Int4Packed(b.codes, b.scales, b.zeros, n, k, b.group))
    if b.format == "nf4":
        return ops.dequantize_nf4(ops.Nf4Packed(b.codes, b.scales, n, k, b.group))
    if b.format == "int8_channel":
        return ops.dequantize_int8(b.codes, b.scales, "channel")
    if b.format == "fp8_row":
        return ops.dequantize_fp8(b.codes, b.scales)
    if b.format in ("gguf_q4_0", "gguf_q8_0"):
        ty = ops.GGML_TYPES["Q4_0" if b.format == "gguf_q4_0" else "Q8_0"]
        return ops.dequantize_gguf(ops.GgufPacked(ty, b.codes, b.scales, n, k))
    raise ValueError(f"unknown packed format {b.format}")
