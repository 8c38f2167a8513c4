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

import torch

from .ir import Dense, QuantPacked, QuantUniform, TensorRef, TensorType, format_scale


@dataclass
class F32Data:
    data: Any  # device f32 tensor


@dataclass
class QuantizedI8:
    data: Any  # device int8 tensor
    scale: float
    zero_point: int


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
                put(name, "F32", shape, b.data.detach().contiguous().cpu().numpy().tobytes())
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
        import numpy as np

        (hlen,) = struct.unpack("<Q", raw[:8])
        header = json.loads(raw[8:8 + hlen].decode())
        base = 8 + hlen
        meta = json.loads(header.pop("__metadata__", {}).get("castforge_packed", "{}"))
        npd = {"F32": np.float32, "F16": np.float16, "I8": np.int8, "I32": np.int32, "U8": np.uint8}
        parts: dict[str, Any] = {}
        loaded = 0
        for name, h in header.items():
            a, b = h["data_offsets"]
            arr = np.frombuffer(raw[base + a:base + b], dtype=npd[h["dtype"]]).reshape(h["shape"]).copy()
            t = torch.from_numpy(arr).to(device)
            stem, _, part = name.rpartition(".")
            if stem in meta and part in ("codes", "scales", "zeros"):
                parts.setdefault(stem, {})[part] = t
                continue
            shape = tuple(h["shape"])
            if h["dtype"] == "I8":
                scale = float(h.get("scale", 1.0))
                zp = int(h.get("zero_point", 0))
                dt = QuantUniform("i8", "f32", format_scale(scale), zp) if "scale" in h else "i8"
                self.insert(TensorEntry(name, TensorType(shape, dt), QuantizedI8(t, scale, zp)))
            elif h["dtype"] in ("F32", "F16"):
                self.insert(TensorEntry(name, TensorType(shape, "f32"), F32Data(t.float())))
            else:
                continue
            loaded += 1
        for stem, m in meta.items():
            p = parts.get(stem, {})
            ty = TensorType(tuple(m["shape"]), QuantPacked(m["format"], m.get("expressed", "f32"), m["group"]))
            self.insert(TensorEntry(stem, ty, QuantizedPacked(m["format"], p.get("codes"), p.get("scales"),
                                                              p.get("zeros"), m["group"], tuple(m["shape"]))))
            loaded += 1
        return loaded


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
