"""GGUF v2/v3 reader and writer over the GPU payload kernels (ir/formats/gguf.rs).

Host side of the reference's `import_gguf_bytes` / `export_gguf_bytes` (gguf.rs:54-246,
248-333): the same header, metadata and tensor-info parsing with the same checks and error
messages, the same synthesized `@forward` graph and TensorStore entries.  Every tensor payload
is decoded or encoded on the GPU (castforge_hip_gguf_decode / _encode); the host only parses
and writes the container.

Beyond the reference, `import_gguf_bytes(..., keep_packed=True)` keeps 2-D Q4_0 / Q8_0 tensors
packed as GGUF planes (QuantizedPacked formats `gguf_q4_0` / `gguf_q8_0`, repacked once on the
GPU) so the dequant-fused GEMV reads them directly, and the writer exports such entries back
as Q4_0 / Q8_0 blocks, bit for bit.
"""
from __future__ import annotations

import struct

import numpy as np
import torch

from . import ops
from .ir import Dense, Module, QuantPacked, TensorRef, TensorType
from .tensor_store import F32Data, QuantizedI8, QuantizedPacked, TensorEntry, TensorStore

GGUF_MAGIC = b"GGUF"
GGUF_DEFAULT_ALIGNMENT = 32
MAX_TENSOR_ELEMENTS = 1_000_000_000  # ir/mlir.rs:144
GGML_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 8: "Q8_0", 30: "BF16"}
PACKED_FORMATS = {2: "gguf_q4_0", 8: "gguf_q8_0"}


class GgufError(ValueError):
    pass


def sanitize_name(s: str) -> str:
    """formats/safetensors.rs:223-233: ASCII alphanumerics and '_' kept, anything else '_'."""
    return "".join(c if (c.isascii() and c.isalnum()) or c == "_" else "_" for c in s)


class _Reader:
    def __init__(self, raw: bytes, pos: int):
        self.raw, self.pos = raw, pos

    def u32(self) -> int:
        if self.pos + 4 > len(self.raw):
            raise GgufError("Unexpected EOF reading u32")
        (v,) = struct.unpack_from("<I", self.raw, self.pos)
        self.pos += 4
        return v

    def u64(self) -> int:
        if self.pos + 8 > len(self.raw):
            raise GgufError("Unexpected EOF reading u64")
        (v,) = struct.unpack_from("<Q", self.raw, self.pos)
        self.pos += 8
        return v

    def string(self) -> str:
        n = self.u64()
        if self.pos + n > len(self.raw):
            raise GgufError("Unexpected EOF reading GGUF string")
        s = self.raw[self.pos:self.pos + n].decode("utf-8", "replace")
        self.pos += n
        return s

    def value(self, ty: int):
        """gguf.rs:421-463: skips a metadata value, returning the integer / string ones as text."""
        if ty in (0, 1, 7):
            if self.pos + 1 > len(self.raw):
                raise GgufError("Unexpected EOF reading 1-byte GGUF metadata value")
            self.pos += 1
            return None
        if ty in (2, 3):
            if self.pos + 2 > len(self.raw):
                raise GgufError("Unexpected EOF reading 2-byte GGUF metadata value")
            self.pos += 2
            return None
        if 4 <= ty <= 6:
            return str(self.u32())
        if ty == 8:
            return self.string()
        if ty == 9:
            elem = self.u32()
            for _ in range(self.u64()):
                self.value(elem)
            return None
        if 10 <= ty <= 12:
            return str(self.u64())
        raise GgufError(f"Unsupported GGUF metadata value type: {ty}")


def read_gguf_header(raw: bytes):
    """gguf.rs:56-137: (model name, [(name, row-major shape, ggml type, offset)], data base)."""
    if len(raw) < 24 or raw[:4] != GGUF_MAGIC:
        raise GgufError("Invalid GGUF header magic (expected 'GGUF')")
    r = _Reader(raw, 4)
    version = r.u32()
    if not 2 <= version <= 3:
        raise GgufError(f"Unsupported GGUF version: {version}")
    tensor_count, kv_count = r.u64(), r.u64()
    if tensor_count > 65_536 or kv_count > 65_536:
        raise GgufError(f"GGUF header counts (tensors={tensor_count}, kv={kv_count}) exceed safety limit")
    name, alignment = "gguf_model", GGUF_DEFAULT_ALIGNMENT
    for _ in range(kv_count):
        key = r.string()
        val = r.value(r.u32())
        if key == "general.name" and val is not None:
            name = sanitize_name(val)
        elif key == "general.alignment" and val is not None:
            try:
                a = int(val)
            except ValueError:
                a = 0
            if a > 0 and a & (a - 1) == 0:
                alignment = a
    infos = []
    for _ in range(tensor_count):
        tname = r.string()
        nd = r.u32()
        if nd > 16:
            raise GgufError(f"GGUF tensor `{tname}` rank {nd} exceeds maximum rank 16")
        dims, elems = [], 1
        for _ in range(nd):
            d = r.u64()
            if d >= 1 << 63:
                raise GgufError("GGUF dimension overflows i64")
            elems *= max(d, 1)
            if elems > MAX_TENSOR_ELEMENTS:
                raise GgufError(f"GGUF tensor `{tname}` exceeds max tensor element limit")
            dims.append(d)
        dims.reverse()  # GGUF stores the innermost dimension first
        if not dims:
            dims = [1]
        ty = r.u32()
        if ty not in GGML_NAMES:
            raise GgufError(f"Unsupported GGML tensor type id: {ty}")
        infos.append((tname, tuple(dims), ty, r.u64()))
    data_base = (r.pos + alignment - 1) // alignment * alignment
    return name, infos, data_base


def import_gguf_bytes(raw: bytes, device=None, keep_packed: bool = False) -> Module:
    """gguf.rs:54-246.  Tensors are decoded to f32 on the GPU; with keep_packed, 2-D Q4_0 /
    Q8_0 tensors whose row length suits the GGUF planes stay packed instead."""
    device = torch.device(device or "cuda")
    name, infos, base = read_gguf_header(raw)
    decoded = []
    for tname, shape, ty, off in infos:
        n = 1
        for d in shape:
            n *= max(d, 1)
        n = max(n, 1)
        start = base + off
        nbytes = ops.gguf_payload_bytes(ty, n)
        if start + nbytes > len(raw):
            raise GgufError(f"GGUF {GGML_NAMES[ty]} tensor data out of bounds")
        payload = torch.frombuffer(bytearray(raw[start:start + nbytes]), dtype=torch.uint8).to(device)
        if keep_packed and ty in PACKED_FORMATS and len(shape) == 2 and ops.gguf_planes_ok(ty, shape[1]):
            p = ops.gguf_repack(ty, payload, shape[0], shape[1])
            decoded.append((tname, shape, QuantizedPacked(PACKED_FORMATS[ty], p.codes, p.scales, None, 32, shape)))
        else:
            decoded.append((tname, shape, F32Data(ops.gguf_decode(ty, payload, n).reshape(shape))))

    m = Module(name)
    if not decoded:
        m.set_results(m.add_argument(TensorType((1, 4), "f32"), "x"))
        return m
    first_k = decoded[0][1][0]
    rows, cols = 1, first_k
    cur = m.add_argument(TensorType((1, first_k), "f32"), "x")
    for idx, (tname, shape, backing) in enumerate(decoded):
        if isinstance(backing, F32Data):
            w = m.constant(f"w{idx}", backing.data, inline=True)
        else:
            qty = TensorType(shape, QuantPacked(backing.format, "f32", 32))
            w = m.add_op("stablehlo.constant", [], [qty], {"value": TensorRef(tname)}, [f"w{idx}"]).results[0]
        if len(shape) == 2 and shape[0] == cols:
            cur = m.dot_general(cur, w, name=f"h{idx}")
            cols = shape[1]
        elif len(shape) == 2 and shape == (rows, cols):
            cur = m.add_op("stablehlo.add", [cur, w], [TensorType((rows, cols), "f32")], {}, [f"h{idx}"]).results[0]
        elif len(shape) == 1 and shape[0] == cols:
            bc = m.add_op("stablehlo.broadcast_in_dim", [w], [TensorType((rows, cols), "f32")],
                          {"broadcast_dimensions": [1]}, [f"bc{idx}"]).results[0]
            op = "stablehlo.multiply" if "norm" in tname else "stablehlo.add"
            cur = m.add_op(op, [cur, bc], [TensorType((rows, cols), "f32")], {}, [f"h{idx}"]).results[0]
    m.set_results(cur)
    m.tensor_store = TensorStore()
    for tname, shape, backing in decoded:
        if isinstance(backing, F32Data):
            m.tensor_store.insert(TensorEntry(tname, TensorType(shape, "f32"), backing))
        else:
            m.tensor_store.insert(TensorEntry(tname, TensorType(shape, QuantPacked(backing.format, "f32", 32)), backing))
    return m


def _module_tensors(module: Module) -> list[tuple[str, TensorEntry]]:
    """formats/safetensors.rs:9-74: the TensorStore, or else the graph's constants."""
    if len(module.tensor_store):
        return list(module.tensor_store.items())
    out, idx = [], 0
    for oid in module.block_ops():
        op = module.ops[oid]
        if not op.is_op("stablehlo", "constant") or not op.results:
            continue
        v = module.values[op.results[0]]
        attr = op.attributes.get("value")
        if not isinstance(attr, Dense):
            continue
        if v.ssa_name:
            nm = v.ssa_name.lstrip("%")
        else:
            idx += 1
            nm = f"const_{idx}.weight"
        out.append((nm, TensorEntry(nm, v.ty, F32Data(attr.data.float().reshape(-1)))))
    return out


def _payload(entry: TensorEntry) -> tuple[int, torch.Tensor]:
    """gguf.rs:280-322: (ggml type, device payload) of one store entry."""
    b = entry.backing
    if isinstance(b, QuantizedI8):
        return 8, ops.gguf_encode(8, b.data.reshape(-1).contiguous(), float(b.scale))
    if isinstance(b, QuantizedPacked):
        n, k = b.shape
        if b.format in ("gguf_q4_0", "gguf_q8_0"):
            ty = 2 if b.format == "gguf_q4_0" else 8
            return ty, ops.gguf_unpack(ops.GgufPacked(ty, b.codes, b.scales, n, k))
        from .tensor_store import dequantize_packed
        return 0, ops.gguf_encode(0, dequantize_packed(b).reshape(-1).contiguous())
    vals = b.data.reshape(-1).float().contiguous()
    dt = entry.ty.dtype
    ty = 1 if dt == "f16" else 30 if dt == "bf16" else 0
    return ty, ops.gguf_encode(ty, vals)


def export_gguf_bytes(module: Module) -> bytes:
    """gguf.rs:248-333: GGUF v3 with one metadata key (general.name), tensors in store order,
    every payload padded to 32 bytes.  (A rank-0 tensor is written with one dimension of 1;
    the reference writes n_dims = 1 and no dimension.)"""
    out = bytearray(GGUF_MAGIC)
    tensors = _module_tensors(module)
    out += struct.pack("<IQQ", 3, len(tensors), 1)

    def put_str(s: str):
        b = s.encode()
        out.extend(struct.pack("<Q", len(b)) + b)

    put_str("general.name")
    out += struct.pack("<I", 8)
    put_str(module.name or "castforge_model")
    payloads, offset = [], 0
    for name, entry in tensors:
        put_str(name)
        dims = [int(d) if int(d) > 0 else 1 for d in entry.ty.shape] or [1]
        out += struct.pack("<I", len(dims))
        for d in reversed(dims):
            out += struct.pack("<Q", d)
        ty, dev_payload = _payload(entry)
        data = dev_payload.cpu().numpy().tobytes()
        data += b"\0" * ((-len(data)) % GGUF_DEFAULT_ALIGNMENT)
        out += struct.pack("<IQ", ty, offset)
        offset += len(data)
        payloads.append(data)
    out += b"\0" * ((-len(out)) % GGUF_DEFAULT_ALIGNMENT)
    for p in payloads:
        out += p
    return bytes(out)


def write_gguf_tensors(tensors: list[tuple[str, tuple, int, np.ndarray]], name: str = "castforge_model") -> bytes:
    """A GGUF v3 container of ready payloads [(name, row-major shape, ggml type, payload
    bytes)], laid out as export_gguf_bytes lays them out."""
    out = bytearray(GGUF_MAGIC)
    out += struct.pack("<IQQ", 3, len(tensors), 1)

    def put_str(s: str):
        b = s.encode()
        out.extend(struct.pack("<Q", len(b)) + b)

    put_str("general.name")
    out += struct.pack("<I", 8)
    put_str(name)
    offset, blobs = 0, []
    for tname, shape, ty, payload in tensors:
        put_str(tname)
        out += struct.pack("<I", len(shape))
        for d in reversed(shape):
            out += struct.pack("<Q", int(d))
        data = bytes(np.ascontiguousarray(payload, np.uint8).tobytes())
        data += b"\0" * ((-len(data)) % GGUF_DEFAULT_ALIGNMENT)
        out += struct.pack("<IQ", ty, offset)
        offset += len(data)
        blobs.append(data)
    out += b"\0" * ((-len(out)) % GGUF_DEFAULT_ALIGNMENT)
    for d in blobs:
        out += d
    return bytes(out)
