"""The slice of the reference's IR that the quantized-weight path touches, as host-side Python.

Mirrors, for this path only:
  * `DType` incl. `QuantUniform` and its printed / parsed form `!quant.uniform<st:ex,scale:zp>`
    (ir/mlir.rs:33-38, 82-91; ir/parser.rs:1336-1351), where the scale is the decimal string
    the quantizer formatted (passes/quantize/formats.rs:680-688);
  * `TensorType` and its `tensor<AxBxT>` form (ir/mlir.rs:159-175);
  * an SSA `Module` with one function body: values, operations, attributes, and the
    `TensorStore` weight plane (ir/tensor_store.rs).
The packed formats the reference has no type for (INT8 per-channel, INT4 asymmetric
group-wise, NF4, FP8 per-row) get `!castforge.packed<format:expressed,group>`.

Constants hold device tensors (torch, for memory only); no computation happens here.
"""
from __future__ import annotations

import copy
from dataclasses import dataclass, field
from typing import Any, Union

# ------------------------------------------------------------------------------------ types ----
SCALAR_DTYPES = ("i1", "i4", "i8", "i16", "i32", "i64", "ui8", "ui16", "ui32", "ui64",
                 "f8E4M3FN", "f8E5M2", "f16", "bf16", "f32", "f64", "index")


@dataclass(frozen=True)
class QuantUniform:
    """`!quant.uniform<storage:expressed,scale:zero_point>`; `scale` is kept as the string the
    quantizer printed, exactly as the reference does (the evaluator parses it back)."""
    storage: str
    expressed: str
    scale: str
    zero_point: int

    def __str__(self) -> str:
        return f"!quant.uniform<{self.storage}:{self.expressed},{self.scale}:{self.zero_point}>"


@dataclass(frozen=True)
class QuantPacked:
    """Packed low-bit weights of this library: format in {int8_channel, int4_asym, nf4,
    fp8_row, gguf_q4_0, gguf_q8_0}; group is the INT4 group / NF4 block / GGUF block (0 when
    not grouped)."""
    format: str
    expressed: str
    group: int

    def __str__(self) -> str:
        return f"!castforge.packed<{self.format}:{self.expressed},{self.group}>"


DType = Union[str, QuantUniform, QuantPacked]


def parse_dtype(s: str) -> DType:
    """parser.rs:1336-1351: unknown scalar names fall back to f32."""
    d = try_parse_dtype(s)
    return "f32" if d is None else d


def try_parse_dtype(s: str) -> DType | None:
    s = s.strip()
    if s.startswith("!quant.uniform<") and s.endswith(">") and "," in s:
        inner = s[len("!quant.uniform<"):-1]
        types_part, scale_part = inner.split(",", 1)
        st, ex = types_part.split(":", 1) if ":" in types_part else ("i8", "f32")
        sc, zp = scale_part.strip().split(":", 1) if ":" in scale_part else ("1.0", "0")
        try:
            zpi = int(zp.strip())
        except ValueError:
            zpi = 0
        return QuantUniform(parse_dtype(st.strip()), parse_dtype(ex.strip()), sc.strip(), zpi)
    if s.startswith("!castforge.packed<") and s.endswith(">"):
        inner = s[len("!castforge.packed<"):-1]
        fe, grp = inner.rsplit(",", 1)
        fmt, ex = fe.split(":", 1)
        return QuantPacked(fmt.strip(), parse_dtype(ex.strip()), int(grp.strip()))
    return s if s in SCALAR_DTYPES else None


def format_scale(scale: float) -> str:
    """formats.rs:680-688: `{:.6}`, trailing zeros and dot trimmed, `.0` appended when no dot
    remains (Rust's {:.6} and C's %.6f both round the exact binary value to nearest)."""
    s = f"{scale:.6f}".rstrip("0").rstrip(".")
    return s if "." in s else s + ".0"


@dataclass(frozen=True)
class TensorType:
    shape: tuple
    dtype: DType

    def num_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= int(d)
        return n

    def __str__(self) -> str:
        dims = "".join(f"{d}x" for d in self.shape)
        return f"tensor<{dims}{self.dtype}>"


def parse_tensor_type(s: str) -> TensorType:
    s = s.strip()
    if not (s.startswith("tensor<") and s.endswith(">")):
        raise ValueError(f"not a tensor type: {s}")
    body = s[len("tensor<"):-1]
    parts = []
    while True:
        head, sep, rest = body.partition("x")
        if sep and head.isdigit():
            parts.append(int(head))
            body = rest
        else:
            break
    return TensorType(tuple(parts), parse_dtype(body))


# ----------------------------------------------------------------------------- attributes ----
@dataclass
class TensorRef:
    """`dense_resource<key>`: the constant's data lives in the TensorStore under `key`."""
    key: str


@dataclass
class Dense:
    """An inline constant (`dense<...>`) holding a device tensor."""
    data: Any


# ------------------------------------------------------------------------------ SSA graph ----
@dataclass
class Value:
    id: int
    ty: TensorType
    ssa_name: str | None = None
    op: int | None = None      # defining op id (None for function arguments)
    arg: int | None = None     # argument index


@dataclass
class Operation:
    id: int
    name: str                  # "dialect.op", e.g. "stablehlo.constant"
    operands: list
    results: list
    attributes: dict = field(default_factory=dict)

    def is_op(self, dialect: str, op: str) -> bool:
        return self.name == f"{dialect}.{op}"


class Module:
    """One function body (`@forward`) in program order, plus the TensorStore."""

    def __init__(self, name: str = "main"):
        from .tensor_store import TensorStore

        self.name = name
        self.values: dict[int, Value] = {}
        self.ops: dict[int, Operation] = {}
        self.order: list[int] = []       # op ids in program order
        self.args: list[int] = []
        self.results: list[int] = []     # func.return operands
        self.tensor_store = TensorStore()
        self._next = 0

    # -- construction ----------------------------------------------------------------------
    def _id(self) -> int:
        self._next += 1
        return self._next

    def add_argument(self, ty: TensorType, name: str | None = None) -> int:
        v = Value(self._id(), ty, name, None, len(self.args))
        self.values[v.id] = v
        self.args.append(v.id)
        return v.id

    def add_op(self, name: str, operands, result_types, attributes=None, ssa_names=None,
               after: int | None = None, before: int | None = None) -> Operation:
        op = Operation(self._id(), name, list(operands), [], dict(attributes or {}))
        for i, ty in enumerate(result_types):
            nm = ssa_names[i] if ssa_names and i < len(ssa_names) else None
            v = Value(self._id(), ty, nm, op.id, None)
            self.values[v.id] = v
            op.results.append(v.id)
        self.ops[op.id] = op
        if after is not None:
            self.order.insert(self.order.index(after) + 1, op.id)
        elif before is not None:
            self.order.insert(self.order.index(before), op.id)
        else:
            self.order.append(op.id)
        return op

    def constant(self, name: str, data, dtype: str = "f32", inline: bool = False) -> int:
        """A `stablehlo.constant` of a device tensor; stored in the TensorStore under `name`
        (dense_resource) unless `inline`."""
        from .tensor_store import F32Data, TensorEntry

        ty = TensorType(tuple(int(d) for d in data.shape), dtype)
        if inline:
            attr = Dense(data)
        else:
            self.tensor_store.insert(TensorEntry(name, ty, F32Data(data)))
            attr = TensorRef(name)
        return self.add_op("stablehlo.constant", [], [ty], {"value": attr}, [name]).results[0]

    def dot_general(self, lhs: int, rhs: int, packed_rhs: bool = False, name: str | None = None) -> int:
        """2-D matmul: rhs [K, N] (contracting [1] x [0]) or, packed, [N, K] ([1] x [1])."""
        a, b = self.values[lhs].ty, self.values[rhs].ty
        n = b.shape[0] if packed_rhs else b.shape[1]
        attrs = {"lhs_contracting_dimensions": [1], "rhs_contracting_dimensions": [1 if packed_rhs else 0]}
        if packed_rhs:
            attrs["packed_rhs"] = True
        ty = TensorType((a.shape[0], n), "f32")
        return self.add_op("stablehlo.dot_general", [lhs, rhs], [ty], attrs, [name]).results[0]

    def set_results(self, *vals: int) -> None:
        self.results = list(vals)

    # -- queries / rewrites ----------------------------------------------------------------
    def block_ops(self) -> list[int]:
        return list(self.order)

    def users(self, val: int) -> list[int]:
        return [oid for oid in self.order if val in self.ops[oid].operands]

    def replace_uses(self, old: int, new: int, skip_op: int | None = None) -> None:
        for oid in self.order:
            if oid == skip_op:
                continue
            op = self.ops[oid]
            op.operands = [new if o == old else o for o in op.operands]
        self.results = [new if r == old else r for r in self.results]

    def erase_op(self, oid: int) -> None:
        op = self.ops.pop(oid)
        self.order.remove(oid)
        for r in op.results:
            self.values.pop(r, None)

    def dce(self) -> int:
        """Removes ops whose results are unused (the SSA-only DCE run after fusion)."""
        removed = 0
        changed = True
        while changed:
            changed = False
            live = set(self.results)
            for oid in self.order:
                live.update(self.ops[oid].operands)
            for oid in list(reversed(self.order)):
                op = self.ops[oid]
                if op.results and not any(r in live for r in op.results):
                    self.erase_op(oid)
                    removed += 1
                    changed = True
        return removed

    def verify(self) -> None:
        """Every operand is defined before use; results exist; constants carry a value."""
        defined = set(self.args)
        for oid in self.order:
            op = self.ops[oid]
            for o in op.operands:
                if o not in defined:
                    raise ValueError(f"op {op.name} (#{oid}) uses undefined value %{o}")
            if op.is_op("stablehlo", "constant") and "value" not in op.attributes:
                raise ValueError(f"constant #{oid} has no value")
            defined.update(op.results)
        for r in self.results:
            if r not in defined:
                raise ValueError(f"return of undefined value %{r}")

    def clone(self) -> "Module":
        """Graph deep copy; the TensorStore is shared copy-on-write (tensor_store.rs:214-233)."""
        m = Module.__new__(Module)
        m.name = self.name
        m.values = copy.deepcopy(self.values)
        m.ops = {k: Operation(o.id, o.name, list(o.operands), list(o.results), dict(o.attributes))
                 for k, o in self.ops.items()}
        m.order = list(self.order)
        m.args = list(self.args)
        m.results = list(self.results)
        m.tensor_store = self.tensor_store.clone()
        m._next = self._next
        return m

    # -- printing ----------------------------------------------------------------------------
    def _vname(self, vid: int) -> str:
        v = self.values[vid]
        return f"%{v.ssa_name}" if v.ssa_name else f"%v{vid}"

    def print_mlir(self) -> str:
        lines = [f"module @{self.name} {{"]
        args = ", ".join(f"{self._vname(a)}: {self.values[a].ty}" for a in self.args)
        rtys = ", ".join(str(self.values[r].ty) for r in self.results)
        lines.append(f"  func.func @forward({args}) -> ({rtys}) {{")
        for oid in self.order:
            op = self.ops[oid]
            res = ", ".join(self._vname(r) for r in op.results)
            opnds = ", ".join(self._vname(o) for o in op.operands)
            attrs = []
            for k, v in op.attributes.items():
                if k == "value":
                    attrs.append(f"dense_resource<{v.key}>" if isinstance(v, TensorRef) else "dense<...>")
                elif isinstance(v, bool):
                    attrs.append(f"{k} = {'true' if v else 'false'}")
                elif isinstance(v, str):
                    attrs.append(f'{k} = "{v}"')
                else:
                    attrs.append(f"{k} = {v}")
            tys = ", ".join(str(self.values[r].ty) for r in op.results)
            head = f"{res} = " if res else ""
            lines.append(f"    {head}{op.name} {opnds} {{{', '.join(attrs)}}} : {tys}".rstrip())
        lines.append(f"    func.return {', '.join(self._vname(r) for r in self.results)}")
        lines.append("  }")
        lines.append("}")
        return "\n".join(lines)
