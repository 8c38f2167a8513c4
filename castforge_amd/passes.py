"""The reference's pass interface for the quantized-weight path, on the HIP kernels.

Mirrors passes/registry/manager.rs (Pass, PassResult, PassRegistry with option validation
against the documented options plus the alias list, PassManager.from_pipeline_str and
verify-after-each-pass) and the passes of this path:

  quantize              QuantizePass factory (registry/families.rs:93-183, schemes.rs:27-153)
  quantize-weights      per-tensor symmetric i8/i4 + uniform_dequantize (schemes.rs:301-453)
  quantize-groupwise    group-wise / AWQ-salient write-back (schemes.rs:456-630)
  quantize-fp8          FP8 / MXFP8 uniform-grid write-back (schemes.rs:633-754)
  lower-mixed-precision bf16 / f16 operand converts on dot_general (formats.rs:520-650)
  fuse-gemm(kind=dequant), fuse-dequant-matmul
                        dot_general(x, uniform_dequantize(w)) -> castforge.fused_qmatmul
                        (passes/fuse/gemm.rs:102-127, epilogue.rs:10-94)
  pack-weights          [K, N] -> [N, K] constant rhs, packed_rhs = true (weights/fold.rs:456-591)

Schemes this library adds behind `quantize(scheme=...)` (the reference has none of them):
  int8_channel  per-output-channel symmetric INT8, `round=half_even`
  int4_asym     INT4 asymmetric group-wise, f16 scale + u4 zero point, 8 codes per u32
  nf4           NF4 block-wise with f32 absmax
  fp8_row       FP8 E4M3 with one f32 scale per row
They quantize 2-D f32 constants stored [N, K] and insert the same `uniform_dequantize`.

Option inference keeps the reference's quirk: `quantize(bits=4,group=128)` has no
`group_size` key, so it selects per-tensor `quantize-weights` (families.rs:93-116).
Everything numeric runs in libcastforge_hip.so; errors are ValueError with the reference's
messages.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import ffi, ops
from .ir import Dense, Module, QuantPacked, QuantUniform, TensorRef, TensorType, format_scale
from .tensor_store import F32Data, QuantizedI8, QuantizedPacked, TensorEntry


# ------------------------------------------------------------------------ framework ----
@dataclass
class PassResult:
    pass_name: str
    changed: bool = False
    ops_removed: int = 0
    ops_modified: int = 0
    ops_created: int = 0

    def with_name(self, name: str) -> "PassResult":
        self.pass_name = name
        return self

    @staticmethod
    def aggregate(name: str, steps: list["PassResult"]) -> "PassResult":
        return PassResult(name, any(s.changed for s in steps), sum(s.ops_removed for s in steps),
                          sum(s.ops_modified for s in steps), sum(s.ops_created for s in steps))


class Pass:
    name = ""
    description = ""

    def run(self, module: Module) -> PassResult:  # pragma: no cover - interface
        raise NotImplementedError


# manager.rs:548-727: option keys accepted by every pass besides its documented ones
# (the subset of the alias list that this path's passes read)
OPTION_ALIASES = frozenset({
    "mode", "kind", "target", "targets", "constants", "hoist", "dtype", "group", "mxfp8", "size",
    "samples", "num_samples", "block_size", "salient_ratio", "awq_salient", "alpha", "bits",
    "group_size", "scheme", "format", "min_elements", "hadamard", "name", "layout",
})

# config/passes.toml documented options (plus `round` and `granularity`, added by this build)
CATALOG = {
    "quantize": ["scheme", "bits", "group_size", "salient_ratio", "format", "block_size", "alpha",
                 "round", "granularity", "hadamard_axis"],
    "quantize-weights": ["bits", "min_elements", "round", "granularity"],
    "quantize-groupwise": ["bits", "group_size", "awq_salient", "salient_ratio"],
    "quantize-fp8": ["format", "mxfp8", "block_size"],
    "lower-mixed-precision": ["dtype"],
    "fuse-gemm": ["kind"],
    "fuse-dequant-matmul": [],
    "pack-weights": [],
    "calibrate-quantize": ["bits", "samples"],
    "rotate-hadamard": ["block_size"],
    "smooth-quantize": ["bits", "alpha", "samples"],
}


class PassRegistry:
    def __init__(self):
        self._passes: dict[str, tuple[str, callable]] = {}

    def register(self, name: str, description: str, factory) -> None:
        self._passes[name] = (description, factory)

    def list(self):
        return [(n, d) for n, (d, _) in self._passes.items()]

    def create_pass(self, name: str, opts: dict[str, str]) -> Pass:
        """manager.rs:512-540."""
        if name not in self._passes:
            raise ValueError(f"Unknown pass `{name}`. Run `castforge list-passes` to see available passes.")
        cat = CATALOG.get(name)
        if opts and cat is not None:
            if not cat:
                raise ValueError(f"Pass `{name}` does not accept options (got `{', '.join(opts)}`)")
            for k in opts:
                if k not in cat and k not in OPTION_ALIASES:
                    raise ValueError(f"Pass `{name}`: unrecognized option `{k}` (documented options: "
                                     f"{', '.join(cat)})")
        return self._passes[name][1](opts)


def split_pipeline_spec(spec: str) -> list[str]:
    """manager.rs:410-427: split at top-level `,` or `|`."""
    out, start, depth = [], 0, 0
    for i, c in enumerate(spec):
        if c == "(":
            depth += 1
        elif c == ")":
            depth = max(0, depth - 1)
        elif c in ",|" and depth == 0:
            out.append(spec[start:i])
            start = i + 1
    out.append(spec[start:])
    return out


def parse_pass_spec_item(item: str) -> tuple[str, dict[str, str]]:
    """manager.rs:430-459: `name(k1=v1,k2=v2)`."""
    item = item.strip()
    opts: dict[str, str] = {}
    if "(" not in item:
        return item, opts
    open_ = item.index("(")
    close = item.rfind(")")
    if close < 0:
        raise ValueError(f"Unclosed `(` in pass specification `{item}`")
    if item[close + 1:].strip():
        raise ValueError(f"Unexpected trailing characters after `)` in pass specification `{item}`")
    for kv in item[open_ + 1:close].split(","):
        kv = kv.strip()
        if not kv:
            continue
        if "=" not in kv:
            raise ValueError(f"Expected `key=value` option in `{item}`")
        k, v = kv.split("=", 1)
        opts[k.strip()] = v.strip().strip('"').strip("'")
    return item[:open_].strip(), opts


class PassManager:
    def __init__(self):
        self.passes: list[Pass] = []
        self.verify_after_each_pass = True

    @staticmethod
    def from_pipeline_str(registry: PassRegistry, spec: str) -> "PassManager":
        pm = PassManager()
        for item in split_pipeline_spec(spec):
            if item.strip():
                name, opts = parse_pass_spec_item(item)
                pm.passes.append(registry.create_pass(name, opts))
        return pm

    def run(self, module: Module) -> list[PassResult]:
        history = []
        for p in self.passes:
            r = p.run(module)
            if self.verify_after_each_pass:
                module.verify()
            history.append(r)
        return history


# ------------------------------------------------------------------- option helpers ----
def _u8(v, default):
    try:
        x = int(v)
        return x if 0 <= x <= 255 else default
    except (TypeError, ValueError):
        return default


def _usize(v, default):
    try:
        x = int(v)
        return x if x >= 0 else default
    except (TypeError, ValueError):
        return default


def _f32(v, default):
    try:
        return float(torch.tensor(float(v), dtype=torch.float32))
    except (TypeError, ValueError):
        return default


def _first(opts, *keys):
    for k in keys:
        if k in opts:
            return opts[k]
    return None


FLOAT_DTYPES = ("f32", "f16", "bf16")


def _const_ops(module: Module):
    for oid in module.block_ops():
        op = module.ops.get(oid)
        if op is not None and op.is_op("stablehlo", "constant") and len(op.results) >= 1:
            yield oid, op


# -------------------------------------------------------------------------- quantize ----
class QuantizeWeightsPass(Pass):
    """schemes.rs:301-453: every float constant with >= min_elements elements becomes i8 codes
    (QuantizedI8 in the store), its type `!quant.uniform<i8|i4:expr,scale:0>`, and a
    `uniform_dequantize` right after it takes over all its uses.  `granularity=tensor` and
    `round=half_away` are the reference; `round=half_even` is this build's option."""
    name = "quantize-weights"
    description = "Post-training symmetric weight quantization (bits=8|4) with uniform_dequantize"

    def __init__(self, bits=8, min_elements=2, round="half_away"):
        self.bits, self.min_elements, self.round = bits, min_elements, round

    def run(self, module: Module) -> PassResult:
        modified = created = 0
        for oid, op in list(_const_ops(module)):
            if len(op.results) != 1:
                continue
            val = module.values[op.results[0]]
            ty = val.ty
            if ty.dtype not in FLOAT_DTYPES or ty.num_elements() < self.min_elements:
                continue
            attr = op.attributes.get("value")
            if attr is None:
                continue
            vals = module.tensor_store.resolve_f32_attr(attr, ty.num_elements())
            if vals is None:
                continue
            codes, scales = ops.quantize_int8(vals.reshape(1, -1).contiguous(), self.bits, "tensor", self.round)
            scale = float(scales[0].item())
            storage = "i4" if self.bits == 4 else "i8"
            qty = TensorType(ty.shape, QuantUniform(storage, ty.dtype, format_scale(scale), 0))
            key = attr.key if isinstance(attr, TensorRef) else (val.ssa_name or f"q_weight_{modified}")
            codes = codes.reshape(ty.shape) if ty.shape else codes.reshape(())
            module.tensor_store.insert(TensorEntry(key, qty, QuantizedI8(codes, scale, 0)))
            val.ty = qty
            op.attributes["value"] = TensorRef(key) if isinstance(attr, TensorRef) else Dense(codes)
            modified += 1
            deq = module.add_op("stablehlo.uniform_dequantize", [val.id], [ty], {},
                                [f"{val.ssa_name}_deq" if val.ssa_name else None], after=oid)
            module.replace_uses(val.id, deq.results[0], skip_op=deq.id)
            created += 1
        return PassResult(self.name, modified > 0, 0, modified, created)


class QuantizePackedPass(Pass):
    """This library's packed schemes on 2-D f32 constants stored [N, K] (rows = output
    channels, groups along K): int8_channel, int4_asym, nf4, fp8_row."""
    name = "quantize-packed"
    description = "Packed low-bit weights (int8_channel | int4_asym | nf4 | fp8_row) for the HIP kernels"

    def __init__(self, fmt: str, group: int = 0, round: str = "half_even", min_elements: int = 2,
                 hadamard: int = 0):
        self.fmt, self.group, self.round, self.min_elements = fmt, group, round, min_elements
        # int4_asym only: rotate each row's K axis in Hadamard blocks first (the block rule of
        # formats.rs:303 applied to K; no rotation when K % b != 0)
        self.hadamard = hadamard
        self.rotated = 0

    def _hadamard_int4(self, w: torch.Tensor):
        k = w.shape[1]
        b = _hadamard_block(self.hadamard, k)
        if k % b != 0:
            p = ops.quantize_int4g(w, self.group)
        elif b & (b - 1):
            raise ValueError(f"quantize: Hadamard block {b} (K = {k}) is not a power of two")
        elif b <= 1024 and self.group >= 16:
            p = ops.quantize_int4g_hadamard(w, self.group, b)  # one pass: rotate in registers
        else:
            p = ops.quantize_int4g(ops.rotate_hadamard(w, b, 1), self.group)
        return QuantizedPacked(self.fmt, p.codes, p.scales, p.zeros, self.group, tuple(w.shape)), b

    def _quantize(self, w: torch.Tensor):
        if self.fmt == "int8_channel":
            c, s = ops.quantize_int8(w, 8, "channel", self.round)
            return QuantizedPacked(self.fmt, c, s, None, 0, tuple(w.shape))
        if self.fmt == "int4_asym":
            p = ops.quantize_int4g(w, self.group)
            return QuantizedPacked(self.fmt, p.codes, p.scales, p.zeros, self.group, tuple(w.shape))
        if self.fmt == "nf4":
            p = ops.quantize_nf4(w, self.group)
            return QuantizedPacked(self.fmt, p.codes, p.absmax, None, self.group, tuple(w.shape))
        if self.fmt == "fp8_row":
            c, s = ops.quantize_fp8(w)
            return QuantizedPacked(self.fmt, c, s, None, 0, tuple(w.shape))
        raise ValueError(f"unknown packed scheme `{self.fmt}`")

    def _fits(self, ty: TensorType) -> bool:
        if ty.dtype != "f32" or len(ty.shape) != 2 or ty.num_elements() < self.min_elements:
            return False
        k = ty.shape[1]
        if self.fmt in ("int4_asym", "nf4"):
            return k % 8 == 0
        return True

    def _quantize_many(self, ws: list[torch.Tensor]) -> list:
        """int8_channel / int4_asym: the batched entry points (one launch per column count);
        the results are bit-identical to _quantize per matrix."""
        if self.hadamard and self.fmt == "int4_asym":
            return [self._hadamard_int4(w) for w in ws]
        if self.fmt == "int8_channel":
            return [QuantizedPacked(self.fmt, c, s, None, 0, tuple(w.shape))
                    for w, (c, s) in zip(ws, ops.quantize_int8_batched(ws, 8, self.round))]
        if self.fmt == "int4_asym":
            return [QuantizedPacked(self.fmt, p.codes, p.scales, p.zeros, self.group, tuple(w.shape))
                    for w, p in zip(ws, ops.quantize_int4g_batched(ws, self.group))]
        return [self._quantize(w) for w in ws]

    def run(self, module: Module) -> PassResult:
        modified = created = 0
        pending = []  # (oid, op, val, ty, attr, f32 values), quantized ffi.MAX_BATCH at a time

        def flush():
            nonlocal modified, created
            packed = self._quantize_many([v for (*_, v) in pending])
            for (oid, op, val, ty, attr, _), b in zip(pending, packed):
                if self.hadamard and self.fmt == "int4_asym":
                    b, hb = b
                    op.attributes["castforge.hadamard_rotated"] = True
                    op.attributes["castforge.hadamard_axis"] = 1
                    _mark_users(module, val.id, {"castforge.hadamard_rotated": True, "castforge.hadamard_block": hb})
                    self.rotated += 1
                qty = TensorType(ty.shape, QuantPacked(self.fmt, "f32", b.group))
                key = attr.key if isinstance(attr, TensorRef) else (val.ssa_name or f"q_weight_{modified}")
                module.tensor_store.insert(TensorEntry(key, qty, b))
                val.ty = qty
                op.attributes["value"] = TensorRef(key)
                modified += 1
                deq = module.add_op("stablehlo.uniform_dequantize", [val.id], [ty], {},
                                    [f"{val.ssa_name}_deq" if val.ssa_name else None], after=oid)
                module.replace_uses(val.id, deq.results[0], skip_op=deq.id)
                created += 1
            pending.clear()

        for oid, op in list(_const_ops(module)):
            val = module.values[op.results[0]]
            ty = val.ty
            attr = op.attributes.get("value")
            if not self._fits(ty) or attr is None:
                continue
            vals = module.tensor_store.resolve_f32_attr(attr, ty.num_elements())
            if vals is None:
                continue
            pending.append((oid, op, val, ty, attr, vals.reshape(ty.shape).contiguous()))
            if len(pending) == ffi.MAX_BATCH:
                flush()
        flush()
        return PassResult(self.name, modified > 0, 0, modified, created)

    def run_steps(self, module: Module) -> list[PassResult]:
        """The Hadamard-fused form as the two steps it replaces (rotate, then quantize)."""
        self.rotated = 0
        r = self.run(module)
        return [PassResult("rotate-hadamard", self.rotated > 0, 0, self.rotated, 0), r]


class QuantizeGroupwisePass(Pass):
    """schemes.rs:456-630 on the GPU (castforge_hip_quantize_groupwise): constants of rank >= 2
    get dequantized f32 written back plus the quant attributes; already-tagged ones are left."""
    name = "quantize-groupwise"
    description = "Group-wise AWQ/GPTQ weight quantization (bits=4|8, group_size=32, awq_salient=true)"

    def __init__(self, bits=4, group_size=32, awq_salient=True, salient_ratio=0.01):
        self.bits, self.group_size, self.awq_salient, self.salient_ratio = bits, group_size, awq_salient, salient_ratio

    def run(self, module: Module) -> PassResult:
        modified = 0
        bits = 4 if self.bits == 4 else 8
        gs = max(self.group_size, 2)
        scheme = "awq_groupwise" if self.awq_salient else "gptq_groupwise"
        for oid, op in list(_const_ops(module)):
            rid = op.results[0]
            ty = module.values[rid].ty
            if len(ty.shape) < 2 or ty.num_elements() < 2:
                continue
            attr = op.attributes.get("value")
            if attr is None:
                continue
            raw = module.tensor_store.resolve_f32_attr(attr, ty.num_elements())
            if raw is None:
                continue
            if op.attributes.get("castforge.quant_scheme") == scheme:
                continue
            deq, scales, count = ops.quantize_groupwise(raw.contiguous(), self.bits, gs, self.awq_salient,
                                                        self.salient_ratio, "half_away")
            nty = TensorType(ty.shape, ty.dtype)
            op.attributes["value"] = module.tensor_store.update_f32_constant(
                module.values[rid].ssa_name, attr, nty, deq)
            tags = {"castforge.quant_scheme": scheme, "castforge.quant_bits": bits, "castforge.group_size": gs}
            op.attributes.update(tags)
            op.attributes["castforge.num_groups"] = scales.numel()
            if self.awq_salient:
                op.attributes["castforge.awq_salient_channels"] = count
            for uid in module.users(rid):
                module.ops[uid].attributes.update(tags)
                if self.awq_salient:
                    module.ops[uid].attributes["castforge.awq_salient_channels"] = count
            modified += 1
        return PassResult(self.name, modified > 0, 0, modified, 0)


class QuantizeFp8Pass(Pass):
    """schemes.rs:633-754 on the GPU (castforge_hip_quantize_fp8_grid)."""
    name = "quantize-fp8"
    description = "Applies FP8 (E4M3/E5M2) and MXFP8 block-scaled quantization to weights and GEMMs"

    def __init__(self, format="e4m3", mxfp8=True, block_size=32):
        self.format, self.mxfp8, self.block_size = format, mxfp8, block_size

    def run(self, module: Module) -> PassResult:
        modified = 0
        e5m2 = self.format.lower() == "e5m2"
        fmt = "fp8_e5m2" if e5m2 else "fp8_e4m3"
        for oid, op in list(_const_ops(module)):
            if op.attributes.get("castforge.fp8_format") == fmt:
                continue
            rid = op.results[0]
            ty = module.values[rid].ty
            if ty.num_elements() < 2:
                continue
            attr = op.attributes.get("value")
            if attr is None:
                continue
            raw = module.tensor_store.resolve_f32_attr(attr, ty.num_elements())
            if raw is None:
                continue
            deq = ops.quantize_fp8_grid(raw.contiguous(), "e5m2" if e5m2 else "e4m3", self.mxfp8, self.block_size)
            op.attributes["value"] = module.tensor_store.update_f32_constant(
                module.values[rid].ssa_name, attr, TensorType(ty.shape, ty.dtype), deq)
            op.attributes["castforge.fp8_format"] = fmt
            for uid in module.users(rid):
                module.ops[uid].attributes["castforge.fp8_format"] = fmt
                module.ops[uid].attributes["castforge.mxfp8"] = self.mxfp8
            modified += 1
        return PassResult(self.name, modified > 0, 0, modified, 0)


class LowerMixedPrecisionPass(Pass):
    """formats.rs:520-650: every dot_general without `compute_precision` gets its f32 operands
    (of the first two) replaced by convert(convert(x -> low) -> f32) tagged `amp_cast`."""
    name = "lower-mixed-precision"
    description = "Applies Automatic Mixed Precision (f16/bf16) casts to GEMM/Conv ops, keeping norms in f32"

    def __init__(self, target_dtype="f16"):
        self.low = "bf16" if target_dtype == "bf16" else "f16"

    def run(self, module: Module) -> PassResult:
        created = modified = 0
        for oid in module.block_ops():
            op = module.ops[oid]
            if "compute_precision" in op.attributes or len(op.operands) < 2:
                continue
            if not op.is_op("stablehlo", "dot_general"):
                continue
            new = list(op.operands)
            for i in range(2):
                t = module.values[new[i]].ty
                if t.dtype != "f32":
                    continue
                down = module.add_op("stablehlo.convert", [new[i]], [TensorType(t.shape, self.low)],
                                     {"amp_cast": True}, before=oid)
                up = module.add_op("stablehlo.convert", [down.results[0]], [t], {"amp_cast": True}, before=oid)
                new[i] = up.results[0]
                created += 2
            op.operands = new
            op.attributes["compute_precision"] = self.low
            modified += 1
        return PassResult(self.name, created > 0 or modified > 0, 0, modified, created)


def calibrate_value_ranges(module: Module, num_samples: int) -> dict[int, float]:
    """formats.rs:115-182: a static bound on max |value| per SSA value.  Function arguments get
    the largest synthetic sample scale (0.5 + s / n, at least 0.8); constants their max |x|
    (at least 1e-5, from the device values); add / subtract add the bounds, multiply multiplies
    them, dot_general multiplies them by sqrt(K) (K = the lhs's last dimension), tanh gives 1,
    anything else passes its first operand's bound; every bound is at least 1e-5, and a missing
    operand bound counts as 1.  f64 throughout, as in the reference."""
    n = max(num_samples, 1)
    peak = 0.8
    for s_ in range(num_samples):
        peak = max(peak, 0.5 + s_ / n)
    max_abs: dict[int, float] = {a: peak for a in module.args}
    for oid in module.block_ops():
        op = module.ops[oid]
        if not op.results:
            continue
        res = op.results[0]
        if op.is_op("stablehlo", "constant"):
            ty = module.values[res].ty
            attr = op.attributes.get("value")
            vals = module.tensor_store.resolve_f32_attr(attr, ty.num_elements()) if attr is not None else None
            max_abs[res] = max(1e-5, ops.absmax(vals.reshape(-1).float())) if vals is not None else 1.0
            continue
        in0 = max_abs.get(op.operands[0], 1.0) if op.operands else 1.0
        in1 = max_abs.get(op.operands[1], 1.0) if len(op.operands) > 1 else 1.0
        if op.name in ("stablehlo.add", "stablehlo.subtract"):
            est = in0 + in1
        elif op.name == "stablehlo.multiply":
            est = in0 * in1
        elif op.name == "stablehlo.dot_general" and op.operands:
            shape = module.values[op.operands[0]].ty.shape
            k = float(max(int(shape[-1]), 1)) if shape and isinstance(shape[-1], int) else 4.0
            est = in0 * in1 * math.sqrt(k)
        elif op.name == "stablehlo.tanh":
            est = 1.0
        else:
            est = in0
        max_abs[res] = max(est, 1e-5)
    return max_abs


class CalibrateQuantizePass(Pass):
    """formats.rs:15-113 (`calibrate-quantize`, `quantize(scheme=w8a8|calibrate|static)`): for
    every dot_general / convolution not yet tagged, whose lhs is f32 / f16 / bf16, a
    `castforge.static_quantize` composite (scale = lhs bound / qmax, the calibrated bits) is
    inserted before the op on its lhs, and the op is tagged quant_mode = "w{b}a{b}_static",
    lhs_scale, rhs_scale, calibration_samples.  The inserted op runs on the GPU
    (castforge_hip_static_quantize) when the module is evaluated."""
    name = "calibrate-quantize"
    description = "Calibrates activation dynamic ranges and inserts static W8A8 quantization scales"

    def __init__(self, bits: int = 8, num_samples: int = 4):
        self.bits, self.num_samples = bits, num_samples

    def run(self, module: Module) -> PassResult:
        eff_bits, qmax = (4, 7.0) if self.bits == 4 else (8, 127.0)  # formats.rs:654-660
        ranges = calibrate_value_ranges(module, max(self.num_samples, 1))
        created = modified = 0
        for oid in module.block_ops():
            op = module.ops.get(oid)
            if op is None or "quant_mode" in op.attributes:
                continue
            if not (op.is_op("stablehlo", "dot_general") or op.is_op("stablehlo", "convolution")):
                continue
            if len(op.operands) < 2:
                continue
            lhs, rhs = op.operands[0], op.operands[1]
            lty = module.values[lhs].ty
            if not isinstance(lty.dtype, str) or lty.dtype not in ("f32", "f16", "bf16"):
                continue
            lhs_scale = max(ranges.get(lhs, 1.0), 1e-5) / qmax
            rhs_scale = max(ranges.get(rhs, 1.0), 1e-5) / qmax
            q = module.add_op("stablehlo.composite", [lhs], [lty],
                              {"name": "castforge.static_quantize", "decomposition": "static_quantize_impl",
                               "scale": lhs_scale, "bits": eff_bits}, before=oid)
            op.operands[0] = q.results[0]
            op.attributes["quant_mode"] = f"w{eff_bits}a{eff_bits}_static"
            op.attributes["lhs_scale"] = lhs_scale
            op.attributes["rhs_scale"] = rhs_scale
            op.attributes["calibration_samples"] = int(self.num_samples)
            created += 1
            modified += 1
        return PassResult(self.name, created > 0 or modified > 0, 0, modified, created)


def _mark_users(module: Module, vid: int, attrs: dict) -> None:
    for uop in module.ops.values():
        if vid in uop.operands:
            uop.attributes.update(attrs)


def _hadamard_block(block_size: int, k: int) -> int:
    """formats.rs:303: next_power_of_two(block_size).min(k).max(2)."""
    p = 1
    while p < block_size:
        p <<= 1
    return max(min(p, k), 2)


class RotateHadamardPass(Pass):
    """formats.rs:230-343 (`rotate-hadamard`): every 2-D constant [k, n] not yet tagged
    castforge.hadamard_rotated, with k >= 2 and n > 0, is rotated down its columns in blocks
    of b = next_power_of_two(block_size).min(k).max(2) when k % b == 0 (on the GPU,
    castforge_hip_rotate_hadamard, bit-exact), and is tagged either way; its users get
    castforge.hadamard_rotated and castforge.hadamard_block = b.  A b that is not a power of
    two (k below the block and not a power of two) makes the reference's butterfly index past
    its buffer and panic; here it raises ValueError."""
    name = "rotate-hadamard"
    description = "Applies orthogonal Walsh-Hadamard rotation (QuaRot/SpinQuant) to suppress outliers"

    def __init__(self, block_size: int = 4):
        self.block_size = block_size

    def run(self, module: Module) -> PassResult:
        modified = 0
        for oid, op in list(_const_ops(module)):
            if not op.results or op.attributes.get("castforge.hadamard_rotated") is True:
                continue
            res = op.results[0]
            ty = module.values[res].ty
            if len(ty.shape) != 2:
                continue
            k, n = int(ty.shape[0]), int(ty.shape[1])
            if k < 2 or n == 0:
                continue
            attr = op.attributes.get("value")
            if attr is None:
                continue
            vals = module.tensor_store.resolve_f32_attr(attr, k * n)
            if vals is None:
                continue
            b = _hadamard_block(self.block_size, k)
            w = vals.reshape(k, n).float().contiguous()
            if k % b == 0:
                if b & (b - 1):
                    raise ValueError(f"rotate-hadamard: block {b} (k = {k}) is not a power of two; the "
                                     f"reference's butterfly indexes past its buffer for it")
                w = ops.rotate_hadamard(w, b, 0)
            v = module.values[res]
            op.attributes["value"] = module.tensor_store.update_f32_constant(v.ssa_name, attr, ty, w.reshape(-1))
            op.attributes["castforge.hadamard_rotated"] = True
            _mark_users(module, res, {"castforge.hadamard_rotated": True, "castforge.hadamard_block": b})
            modified += 1
        return PassResult(self.name, modified > 0, 0, modified, 0)


class SmoothQuantizePass(Pass):
    """schemes.rs:155-298 (`smooth-quantize`, `quantize(scheme=smoothquant|smooth)`): alpha
    clamped to [0.05, 0.95]; for every constant of >= 2 elements, with act_max its calibrated
    bound (calibrate_value_ranges, computed once before any rewrite) and w_max its max |w| (at
    least 1e-5), the per-tensor scalars s and e (castforge_hip_smoothquant_scales, the C
    library's powf) and the fake quantization (q e) / s of every element
    (castforge_hip_smoothquant) replace its values; it and its users are tagged
    castforge.quant_scheme = "smoothquant", castforge.smoothquant_alpha, castforge.quant_bits."""
    name = "smooth-quantize"
    description = "Migrates activation outlier difficulty into weights via SmoothQuant alpha scaling"

    def __init__(self, bits: int = 8, alpha: float = 0.5, num_samples: int = 4):
        self.bits, self.alpha, self.num_samples = bits, alpha, num_samples

    def run(self, module: Module) -> PassResult:
        a = np.float32(self.alpha)
        alpha = a if a != a else np.float32(min(max(a, np.float32(0.05)), np.float32(0.95)))
        bits = 4 if self.bits == 4 else 8  # formats.rs:654-660
        ranges = calibrate_value_ranges(module, max(self.num_samples, 1))
        modified = 0
        tags = {"castforge.quant_scheme": "smoothquant", "castforge.smoothquant_alpha": float(alpha),
                "castforge.quant_bits": bits}
        for oid, op in list(_const_ops(module)):
            if not op.results:
                continue
            res = op.results[0]
            ty = module.values[res].ty
            n = ty.num_elements()
            if n < 2:
                continue
            attr = op.attributes.get("value")
            if attr is None:
                continue
            vals = module.tensor_store.resolve_f32_attr(attr, n)
            if vals is None:
                continue
            vals = vals.reshape(-1).float().contiguous()
            act_max = float(np.float32(ranges.get(res, 1.0)))
            w_max = max(float(np.float32(ops.absmax(vals))), float(np.float32(1e-5)))
            sc, eq = ops.smoothquant_scales(act_max, w_max, float(alpha), bits)
            new = ops.smoothquant(vals, sc, eq, bits)
            if isinstance(attr, TensorRef):
                e = module.tensor_store.get(attr.key)
                if e is not None:
                    module.tensor_store.insert(TensorEntry(attr.key, e.ty, F32Data(new)))
            else:
                op.attributes["value"] = Dense(new.reshape(ty.shape))
            op.attributes.update(tags)
            _mark_users(module, res, tags)
            modified += 1
        return PassResult("quantize", modified > 0, 0, modified, 0)


class QuantizePass(Pass):
    """schemes.rs:85-153 dispatch."""
    name = "quantize"
    description = "Unified quantization & precision (weight|awq|fp8|nvfp4|f16|bf16|w8a8|smoothquant|hadamard)"

    def __init__(self, scheme="weight", bits=8, min_elements=2, group_size=32, awq_salient=True,
                 salient_ratio=0.01, format="e4m3", mxfp8=True, block_size=32, hadamard=False,
                 round=None, granularity="tensor", group_given=False, block_given=False, samples=4,
                 alpha=0.5, hadamard_axis="0"):
        self.__dict__.update(locals())
        del self.__dict__["self"]

    _UNSUPPORTED = ("fp4", "mxfp4", "nvfp4", "e2m1", "qat", "qat_ste", "ste")

    def run(self, module: Module) -> PassResult:
        s = self.scheme.lower()
        # rejected before any step (e.g. hadamard=true's rotation) touches the module
        if s in self._UNSUPPORTED:
            raise ValueError(f"quantize: scheme `{s}` is not part of the HIP quantized-weight path")
        if s in ("f16", "bf16", "mixed_precision", "amp"):
            tgt = "bf16" if s == "bf16" or self.format.lower() == "bf16" else "f16"
            return LowerMixedPrecisionPass(tgt).run(module).with_name(self.name)
        if s in ("hadamard", "quarot", "spinquant"):
            return RotateHadamardPass(max(self.block_size, 2)).run(module).with_name(self.name)
        steps = []
        fused_k = self.hadamard and self.hadamard_axis in ("1", "k") and s in ("int4_asym", "int4g")
        if self.hadamard and not fused_k:
            steps.append(RotateHadamardPass(max(self.block_size, 2)).run(module))
        if fused_k:
            # this build's K-axis rotation of packed [N, K] weights, fused into the INT4g kernel
            steps += QuantizePackedPass("int4_asym", self.group_size if self.group_given else 128,
                                        min_elements=self.min_elements,
                                        hadamard=max(self.block_size, 2)).run_steps(module)
            return PassResult.aggregate(self.name, steps)
        if s in ("groupwise", "awq", "gptq"):
            r = QuantizeGroupwisePass(self.bits, self.group_size, self.awq_salient or s == "awq",
                                      self.salient_ratio).run(module)
        elif s in ("fp8", "mxfp8", "e4m3", "e5m2"):
            r = QuantizeFp8Pass(self.format, self.mxfp8, self.block_size).run(module)
        elif s in ("int8_channel", "per_channel"):
            r = QuantizePackedPass("int8_channel", 0, self.round or "half_even", self.min_elements).run(module)
        elif s in ("int4_asym", "int4g"):
            r = QuantizePackedPass("int4_asym", self.group_size if self.group_given else 128,
                                   min_elements=self.min_elements).run(module)
        elif s == "nf4":
            r = QuantizePackedPass("nf4", self.block_size if self.block_given else 64,
                                   min_elements=self.min_elements).run(module)
        elif s in ("fp8_row", "w8a8_fp8"):
            r = QuantizePackedPass("fp8_row", min_elements=self.min_elements).run(module)
        elif s in ("w8a8", "calibrate", "static"):
            r = CalibrateQuantizePass(self.bits, self.samples).run(module)
        elif s in ("smoothquant", "smooth"):
            r = SmoothQuantizePass(self.bits, self.alpha, self.samples).run(module)
        elif self.granularity in ("channel", "per_channel"):
            r = QuantizePackedPass("int8_channel", 0, self.round or "half_even", self.min_elements).run(module)
        else:
            r = QuantizeWeightsPass(self.bits, self.min_elements, self.round or "half_away").run(module)
        return PassResult.aggregate(self.name, steps + [r])


def _quantize_factory(opts: dict[str, str]) -> QuantizePass:
    """registry/families.rs:93-183."""
    scheme = _first(opts, "scheme", "mode", "dtype")
    if scheme is None:
        if "alpha" in opts:
            scheme = "smoothquant"
        elif "salient_ratio" in opts:
            scheme = "awq"
        elif "group_size" in opts or "awq_salient" in opts:
            scheme = "groupwise"
        elif "format" in opts or "mxfp8" in opts:
            scheme = "fp8"
        elif "samples" in opts or "num_samples" in opts:
            scheme = "w8a8"
        elif "block_size" in opts and "bits" not in opts:
            scheme = "hadamard"
        else:
            scheme = "weight"
    four = ("groupwise", "awq", "gptq", "fp4", "mxfp4", "nvfp4", "int4_asym", "int4g", "nf4")
    default_bits = 4 if scheme in four else 8
    group = _first(opts, "group_size", "group")
    block = _first(opts, "block_size", "size")
    rnd = opts.get("round")
    if rnd is not None and rnd not in ("half_away", "half_even"):
        raise ValueError(f"quantize: round must be half_away or half_even (got `{rnd}`)")
    return QuantizePass(
        scheme=scheme,
        bits=_u8(opts.get("bits"), default_bits),
        min_elements=_usize(opts.get("min_elements"), 2),
        group_size=_usize(group, 32),
        awq_salient=opts.get("awq_salient", "true") != "false",
        salient_ratio=_f32(opts.get("salient_ratio"), 0.01),
        format=_first(opts, "format", "dtype") or "e4m3",
        mxfp8=opts.get("mxfp8", "true") != "false",
        block_size=_usize(block, 32),
        hadamard=opts.get("hadamard") in ("true", "1"),
        round=rnd,
        granularity=opts.get("granularity", "tensor"),
        group_given=group is not None and _usize(group, -1) > 0,
        block_given=block is not None and _usize(block, -1) > 0,
        samples=_usize(_first(opts, "samples", "num_samples"), 4),
        alpha=_f32(opts.get("alpha"), 0.5),
        hadamard_axis=opts.get("hadamard_axis", "0"),
    )


# ---------------------------------------------------------------------------- fusion ----
class FuseDequantMatmulPass(Pass):
    """epilogue.rs:10-94 + gemm.rs:102-127: dot_general(lhs, uniform_dequantize(wq)) becomes
    `stablehlo.composite {name = "castforge.fused_qmatmul"}(lhs, wq)` with the type's scale /
    zero point and packed_rhs; a fused_matmul_epilogue composite is upgraded likewise; the
    dead dequantize ops are removed."""
    name = "fuse-dequant-matmul"
    description = "Fuses uniform_dequantize + dot_general into on-the-fly quantized GEMM (fused_qmatmul)"

    def _match(self, module: Module, vid: int):
        v = module.values.get(vid)
        if v is None or v.op is None:
            return None
        d = module.ops[v.op]
        if not d.is_op("stablehlo", "uniform_dequantize") or len(d.operands) != 1:
            return None
        wq = d.operands[0]
        dt = module.values[wq].ty.dtype
        if isinstance(dt, QuantUniform):
            try:
                scale = float(dt.scale)
            except ValueError:
                scale = 1.0
            return wq, scale, dt.zero_point
        return wq, 1.0, 0

    def run(self, module: Module) -> PassResult:
        created = 0
        for oid in module.block_ops():
            op = module.ops[oid]
            if op.is_op("stablehlo", "dot_general") and len(op.operands) == 2:
                m = self._match(module, op.operands[1])
                if m is None:
                    continue
                wq, scale, zp = m
                packed = op.attributes.get("rhs_contracting_dimensions") == [1]
                op.name = "stablehlo.composite"
                op.operands = [op.operands[0], wq]
                op.attributes = {"name": "castforge.fused_qmatmul", "decomposition": "@fused_qmatmul_impl",
                                 "scale": scale, "zero_point": zp}
                if packed:
                    op.attributes["packed_rhs"] = True
                created += 1
            elif (op.is_op("stablehlo", "composite") and op.attributes.get("name") == "castforge.fused_matmul_epilogue"
                  and len(op.operands) >= 3):
                m = self._match(module, op.operands[1])
                if m is None:
                    continue
                wq, scale, zp = m
                op.operands[1] = wq
                op.attributes.update({"name": "castforge.fused_qmatmul", "decomposition": "@fused_qmatmul_impl",
                                      "scale": scale, "zero_point": zp})
                created += 1
        removed = module.dce() if created else 0
        return PassResult(self.name, created > 0 or removed > 0, removed, 0, created)


class FuseGemmPass(Pass):
    """registry/families.rs:362-371 `fuse-gemm(kind=...)`: only the dequant fusion is on this path."""
    name = "fuse-gemm"
    description = "Unified GEMM fusion (horizontal QKV/MLP dot, dequant+GEMM, and GEMM+bias/act/res)"

    def __init__(self, kind="all"):
        if kind not in ("dequant", "all"):
            raise ValueError(f"fuse-gemm: kind `{kind}` is not part of the HIP quantized-weight path "
                             "(supported: dequant)")
        self.kind = kind

    def run(self, module: Module) -> PassResult:
        return FuseDequantMatmulPass().run(module).with_name(self.name)


class PackWeightsPass(Pass):
    """fold.rs:456-591: a dot_general with contracting [1] x [0] whose rhs is a 2-D f32
    constant [K, N] gets that constant transposed to [N, K] (on the GPU) and packed_rhs."""
    name = "pack-weights"
    description = "Pre-packs 2D constant RHS weights from [K, N] to [N, K] for unit-stride SIMD MatMul"

    def run(self, module: Module) -> PassResult:
        modified = 0
        packed = set()
        for oid in module.block_ops():
            op = module.ops[oid]
            is_cand = (op.is_op("stablehlo", "dot_general") and op.attributes.get("lhs_contracting_dimensions", [1]) == [1]
                       and op.attributes.get("rhs_contracting_dimensions", [0]) == [0])
            if (op.is_op("stablehlo", "composite") and op.attributes.get("name") == "castforge.fused_matmul_epilogue"
                    and len(op.operands) >= 3):
                is_cand = op.attributes.get("rhs_contracting_dimensions", [0]) == [0]
            if not is_cand or len(op.operands) < 2:
                continue
            rhs = op.operands[1]
            v = module.values[rhs]
            if v.op is None:
                continue
            wop = module.ops[v.op]
            if v.op not in packed:
                if not wop.is_op("stablehlo", "constant"):
                    continue
                if v.ty.dtype != "f32" or len(v.ty.shape) != 2:
                    continue
                k, n = v.ty.shape
                attr = wop.attributes.get("value")
                vals = module.tensor_store.resolve_f32_attr(attr, k * n) if attr is not None else None
                if vals is None:
                    continue
                pt = ops.transpose2d(vals.reshape(k, n).contiguous())
                nty = TensorType((n, k), "f32")
                wop.attributes["value"] = module.tensor_store.update_f32_constant(v.ssa_name, attr, nty, pt)
                v.ty = nty
                packed.add(v.op)
                modified += 1
            op.attributes["lhs_contracting_dimensions"] = [1]
            op.attributes["rhs_contracting_dimensions"] = [1]
            op.attributes["packed_rhs"] = True
            modified += 1
        return PassResult(self.name, modified > 0, 0, modified, 0)


def default_registry() -> PassRegistry:
    reg = PassRegistry()
    reg.register("quantize", QuantizePass.description, _quantize_factory)
    reg.register("quantize-weights", QuantizeWeightsPass.description,
                 lambda o: QuantizeWeightsPass(_u8(o.get("bits"), 8), _usize(o.get("min_elements"), 2),
                                               o.get("round", "half_away")))
    reg.register("quantize-groupwise", QuantizeGroupwisePass.description,
                 lambda o: QuantizeGroupwisePass(_u8(o.get("bits"), 4), _usize(_first(o, "group_size", "group"), 32),
                                                 o.get("awq_salient", "true") != "false",
                                                 _f32(o.get("salient_ratio"), 0.01)))
    reg.register("quantize-fp8", QuantizeFp8Pass.description,
                 lambda o: QuantizeFp8Pass(_first(o, "format", "dtype") or "e4m3", o.get("mxfp8", "true") != "false",
                                           _usize(o.get("block_size"), 32)))
    reg.register("lower-mixed-precision", LowerMixedPrecisionPass.description,
                 lambda o: LowerMixedPrecisionPass("bf16" if (_first(o, "dtype", "format") or "").lower() == "bf16"
                                                   else "f16"))
    reg.register("fuse-gemm", FuseGemmPass.description, lambda o: FuseGemmPass(o.get("kind", "all")))
    reg.register("fuse-dequant-matmul", FuseDequantMatmulPass.description, lambda o: FuseDequantMatmulPass())
    reg.register("pack-weights", PackWeightsPass.description, lambda o: PackWeightsPass())
    reg.register("rotate-hadamard", RotateHadamardPass.description,
                 lambda o: RotateHadamardPass(_usize(_first(o, "block_size", "size"), 4)))
    reg.register("smooth-quantize", SmoothQuantizePass.description,
                 lambda o: SmoothQuantizePass(_u8(o.get("bits"), 8), _f32(o.get("alpha"), 0.5),
                                              _usize(_first(o, "samples", "num_samples"), 4)))
    reg.register("calibrate-quantize", "Profile-guided static W8A8/W4A8 calibration and quantization",
                 lambda o: CalibrateQuantizePass(_u8(o.get("bits"), 8),
                                                 _usize(_first(o, "samples", "num_samples"), 4)))
    return reg
