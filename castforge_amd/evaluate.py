"""Evaluation of a quantized module on the GPU: the reference interpreter's semantics for the
ops of this path (codegen/eval.rs:52-165, 296-347, 674-676, 1145-1179, 1465-1507), dispatched to
libcastforge_hip.so.

  stablehlo.constant         f32 values; a `!quant.uniform` constant evaluates to
                             (q - zp) * f32(scale string) as eval.rs:303-318 does (the scale
                             goes through the printed 6-decimal string); a packed constant
                             evaluates to its dequantized f32 values
  stablehlo.uniform_dequantize  the same dequantization (eval.rs:324-343)
  stablehlo.convert          a copy (eval.rs:674-676)
  stablehlo.dot_general      eval_matmul_2d, bit-identical on the GPU (castforge_hip_matmul_f32);
                             with batching dimensions or an operand of rank > 2, eval_dot_general's
                             flat [batch, m, k] x [batch, (n, k) | (k, n)] form (eval.rs:1509-1604)
                             as one such matmul per batch
  castforge.fused_qmatmul    the dequant-fused GEMV / GEMM kernels, then the epilogue
                             (eval.rs:1145-1179)
  castforge.fused_matmul_epilogue  f32 matmul + epilogue

`activations`: "f32" keeps the interpreter's f32 operands everywhere, so a fused_qmatmul is
evaluated as dequantize + eval_matmul_2d; "bf16" (the W4A16 / W8A16 path this library
accelerates) rounds every matmul's activations to bf16 (RNE) and runs fused_qmatmul on the
packed-weight kernels.  Either way both sides of `verify_module_numerics` see the same operands.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import ops
from .ir import Module, QuantPacked, QuantUniform
from .tensor_store import QuantizedPacked, dequantize_packed


@dataclass
class NumericVerificationReport:
    passed: bool
    max_abs_diff: float
    tolerance: float
    num_outputs_checked: int


def generate_synthetic_inputs(module: Module, device) -> list[torch.Tensor]:
    """eval.rs:32-44: argument a, element i -> (((i * 7 + a * 13 + 3) % 19) - 9) * 0.1 (f32)."""
    out = []
    for a, vid in enumerate(module.args):
        ty = module.values[vid].ty
        n = ty.num_elements()
        i = torch.arange(n, dtype=torch.int64)
        raw = ((i * 7 + a * 13 + 3) % 19).to(torch.float32)
        vals = (raw - torch.tensor(9.0, dtype=torch.float32)) * torch.tensor(0.1, dtype=torch.float32)
        out.append(vals.reshape(ty.shape).to(device))
    return out


def _scale_f32(dt: QuantUniform) -> float:
    try:
        return float(torch.tensor(float(dt.scale), dtype=torch.float32))
    except ValueError:
        return 1.0


def _dequant_uniform(q: torch.Tensor, dt: QuantUniform) -> torch.Tensor:
    if dt.zero_point != 0:
        raise NotImplementedError("uniform_dequantize with a non-zero zero point has no HIP kernel")
    s = torch.tensor([_scale_f32(dt)], dtype=torch.float32, device=q.device)
    return ops.dequantize_int8(q.reshape(1, -1).contiguous(), s, "tensor").reshape(q.shape)


def _as2d(t: torch.Tensor, shape) -> torch.Tensor:
    return t.reshape(shape[0] if len(shape) > 0 else 1, -1)


class _Evaluator:
    def __init__(self, module: Module, activations: str):
        if activations not in ("f32", "bf16"):
            raise ValueError("activations must be 'f32' or 'bf16'")
        self.m, self.act = module, activations
        self.env: dict[int, torch.Tensor] = {}
        self.q_env: dict[int, object] = {}

    def _act(self, x: torch.Tensor) -> torch.Tensor:
        """Activations as the matmul sees them (f32 tensor)."""
        if self.act == "bf16":
            return ops.to_f32(ops.to_bf16(x.contiguous()))
        return x

    def _matmul(self, lhs: int, rhs_vals: torch.Tensor, rhs_shape, packed: bool) -> torch.Tensor:
        a = self._act(_as2d(self.env[lhs], self.m.values[lhs].ty.shape).contiguous())
        b = rhs_vals.reshape(rhs_shape).contiguous()
        return ops.matmul_f32(a, b, packed)

    def _dot_general(self, op, ty) -> torch.Tensor:
        """eval.rs:934-952 + eval_dot_general (eval.rs:1509-1604).

        Without batching dimensions and with both operands of rank <= 2 this is
        eval_matmul_2d, packed when the rhs is 2-D and contracts its last dimension.  Otherwise
        the reference reads both operands flat: batch = product of the lhs batching dimensions,
        k = product of the lhs contracting dimensions, m = |lhs| / (batch k), n = |rhs| / (batch k);
        lhs as [batch, m, k] and rhs as [batch, n, k] when its last contracting dimension is its
        last dimension, else [batch, k, n]; out [batch, m, n], each output an f32 sum over kk
        in order -- per batch exactly eval_matmul_2d's loop, which castforge_hip_matmul_f32
        reproduces bit for bit.  Operands that do not factor that way (the reference would read
        zeros past their ends) are rejected."""
        lhs, rhs = op.operands[0], op.operands[1]
        ls, rs = tuple(self.m.values[lhs].ty.shape), tuple(self.m.values[rhs].ty.shape)
        at = op.attributes
        lb = list(at.get("lhs_batching_dimensions") or [])
        rb = list(at.get("rhs_batching_dimensions") or [])
        lc = list(at.get("lhs_contracting_dimensions") or [])
        rc = list(at.get("rhs_contracting_dimensions") or [])
        if not lb and not rb and len(ls) <= 2 and len(rs) <= 2:
            if "rhs_contracting_dimensions" in at:
                packed = len(rs) == 2 and bool(rc) and rc[-1] == len(rs) - 1
            else:
                packed = bool(at.get("packed_rhs", False))
            return self._matmul(lhs, self.env[rhs], rs, packed).reshape(ty.shape)

        def prod(v):
            r = 1
            for d in v:
                r *= int(d)
            return r

        def dims_of(shape, axes, what):
            for ax in axes:
                if not 0 <= int(ax) < len(shape):
                    raise ValueError(f"dot_general: {what} dimension {ax} is outside an operand of rank {len(shape)}")
            return [int(shape[int(ax)]) for ax in axes]

        batch = max(prod(dims_of(ls, lb, "lhs batching")), 1)
        k = max(prod(dims_of(ls, lc, "lhs contracting")), 1)
        dims_of(rs, rc, "rhs contracting")
        lt, rt = max(prod(ls), 1), max(prod(rs), 1)
        mm = max(lt // max(batch * k, 1), 1)
        nn = max(rt // max(batch * k, 1), 1)
        if lt != batch * mm * k or rt != batch * k * nn or prod(ty.shape) != batch * mm * nn:
            raise ValueError(
                f"dot_general: lhs {ls} and rhs {rs} (batching {lb} x {rb}, contracting {lc} x {rc}) do not "
                f"factor as [batch={batch}, m, k={k}] x [batch, k, n] with a result of {batch * mm * nn} elements "
                f"(result type {tuple(ty.shape)}); the reference evaluator would read zeros past the operands")
        contract_last = bool(rc) and rc[-1] + 1 == len(rs)
        a = self._act(self.env[lhs].reshape(batch, mm, k).contiguous())
        b = self.env[rhs].reshape((batch, nn, k) if contract_last else (batch, k, nn)).contiguous()
        out = torch.empty((batch, mm, nn), dtype=torch.float32, device=a.device)
        for i in range(batch):
            out[i] = ops.matmul_f32(a[i], b[i], contract_last)
        return out.reshape(ty.shape)

    def _fused(self, op) -> torch.Tensor:
        lhs, wq = op.operands[0], op.operands[1]
        wty = self.m.values[wq].ty
        packed = bool(op.attributes.get("packed_rhs", False))
        if self.act == "f32":
            return self._matmul(lhs, self.env[wq], wty.shape, packed)
        x = ops.to_bf16(_as2d(self.env[lhs], self.m.values[lhs].ty.shape).contiguous())
        dt = wty.dtype
        if isinstance(dt, QuantUniform):
            q = self.q_env[wq]
            codes = q.reshape(wty.shape)
            if not packed:
                codes = ops.transpose2d(codes.contiguous())  # [K, N] -> [N, K] i8 codes
            if dt.zero_point != 0:
                raise NotImplementedError("fused_qmatmul with a non-zero zero point has no HIP kernel")
            s = torch.tensor([_scale_f32(dt)], dtype=torch.float32, device=x.device)
            return ops.gemm_w8a16(x, codes.contiguous(), s, "tensor", torch.float32)
        if isinstance(dt, QuantPacked):
            b: QuantizedPacked = self.q_env[wq]
            if not packed:
                raise ValueError("a packed-format weight is [N, K]: fused_qmatmul needs packed_rhs "
                                 "(run pack-weights before quantize)")
            n, k = b.shape
            if b.format == "int4_asym":
                return ops.gemm_w4a16(x, ops.Int4Packed(b.codes, b.scales, b.zeros, n, k, b.group), torch.float32)
            if b.format == "nf4":
                return ops.gemm_nf4(x, ops.Nf4Packed(b.codes, b.scales, n, k, b.group), torch.float32)
            if b.format == "int8_channel":
                return ops.gemm_w8a16(x, b.codes, b.scales, "channel", torch.float32)
            if b.format == "fp8_row":
                qa, sa = ops.quantize_fp8(x)  # per-token dynamic E4M3 activations (W8A8)
                # f16-MFMA form: stays within the f32 evaluator's tolerance on any input
                return ops.gemm_fp8(qa, sa, b.codes, b.scales, out_dtype=torch.float32, exact=True)
            if b.format in ("gguf_q4_0", "gguf_q8_0"):
                ty = ops.GGML_TYPES["Q4_0" if b.format == "gguf_q4_0" else "Q8_0"]
                return ops.gemm_gguf(x, ops.GgufPacked(ty, b.codes, b.scales, n, k), torch.float32)
        # an f32 weight (not quantized): plain matmul
        return self._matmul(lhs, self.env[wq], wty.shape, packed)

    def _epilogue(self, op, mm: torch.Tensor) -> torch.Tensor:
        if len(op.operands) < 3:
            return mm
        bias = self.env[op.operands[2]].reshape(-1).contiguous()
        z = self.env[op.operands[3]].reshape(-1).contiguous() if len(op.operands) > 3 else None
        return ops.qmatmul_epilogue(mm.contiguous(), bias, z, op.attributes.get("epilogue", "bias"))

    def run(self, inputs) -> list[torch.Tensor]:
        m = self.m
        if len(inputs) != len(m.args):
            raise ValueError(f"expected {len(m.args)} inputs, got {len(inputs)}")
        for vid, x in zip(m.args, inputs):
            self.env[vid] = x.float() if x.dtype != torch.float32 else x
        for oid in m.block_ops():
            op = m.ops[oid]
            if not op.results:
                continue
            res = op.results[0]
            ty = m.values[res].ty
            if op.is_op("stablehlo", "constant"):
                attr = op.attributes.get("value")
                if isinstance(ty.dtype, QuantUniform):
                    q = m.tensor_store.resolve_i8_attr(attr, ty.num_elements())
                    if q is None:
                        q = torch.zeros(ty.shape, dtype=torch.int8, device=self._device())
                    self.q_env[res] = q
                    self.env[res] = _dequant_uniform(q, ty.dtype)
                elif isinstance(ty.dtype, QuantPacked):
                    b = m.tensor_store.get(attr.key).backing
                    self.q_env[res] = b
                    self.env[res] = dequantize_packed(b)
                else:
                    v = m.tensor_store.resolve_f32_attr(attr, ty.num_elements())
                    if v is None:
                        v = torch.zeros(ty.num_elements(), dtype=torch.float32, device=self._device())
                    self.env[res] = v.reshape(ty.shape)
            elif op.is_op("stablehlo", "uniform_dequantize"):
                src = op.operands[0]
                sdt = m.values[src].ty.dtype
                if isinstance(sdt, QuantUniform):
                    self.env[res] = _dequant_uniform(self.q_env[src], sdt)
                else:
                    self.env[res] = self.env[src]
            elif op.is_op("stablehlo", "convert"):
                self.env[res] = self.env[op.operands[0]]
            elif op.is_op("stablehlo", "dot_general"):
                self.env[res] = self._dot_general(op, ty)
            elif op.is_op("stablehlo", "composite") and op.attributes.get("name") == "castforge.fused_qmatmul":
                self.env[res] = self._epilogue(op, self._fused(op)).reshape(ty.shape)
            elif op.is_op("stablehlo", "composite") and op.attributes.get("name") == "castforge.static_quantize":
                # eval.rs:1369-1382: a positive float scale attribute as f32, else 1/127; bits
                # defaults to 8
                sc = op.attributes.get("scale")
                if isinstance(sc, float) and not isinstance(sc, bool) and sc > 0.0:
                    scf = float(np.float32(sc))
                else:
                    scf = float(np.float32(1.0) / np.float32(127.0))
                bits = op.attributes.get("bits", 8)
                bits = bits if isinstance(bits, int) and not isinstance(bits, bool) else 8
                self.env[res] = ops.static_quantize(self.env[op.operands[0]].float(), scf, bits).reshape(ty.shape)
            elif op.is_op("stablehlo", "composite") and op.attributes.get("name") == "castforge.fused_matmul_epilogue":
                rhs = op.operands[1]
                mm = self._matmul(op.operands[0], self.env[rhs], m.values[rhs].ty.shape,
                                  bool(op.attributes.get("packed_rhs", False)))
                self.env[res] = self._epilogue(op, mm).reshape(ty.shape)
            else:
                raise NotImplementedError(f"op `{op.name}` is outside the quantized-weight path")
        return [self.env[r] for r in m.results]

    def _device(self):
        for t in self.env.values():
            return t.device
        return torch.device("cuda")


def evaluate_module(module: Module, inputs, activations: str = "f32") -> list[torch.Tensor]:
    """eval.rs:159-165: evaluates the function with the given device inputs."""
    return _Evaluator(module, activations).run(inputs)


def compare_output_tensors(a, b, tolerance: float) -> NumericVerificationReport:
    """eval.rs:72-109."""
    if len(a) != len(b):
        raise ValueError(f"Output count mismatch: before={len(a)} vs after={len(b)}")
    mx, n = 0.0, 0
    for x, y in zip(a, b):
        if x.numel() != y.numel():
            raise ValueError(f"Output tensor shape mismatch: before len={x.numel()} vs after len={y.numel()}")
        if x.numel():
            mx = max(mx, float((x.reshape(-1).float() - y.reshape(-1).float()).abs().max().item()))
        n += x.numel()
    return NumericVerificationReport(mx <= tolerance, mx, tolerance, n)


def verify_module_numerics(before: Module, after: Module, tolerance: float, device=None,
                           activations: str = "f32") -> NumericVerificationReport:
    """eval.rs:57-66: both modules on the same deterministic synthetic inputs."""
    device = device or torch.device("cuda")
    inputs = generate_synthetic_inputs(before, device)
    return compare_output_tensors(evaluate_module(before, inputs, activations),
                                  evaluate_module(after, inputs, activations), tolerance)
