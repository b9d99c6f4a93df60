"""UOp graph -> tensor-plan wire format (the reference's _gpu_plan).

build_gpu_execution_plan (_gpu_plan.py:285-638): fuse unless custom ops are
allowed, refuse CUSTOM, then one step per toposorted node with
value_id = step = topo index, input_ids by the same index, the node's
shape / dtype / arg, and one buffer record per value
{bytes, first_step, last_step (last reader), materialize: node is root};
peak_live_bytes is the largest sum of bytes over values live at a step.

build_gpu_execution_submission (:641-666) adds the semantic side table: one
dense-permutation-view-copy request per PERMUTE (float32, source rank 2 or 3,
positive static extents as canonical decimal strings, axes an exact
permutation), and plan_summary() erases each PERMUTE's legacy arg to None
(:252-258).

Differences from the reference (the executor in libbghip lowers them):
CMP, WHERE, CONST, SLICE and CAUSAL_MASK are accepted, as are rank > 2
MATMULs and float16 / bfloat16 / bool values; the reference refuses WHERE
here (:561-566) and its executor refuses the rest.
"""
from __future__ import annotations

import json
import math
from dataclasses import dataclass
from typing import Any, Dict, List, Tuple

from .fusion import fuse
from .ir import (
    CONV_OPS,
    OP_ADD, OP_BROADCAST_TO, OP_BUFFER, OP_CAST, OP_CMP, OP_CONST, OP_CUSTOM, OP_DIV, OP_EXP,
    OP_FUSED_ELEMENTWISE, OP_FUSED_SOFTMAX, OP_LAYER_NORM, OP_LOAD, OP_LOG, OP_MATMUL, OP_MUL, OP_NEG,
    OP_CAUSAL_MASK, OP_PERMUTE, OP_REDUCE, OP_RESHAPE, OP_SLICE, OP_WHERE, UOp, toposort,
)
from ..errors import JitNotImplementedError

TENSOR_PLAN_SEMANTIC_REQUEST_SCHEMA = "browsergrad.jit.tensor-plan-semantic-requests"
TENSOR_PLAN_SEMANTIC_REQUEST_VERSION = (1, 0)
DENSE_PERMUTATION_VIEW_COPY_REQUEST = "dense-permutation-view-copy"
_WIRE_I64_MAX = (1 << 63) - 1

_DTYPE_BYTES = {"float32": 4, "float16": 2, "bfloat16": 2, "float64": 8, "int64": 8, "int32": 4, "bool": 1}

# OP_CAUSAL_MASK (extension, ir.py): the plan builder of the HIP route
# writes it in place of a LOAD of a causal-mask buffer, so the executor can
# recognise masked attention without reading the mask.

PLAN_OPS = frozenset({
    OP_BUFFER, OP_LOAD, OP_CONST, OP_CAST, OP_ADD, OP_MUL, OP_DIV, OP_NEG, OP_EXP, OP_LOG, OP_CMP, OP_WHERE,
    OP_MATMUL, OP_REDUCE, OP_RESHAPE, OP_PERMUTE, OP_BROADCAST_TO, OP_LAYER_NORM, OP_FUSED_ELEMENTWISE,
    OP_FUSED_SOFTMAX, OP_SLICE, OP_CAUSAL_MASK,
}) | CONV_OPS


class GpuPlanUnsupported(JitNotImplementedError):
    """A graph that cannot enter the tensor plan."""


@dataclass(frozen=True)
class PlanStep:
    step: int
    value_id: int
    op: str
    input_ids: Tuple[int, ...]
    shape: Tuple[int, ...]
    dtype: str
    arg: Any


@dataclass(frozen=True)
class PlanBuffer:
    value_id: int
    op: str
    shape: Tuple[int, ...]
    dtype: str
    bytes: int
    first_step: int
    last_step: int
    materialize: bool


def _jsonable(arg: Any) -> Any:
    if isinstance(arg, dict):
        return {str(k): _jsonable(v) for k, v in arg.items()}
    if isinstance(arg, (tuple, list)):
        return [_jsonable(v) for v in arg]
    if isinstance(arg, float) and not math.isfinite(arg):
        return arg  # json.dumps writes Infinity / -Infinity / NaN; the executor reads them
    return arg


@dataclass(frozen=True)
class GpuExecutionPlan:
    steps: Tuple[PlanStep, ...]
    buffers: Tuple[PlanBuffer, ...]
    root_id: int
    materialization_boundary: str
    peak_live_bytes: int
    has_custom_ops: bool

    def summary(self) -> Dict[str, Any]:
        return {
            "step_count": len(self.steps),
            "root_id": self.root_id,
            "materialization_boundary": self.materialization_boundary,
            "peak_live_bytes": self.peak_live_bytes,
            "has_custom_ops": self.has_custom_ops,
            "ops": [s.op for s in self.steps],
            "steps": [{"step": s.step, "value_id": s.value_id, "op": s.op, "input_ids": list(s.input_ids),
                       "shape": list(s.shape), "dtype": s.dtype, "arg": _jsonable(s.arg)} for s in self.steps],
            "buffers": [{"value_id": b.value_id, "op": b.op, "shape": list(b.shape), "dtype": b.dtype,
                         "bytes": b.bytes, "first_step": b.first_step, "last_step": b.last_step,
                         "materialize": b.materialize} for b in self.buffers],
        }


@dataclass(frozen=True)
class DensePermutationViewCopyRequest:
    value_id: int
    input_shape: Tuple[str, ...]
    axes: Tuple[int, ...]
    dtype: str

    def summary(self) -> Dict[str, Any]:
        return {"kind": DENSE_PERMUTATION_VIEW_COPY_REQUEST, "valueId": self.value_id,
                "inputShape": list(self.input_shape), "axes": list(self.axes), "dtype": self.dtype}


@dataclass(frozen=True)
class GpuExecutionSubmission:
    plan: GpuExecutionPlan
    semantic_requests: Tuple[DensePermutationViewCopyRequest, ...]

    def plan_summary(self) -> Dict[str, Any]:
        s = self.plan.summary()
        for st in s["steps"]:
            if st["op"] == OP_PERMUTE:
                st["arg"] = None
        return s

    def semantic_request_summary(self) -> Dict[str, Any]:
        return {"schema": TENSOR_PLAN_SEMANTIC_REQUEST_SCHEMA,
                "version": {"major": TENSOR_PLAN_SEMANTIC_REQUEST_VERSION[0],
                            "minor": TENSOR_PLAN_SEMANTIC_REQUEST_VERSION[1]},
                "requests": [r.summary() for r in self.semantic_requests]}


def _bytes_for(shape: Tuple[int, ...], dtype: str) -> int:
    n = 1
    for d in shape:
        n *= max(int(d), 1)
    return n * _DTYPE_BYTES.get(dtype, 4)


def build_gpu_execution_plan(root: UOp, *, allow_custom: bool = False) -> GpuExecutionPlan:
    if not allow_custom:  # fused whatever the fusion switch says (_gpu_plan.py:292-294)
        root = fuse(root)
    order = toposort(root)
    custom = next((n for n in order if n.op == OP_CUSTOM), None)
    if custom is not None and not allow_custom:
        label = custom.arg.get("op") if isinstance(custom.arg, dict) else None
        raise GpuPlanUnsupported(
            f"GPU tensor plan refuses CUSTOM op {label!r}. Promote framework ops to primitive IR; use the "
            f"custom-kernel path only for explicit lab/user kernels.")
    index = {id(n): i for i, n in enumerate(order)}
    last = {id(n): i for i, n in enumerate(order)}
    for i, n in enumerate(order):
        if n.op not in PLAN_OPS and not (allow_custom and n.op == OP_CUSTOM):
            raise GpuPlanUnsupported(f"GPU tensor plan does not support opcode {n.op!r}. "
                                     f"Add primitive IR lowering/refusal before GPU codegen.")
        for inp in n.inputs:
            last[id(inp)] = i
    steps, bufs = [], []
    for n in order:
        sid = index[id(n)]
        arg = n.arg
        if n.op == OP_BUFFER:
            arg = n.arg  # the buffer id: inputs bind to value_id
        steps.append(PlanStep(sid, sid, n.op, tuple(index[id(i)] for i in n.inputs), tuple(n.shape), n.dtype, arg))
        bufs.append(PlanBuffer(sid, n.op, tuple(n.shape), n.dtype, _bytes_for(tuple(n.shape), n.dtype), sid,
                               last[id(n)], n is root))
    peak = 0
    for i in range(len(order)):
        peak = max(peak, sum(b.bytes for b in bufs if b.first_step <= i <= b.last_step))
    return GpuExecutionPlan(tuple(steps), tuple(bufs), index[id(root)], "root", peak, custom is not None)


def gpu_plan_summary(root: UOp, *, allow_custom: bool = False) -> Dict[str, Any]:
    return build_gpu_execution_plan(root, allow_custom=allow_custom).summary()


def _unsupported(path: str, message: str) -> None:
    raise GpuPlanUnsupported(f"GPU semantic request {path}: {message}")


def _dense_permutation_request(step: PlanStep, by_id: Dict[int, PlanStep]) -> DensePermutationViewCopyRequest:
    path = f"PERMUTE value_id={step.value_id}"
    if len(step.input_ids) != 1:
        _unsupported(path, "requires exactly one input")
    src = by_id.get(step.input_ids[0])
    if src is None:
        _unsupported(path, f"references missing source value_id={step.input_ids[0]}")
    if step.dtype != "float32" or src.dtype != "float32":
        _unsupported(path, "initial semantic view-copy lowering requires float32 source and destination")
    shape = tuple(src.shape)
    rank = len(shape)
    if rank not in (2, 3):
        _unsupported(path, f"initial semantic view-copy lowering requires rank 2 or 3, got {rank}")
    for a, e in enumerate(shape):
        if type(e) is not int or e <= 0:
            _unsupported(path, f"input shape axis {a} must be a positive static integer, got {e!r}")
        if e > _WIRE_I64_MAX:
            _unsupported(path, f"input shape axis {a} exceeds canonical signed-64 wire range")
    if type(step.arg) is not dict or "axes" not in step.arg:
        _unsupported(path, "arg must contain canonical tuple axes")
    extra = set(step.arg) - {"axes", "vjp_of"}
    if extra:
        _unsupported(path, f"arg contains unsupported fields {sorted(extra)!r}")
    axes = step.arg["axes"]
    if type(axes) is not tuple:
        _unsupported(path, "axes must be a canonical tuple")
    if len(axes) != rank or any(type(a) is not int or a < 0 or a >= rank for a in axes) or len(set(axes)) != rank:
        _unsupported(path, f"axes must be an exact permutation of [0, {rank})")
    derived = tuple(shape[a] for a in axes)
    if tuple(step.shape) != derived:
        _unsupported(path, f"declared output shape {tuple(step.shape)!r} does not match derived shape {derived!r}")
    return DensePermutationViewCopyRequest(step.value_id, tuple(str(e) for e in shape), tuple(axes), "f32")


def build_gpu_execution_submission(root: UOp, *, allow_custom: bool = False) -> GpuExecutionSubmission:
    plan = build_gpu_execution_plan(root, allow_custom=allow_custom)
    by_id = {s.value_id: s for s in plan.steps}
    reqs = tuple(_dense_permutation_request(s, by_id) for s in plan.steps if s.op == OP_PERMUTE)
    return GpuExecutionSubmission(plan, reqs)


def plan_json(summary: Dict[str, Any]) -> str:
    return json.dumps(summary, separators=(",", ":"))


__all__ = [
    "PLAN_OPS", "PlanStep", "PlanBuffer", "GpuExecutionPlan", "DensePermutationViewCopyRequest",
    "GpuExecutionSubmission", "GpuPlanUnsupported", "build_gpu_execution_plan", "build_gpu_execution_submission",
    "gpu_plan_summary", "plan_json", "TENSOR_PLAN_SEMANTIC_REQUEST_SCHEMA", "TENSOR_PLAN_SEMANTIC_REQUEST_VERSION",
    "DENSE_PERMUTATION_VIEW_COPY_REQUEST", "OP_CAUSAL_MASK",
]
