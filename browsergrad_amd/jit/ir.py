"""The UOp IR the walker and the plan builder consume.

Mirrors packages/browsergrad-jit/src/python/_ir.py: a DAG of frozen UOp nodes
(op, inputs, shape, dtype, arg) with opcode strings, leaf ops (BUFFER, CONST)
with no inputs, and an iterative toposort keyed on id() (_ir.py:403-432).
Only the opcodes on the realizer path are listed; the names and arg layouts
are the reference's (_ir.py:80-185):

    BUFFER  arg: buffer_id            LOAD   arg: None
    CONST   arg: {value}              CAST   arg: {dtype}
    ADD MUL DIV NEG EXP LOG           CMP    arg: {op: eq|ne|lt|le|gt|ge}
    WHERE   inputs (cond, a, b)       MATMUL
    REDUCE  arg: {op, axis, keepdims} RESHAPE arg: {new_shape}
    PERMUTE arg: {axes}               BROADCAST_TO arg: {shape}
    SLICE   arg: {slices: ((start, stop, step), ...)} one triple per axis
    LAYER_NORM arg: {normalized_shape, rows, cols, eps}
    FUSED_ELEMENTWISE arg: {ops}      FUSED_SOFTMAX arg: {axis}
    ATTENTION_FORWARD                 CUSTOM (refused by the walker)
    CONV1D / CONV2D / CONV3D / CONV_TRANSPOSE2D and their _BACKWARD_INPUT /
    _WEIGHT / _BIAS forms, arg: the plan's conv fields (n, c_in, ..., groups)

Equality is identity (every pass here keys on id(), as the reference's
realizers do), so no structural hash cache is needed.
"""
from __future__ import annotations

from ..errors import ShapeError  # the reference's _errors.ShapeError (one class package-wide)

from dataclasses import dataclass
from typing import Any, FrozenSet, List, Tuple

OP_BUFFER = "BUFFER"
OP_LOAD = "LOAD"
OP_CONST = "CONST"
OP_CAST = "CAST"
OP_ADD = "ADD"
OP_MUL = "MUL"
OP_DIV = "DIV"
OP_NEG = "NEG"
OP_EXP = "EXP"
OP_LOG = "LOG"
OP_CMP = "CMP"
OP_WHERE = "WHERE"
OP_MATMUL = "MATMUL"
OP_REDUCE = "REDUCE"
OP_RESHAPE = "RESHAPE"
OP_PERMUTE = "PERMUTE"
OP_SLICE = "SLICE"
OP_BROADCAST_TO = "BROADCAST_TO"
OP_LAYER_NORM = "LAYER_NORM"
OP_FUSED_ELEMENTWISE = "FUSED_ELEMENTWISE"
OP_FUSED_SOFTMAX = "FUSED_SOFTMAX"
OP_ATTENTION_FORWARD = "ATTENTION_FORWARD"
OP_CUSTOM = "CUSTOM"

CONV_OPS: FrozenSet[str] = frozenset(
    base + suffix
    for base in ("CONV1D", "CONV2D", "CONV3D", "CONV_TRANSPOSE2D")
    for suffix in ("", "_BACKWARD_INPUT", "_BACKWARD_WEIGHT", "_BACKWARD_BIAS"))

# Rewrites produced by this package's own fusion pass (hip_fusion.py); they
# never appear in graphs the reference builds.
OP_HIP_LINEAR = "HIP_LINEAR"          # GEMM + AMP rounding + bias + activation epilogue
OP_HIP_ATTENTION = "HIP_ATTENTION"    # the SDPA subgraph as one flash-attention kernel
OP_HIP_REDUCE_FUSED = "HIP_REDUCE_FUSED"  # elementwise program + last-axis reduction
# Plan-only leaf of the HIP tensor-plan route: the top-left causal mask
# ([lq, lk] bool, true where the key index exceeds the query index).
OP_CAUSAL_MASK = "CAUSAL_MASK"

ALL_OPS: FrozenSet[str] = frozenset({
    OP_BUFFER, OP_LOAD, OP_CONST, OP_CAST, OP_ADD, OP_MUL, OP_DIV, OP_NEG, OP_EXP, OP_LOG,
    OP_CMP, OP_WHERE, OP_MATMUL, OP_REDUCE, OP_RESHAPE, OP_PERMUTE, OP_SLICE, OP_BROADCAST_TO,
    OP_LAYER_NORM, OP_FUSED_ELEMENTWISE, OP_FUSED_SOFTMAX, OP_ATTENTION_FORWARD, OP_CUSTOM,
    OP_HIP_LINEAR, OP_HIP_ATTENTION, OP_HIP_REDUCE_FUSED, OP_CAUSAL_MASK,
}) | CONV_OPS

_LEAF_OPS: FrozenSet[str] = frozenset({OP_BUFFER, OP_CONST, OP_CAUSAL_MASK})

# NumPy dtype names (_ir.py:348-353) plus "bfloat16", an extension of this build.
KNOWN_DTYPES: FrozenSet[str] = frozenset({
    "float16", "float32", "float64", "bfloat16",
    "int8", "int16", "int32", "int64", "uint8", "uint16", "uint32", "uint64", "bool",
})

MAX_ELEMENTS = 2 ** 34  # sized for one MI355X (288 GB HBM); the reference caps at 2**30


def set_max_elements(n: int) -> None:
    """Change the per-tensor element ceiling (_ir.py:360-368); graphs built
    afterwards are checked against the new value."""
    global MAX_ELEMENTS
    if isinstance(n, bool) or not isinstance(n, int) or n <= 0:
        raise ValueError(f"set_max_elements: expected a positive int, got {n!r}")
    MAX_ELEMENTS = n




@dataclass(frozen=True, eq=False)
class UOp:
    op: str
    inputs: Tuple["UOp", ...]
    shape: Tuple[int, ...]
    dtype: str
    arg: Any = None

    def __post_init__(self) -> None:  # _ir.py:277-330
        if self.op not in ALL_OPS:
            raise ValueError(f"unknown opcode {self.op!r}")
        if self.op in _LEAF_OPS:
            if self.inputs:
                raise ShapeError(f"{self.op} is a leaf opcode and must have zero inputs, got {len(self.inputs)}")
        elif not self.inputs:
            raise ShapeError(f"{self.op} is not a leaf and must have at least one input")
        if not isinstance(self.shape, tuple):
            raise ShapeError(f"{self.op}: shape must be a tuple, got {type(self.shape).__name__}")
        n = 1
        for i, d in enumerate(self.shape):
            if not isinstance(d, int) or d < 0:
                raise ShapeError(f"{self.op}: shape[{i}] must be a non-negative int, got {d!r}")
            n *= max(d, 1)
        if n > MAX_ELEMENTS:
            raise ShapeError(f"{self.op}: shape {self.shape} = {n} elements exceeds the {MAX_ELEMENTS}-element ceiling")
        if self.dtype not in KNOWN_DTYPES:
            raise ValueError(f"{self.op}: unknown dtype {self.dtype!r}")

    @property
    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


def toposort(root: UOp) -> List[UOp]:
    """Leaves-first order, iterative, keyed on id() (_ir.py:403-432)."""
    order: List[UOp] = []
    visited: set = set()
    stack: List[Tuple[UOp, int]] = [(root, 0)]
    while stack:
        node, child = stack[-1]
        if id(node) in visited:
            stack.pop()
            continue
        if child < len(node.inputs):
            stack[-1] = (node, child + 1)
            nxt = node.inputs[child]
            if id(nxt) not in visited:
                stack.append((nxt, 0))
            continue
        visited.add(id(node))
        order.append(node)
        stack.pop()
    return order


def buffer(buffer_id: str, shape: Tuple[int, ...], dtype: str) -> UOp:
    return UOp(OP_BUFFER, (), tuple(shape), dtype, buffer_id)


def load(buf: UOp) -> UOp:
    if buf.op != OP_BUFFER:
        raise ShapeError(f"load() expects a BUFFER UOp, got {buf.op!r}")
    return UOp(OP_LOAD, (buf,), buf.shape, buf.dtype, None)


def const(value: float, dtype: str = "float32") -> UOp:
    return UOp(OP_CONST, (), (), dtype, {"value": value})


__all__ = [name for name in dir() if name.startswith("OP_")] + [
    "ALL_OPS", "KNOWN_DTYPES", "ShapeError", "UOp", "toposort", "buffer", "load", "const", "set_max_elements",
]
