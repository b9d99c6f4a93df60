"""Compile an elementwise sub-DAG of UOps into one fused-kernel program.

The fused kernel of libbghip (bg_fused_ex) evaluates a straight-line program
of <= 32 ops over <= 8 broadcast inputs and <= 16 immediates in float32
registers, storing the last op's value in the output dtype, optionally
reducing the innermost axis.  This module lowers a set of IR nodes to that
form:

  ADD MUL DIV NEG EXP LOG        -> the reference's fused opcodes
                                    (fused_elementwise.ts:83-90)
  CMP {eq,ne,lt,le,gt,ge}        -> CMP_* (1.0 / 0.0 in registers, bool on store)
  WHERE                          -> WHERE(cond != 0 ? a : b)
  CAST                           -> ROUND_F16 / ROUND_BF16 (to a narrow float),
                                    CMP_NE 0 (to bool), COPY (to float32)
  CONST                          -> IMM (immediate table; float64 values land
                                    in f32 exactly as CAST(f64 -> f32) would)

Every node whose dtype is float16 / bfloat16 is followed by a rounding op so
the program reproduces numpy's per-op rounding in that dtype (_realize.py
computes each op in the IR dtype); float32 nodes need none.  float64 nodes
other than CONST are refused: the HIP path has no float64 arithmetic.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

from .ir import OP_ADD, OP_CAST, OP_CMP, OP_CONST, OP_DIV, OP_EXP, OP_LOG, OP_MUL, OP_NEG, OP_WHERE, UOp

ELEMENTWISE = frozenset({OP_ADD, OP_MUL, OP_DIV, OP_NEG, OP_EXP, OP_LOG, OP_CMP, OP_WHERE, OP_CAST})
_CMP = {"eq": "CMP_EQ", "ne": "CMP_NE", "lt": "CMP_LT", "le": "CMP_LE", "gt": "CMP_GT", "ge": "CMP_GE"}
_ROUND = {"float16": "ROUND_F16", "bfloat16": "ROUND_BF16"}
DEVICE_FLOATS = ("float32", "float16", "bfloat16")
MAX_OPS, MAX_INPUTS, MAX_IMMS = 32, 8, 16


class ProgramTooLarge(Exception):
    pass


class NotLowerable(Exception):
    pass


@dataclass
class Program:
    ops: List[Tuple[str, int, int, int]]
    imms: List[float]
    inputs: List[UOp]            # external inputs, in ref order (-1, -2, ...)
    shape: Tuple[int, ...]       # iteration shape
    out_dtype: str

    def strides(self) -> List[List[int]]:
        return [broadcast_strides(u.shape, self.shape) for u in self.inputs]


def broadcast_strides(src: Sequence[int], out: Sequence[int]) -> List[int]:
    """Element strides of a contiguous `src` viewed with numpy broadcasting as `out`."""
    st = [0] * len(out)
    stride = 1
    for k in range(1, len(src) + 1):
        s, o = src[-k], out[-k]
        if s == o and s != 1:
            st[-k] = stride
        elif s != 1:
            raise NotLowerable(f"shape {tuple(src)} does not broadcast to {tuple(out)}")
        stride *= s
    return st


def lowerable(n: UOp) -> bool:
    if n.op == OP_CAST:
        return n.dtype in DEVICE_FLOATS + ("bool",) and (n.inputs[0].dtype in DEVICE_FLOATS + ("bool",)
                                                          or n.inputs[0].op == OP_CONST)
    if n.op in ELEMENTWISE:
        return n.dtype in DEVICE_FLOATS + ("bool",)
    return False


def compile_program(nodes: Sequence[UOp], root: UOp, shape: Optional[Tuple[int, ...]] = None) -> Program:
    """`nodes`: the DAG's interior nodes in topological order (root last).
    Inputs of interior nodes that are not interior are external inputs,
    except CONST leaves, which become immediates."""
    inside = {id(n) for n in nodes}
    ops: List[Tuple[str, int, int, int]] = []
    imms: List[float] = []
    inputs: List[UOp] = []
    ref: Dict[int, int] = {}

    def emit(code: str, a: int, b: int = 0, c: int = 0) -> int:
        ops.append((code, a, b, c))
        if len(ops) > MAX_OPS:
            raise ProgramTooLarge("more than 32 ops")
        return len(ops) - 1

    def operand(u: UOp) -> int:
        if id(u) in ref:
            return ref[id(u)]
        if u.op == OP_CONST and id(u) not in inside:
            v = u.arg["value"]
            imms.append(float(v))
            if len(imms) > MAX_IMMS:
                raise ProgramTooLarge("more than 16 immediates")
            r = emit("IMM", len(imms) - 1)
            ref[id(u)] = r
            return r
        if id(u) in inside:
            raise NotLowerable("interior node used before definition")
        if u.dtype not in DEVICE_FLOATS + ("bool",):
            raise NotLowerable(f"external input dtype {u.dtype} has no device kernel")
        inputs.append(u)
        if len(inputs) > MAX_INPUTS:
            raise ProgramTooLarge("more than 8 inputs")
        r = -len(inputs)
        ref[id(u)] = r
        return r

    for n in nodes:
        if not lowerable(n):
            raise NotLowerable(f"{n.op} ({n.dtype}) is not an elementwise device op")
        a = [operand(i) for i in n.inputs]
        if n.op in (OP_ADD, OP_MUL, OP_DIV):
            r = emit(n.op, a[0], a[1])
        elif n.op in (OP_NEG, OP_EXP, OP_LOG):
            r = emit(n.op, a[0])
        elif n.op == OP_CMP:
            r = emit(_CMP[n.arg["op"]], a[0], a[1])
        elif n.op == OP_WHERE:
            r = emit("WHERE", a[0], a[1], a[2])
        else:  # CAST
            src = n.inputs[0]
            if n.dtype in _ROUND:
                r = emit(_ROUND[n.dtype], a[0])
            elif n.dtype == "bool":
                imms.append(0.0)
                z = emit("IMM", len(imms) - 1)
                r = emit("CMP_NE", a[0], z)
            elif src.op == OP_CONST:
                r = a[0]  # f64 -> f32 of an immediate: the kernel reads it as f32
            else:
                r = emit("COPY", a[0])
        if n.op != OP_CAST and n.op != OP_CMP and n.dtype in _ROUND:
            r = emit(_ROUND[n.dtype], r)
        ref[id(n)] = r
    if not ops or ref.get(id(root)) != len(ops) - 1:
        # the root's value must be the last op (e.g. a CAST of an immediate)
        emit("COPY", ref[id(root)])
    return Program(ops, imms, inputs, tuple(shape if shape is not None else root.shape), root.dtype)


__all__ = ["Program", "compile_program", "broadcast_strides", "lowerable", "ELEMENTWISE", "ProgramTooLarge",
           "NotLowerable", "DEVICE_FLOATS"]
