"""Cast insertion for autocast (the reference's _amp.insert_cast_pass).

Policy (_amp.py:56-69):
  ALLOWLIST  MATMUL                         inputs -> narrow dtype, output narrow
  BLOCKLIST  EXP LOG REDUCE DIV FUSED_SOFTMAX inputs -> float32, output float32
  PROMOTE    ADD MUL NEG WHERE              all inputs -> float32 if any input is
                                            float32, else the first input's dtype
Only nodes whose arg carries `autocast_hint` are rewritten; everything else
passes through with rewired inputs (_amp.py:183-261).  CASTs the pass adds
carry arg {"dtype": d, "amp_inserted": True}.

The narrow dtype is the hint itself: "float16" as in the reference, or
"bfloat16" (an extension; MI355X runs both on MFMA at the same rate).
"""
from __future__ import annotations

from typing import Any, Dict

from .ir import (
    OP_ADD, OP_CAST, OP_DIV, OP_EXP, OP_FUSED_SOFTMAX, OP_LOG, OP_MATMUL, OP_MUL, OP_NEG, OP_REDUCE,
    OP_WHERE, UOp, toposort,
)

ALLOWLIST_NARROW = frozenset({OP_MATMUL})
BLOCKLIST_F32 = frozenset({OP_EXP, OP_LOG, OP_REDUCE, OP_DIV, OP_FUSED_SOFTMAX})
PROMOTE_OPS = frozenset({OP_ADD, OP_MUL, OP_NEG, OP_WHERE})


def _hint(arg: Any) -> str:
    if isinstance(arg, dict) and arg.get("autocast_hint") in ("float16", "bfloat16"):
        return arg["autocast_hint"]
    return ""


def cast_to(u: UOp, dtype: str) -> UOp:
    if u.dtype == dtype:
        return u
    return UOp(OP_CAST, (u,), u.shape, dtype, {"dtype": dtype, "amp_inserted": True})


def insert_cast_pass(root: UOp) -> UOp:
    nodes = toposort(root)
    if not any(_hint(n.arg) for n in nodes):
        return root
    new: Dict[int, UOp] = {}
    for node in nodes:
        if not node.inputs:
            new[id(node)] = node
            continue
        ins = tuple(new.get(id(i), i) for i in node.inputs)
        narrow = _hint(node.arg)
        if narrow and node.op in ALLOWLIST_NARROW:
            out = UOp(node.op, tuple(cast_to(i, narrow) for i in ins), node.shape, narrow, node.arg)
        elif narrow and node.op in BLOCKLIST_F32:
            out = UOp(node.op, tuple(cast_to(i, "float32") for i in ins), node.shape, "float32", node.arg)
        elif narrow and node.op in PROMOTE_OPS:
            target = "float32" if any(i.dtype == "float32" for i in ins) else ins[0].dtype
            out = UOp(node.op, tuple(cast_to(i, target) for i in ins), node.shape, target, node.arg)
        elif all(a is b for a, b in zip(ins, node.inputs)):
            out = node
        else:
            out = UOp(node.op, ins, node.shape, node.dtype, node.arg)
        new[id(node)] = out
    return new.get(id(root), root)


__all__ = ["insert_cast_pass", "cast_to", "ALLOWLIST_NARROW", "BLOCKLIST_F32", "PROMOTE_OPS"]
