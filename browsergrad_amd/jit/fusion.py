"""Elementwise-chain and softmax fusion (the reference's _fusion.fuse).

Two matchers, run in the reference's order (_fusion.py:413-517):

  1. softmax DAG (_fusion.py:273-361): DIV(EXP(ADD(x, NEG(REDUCE max keepdims
     x))), REDUCE sum keepdims of the same EXP), EXP read exactly twice, every
     other interior node read once, max/sum axes equal -> FUSED_SOFTMAX{axis}.
  2. elementwise chains (_fusion.py:141-232): maximal linear runs of
     ADD MUL DIV NEG EXP LOG where every non-terminal node has exactly one
     consumer and shape/dtype stay equal, length >= 2 ->
     FUSED_ELEMENTWISE{ops: ((opcode, lhs_ref, rhs_ref|None), ...)} with
     refs < 0 naming external inputs (-1 = first) and refs >= 0 earlier steps.
     A node is a chain start unless one of its inputs is an unfused
     elementwise node with a single consumer.

`holdout` ids (values backward closures read) never become chain interiors.
The per-call report (fused / unfused records) is kept for introspection.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Iterable, List, Optional, Set, Tuple

from .ir import (
    OP_ADD, OP_DIV, OP_EXP, OP_FUSED_ELEMENTWISE, OP_FUSED_SOFTMAX, OP_LOG, OP_MUL, OP_NEG, OP_REDUCE, UOp,
    toposort,
)

ELEMENTWISE_OPS = frozenset({OP_ADD, OP_MUL, OP_DIV, OP_NEG, OP_EXP, OP_LOG})


@dataclass
class FusedKernelInfo:
    pattern: str
    n_ops: int
    shape: Tuple[int, ...]
    dtype: str
    ops: Tuple[str, ...]


@dataclass
class UnfusedReason:
    pattern: str
    op: str
    shape: Tuple[int, ...]
    reason: str


@dataclass
class FusionReport:
    fused: List[FusedKernelInfo] = field(default_factory=list)
    unfused: List[UnfusedReason] = field(default_factory=list)


_LAST = FusionReport()


def get_last_report() -> FusionReport:
    return _LAST


def consumers_of(root: UOp) -> Dict[int, List[UOp]]:
    cons: Dict[int, List[UOp]] = {}
    for n in toposort(root):
        cons.setdefault(id(n), [])
        for i in n.inputs:
            cons.setdefault(id(i), []).append(n)
    return cons


def _reduce_arg(n: UOp, op: str) -> bool:
    return n.op == OP_REDUCE and isinstance(n.arg, dict) and n.arg.get("op") == op and bool(n.arg.get("keepdims"))


def _match_softmax(div: UOp, cons: Dict[int, List[UOp]], hold: Set[int], done: Set[int]) -> Optional[Tuple[UOp, ...]]:
    if div.op != OP_DIV or id(div) in done or len(div.inputs) != 2:
        return None
    ex, sm = div.inputs
    if ex.op != OP_EXP or not _reduce_arg(sm, "sum") or id(ex) in done or id(sm) in done:
        return None
    if len(sm.inputs) != 1 or sm.inputs[0] is not ex:
        return None
    ex_cons = cons.get(id(ex), [])
    if len(ex_cons) != 2 or {c.op for c in ex_cons} != {OP_DIV, OP_REDUCE}:
        return None
    if len(ex.inputs) != 1:
        return None
    add = ex.inputs[0]
    if add.op != OP_ADD or len(add.inputs) != 2 or id(add) in done:
        return None
    x, neg = add.inputs
    if neg.op != OP_NEG:
        x, neg = neg, x
    if neg.op != OP_NEG or len(neg.inputs) != 1:
        return None
    mx = neg.inputs[0]
    if not _reduce_arg(mx, "max") or len(mx.inputs) != 1 or mx.inputs[0] is not x:
        return None
    if mx.arg.get("axis") != sm.arg.get("axis"):
        return None
    interior = (mx, neg, add, ex, sm)
    if any(id(n) in hold for n in interior):
        return None
    if any(len(cons.get(id(n), [])) != 1 for n in (mx, neg, add, sm)):
        return None
    return (x, mx, neg, add, ex, sm, div)


def _match_chain(start: UOp, cons: Dict[int, List[UOp]], hold: Set[int], done: Set[int]) -> Optional[List[UOp]]:
    if start.op not in ELEMENTWISE_OPS or id(start) in done:
        return None
    chain = [start]
    cur = start
    while True:
        cl = cons.get(id(cur), [])
        if len(cl) != 1:
            break
        nxt = cl[0]
        if nxt.op not in ELEMENTWISE_OPS or id(nxt) in done or id(cur) in hold:
            break
        if nxt.shape != cur.shape or nxt.dtype != cur.dtype:
            break
        chain.append(nxt)
        cur = nxt
    return chain if len(chain) >= 2 else None


def _build_chain(chain: List[UOp]) -> UOp:
    external: List[UOp] = []
    ext_ref: Dict[int, int] = {}
    step_of: Dict[int, int] = {}

    def ref(n: UOp) -> int:
        if id(n) in step_of:
            return step_of[id(n)]
        if id(n) not in ext_ref:
            external.append(n)
            ext_ref[id(n)] = -len(external)
        return ext_ref[id(n)]

    ops = []
    for i, n in enumerate(chain):
        lhs = ref(n.inputs[0])
        rhs = ref(n.inputs[1]) if len(n.inputs) == 2 else None
        ops.append((n.op, lhs, rhs))
        step_of[id(n)] = i
    last = chain[-1]
    return UOp(OP_FUSED_ELEMENTWISE, tuple(external), last.shape, last.dtype, {"ops": tuple(ops)})


def substitute(root: UOp, subs: Dict[int, UOp]) -> UOp:
    if not subs:
        return root
    built: Dict[int, UOp] = {}
    for n in toposort(root):
        if id(n) in subs:
            built[id(n)] = subs[id(n)]
            # the replacement's own inputs may need rewiring too
            r = subs[id(n)]
            ins = tuple(built.get(id(i), i) for i in r.inputs)
            if any(a is not b for a, b in zip(ins, r.inputs)):
                built[id(n)] = UOp(r.op, ins, r.shape, r.dtype, r.arg)
            continue
        if not n.inputs:
            built[id(n)] = n
            continue
        ins = tuple(built.get(id(i), i) for i in n.inputs)
        built[id(n)] = n if all(a is b for a, b in zip(ins, n.inputs)) else UOp(n.op, ins, n.shape, n.dtype, n.arg)
    return built[id(root)]


def fuse(root: UOp, holdout: Optional[Iterable[int]] = None, *, include_softmax: bool = True,
         include_elementwise: bool = True) -> UOp:
    global _LAST
    _LAST = FusionReport()
    hold: Set[int] = set(holdout or ())
    cons = consumers_of(root)
    done: Set[int] = set()
    subs: Dict[int, UOp] = {}
    nodes = toposort(root)
    if include_softmax:
        for n in nodes:
            m = _match_softmax(n, cons, hold, done)
            if m is None:
                if n.op == OP_DIV and id(n) not in done:
                    _LAST.unfused.append(UnfusedReason("softmax", n.op, n.shape, "DIV did not match softmax template"))
                continue
            x, mx = m[0], m[1]
            div = m[-1]
            subs[id(div)] = UOp(OP_FUSED_SOFTMAX, (x,), div.shape, div.dtype, {"axis": mx.arg.get("axis")})
            done.update(id(k) for k in m[1:])
            _LAST.fused.append(FusedKernelInfo("softmax", 6, div.shape, div.dtype,
                                               ("REDUCE(max)", "NEG", "ADD", "EXP", "REDUCE(sum)", "DIV")))
    if include_elementwise:
        for n in nodes:
            if id(n) in done or n.op not in ELEMENTWISE_OPS:
                continue
            if any(i.op in ELEMENTWISE_OPS and id(i) not in done and len(cons.get(id(i), [])) == 1
                   for i in n.inputs):
                continue  # mid-chain: the chain is walked from its start
            chain = _match_chain(n, cons, hold, done)
            if chain is None:
                _LAST.unfused.append(UnfusedReason("elementwise_chain", n.op, n.shape,
                                                   "chain length < 2 or autograd holdout / shape mismatch"))
                continue
            subs[id(chain[-1])] = _build_chain(chain)
            done.update(id(k) for k in chain)
            _LAST.fused.append(FusedKernelInfo("elementwise_chain", len(chain), chain[-1].shape, chain[-1].dtype,
                                               tuple(k.op for k in chain)))
    return substitute(root, subs)


__all__ = ["fuse", "substitute", "consumers_of", "get_last_report", "FusionReport", "FusedKernelInfo",
           "UnfusedReason", "ELEMENTWISE_OPS"]
