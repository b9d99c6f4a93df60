"""Graph rewrites that map whole subgraphs onto single HIP kernels.

Run by the walker after cast insertion and before the reference's fusion
pass.  The reference has no counterpart: its realizer dispatches one kernel
per (fused) op, with 2-D matmul only and no causal attention
(_realize_webgpu.py:121-128, 290-302).  Each rewrite preserves the values of
the subgraph it replaces (the tests compare against the unfused graph on the
CPU oracle):

HIP_ATTENTION  the SDPA graph of _functional.py:1505-1533 after autocast:
      S  = MATMUL(Q, PERMUTE(K, swap last two) [-> CAST])        (narrow dtype)
      S' = MUL(CAST_f32(S), scale)            scale: full() buffer or CONST
      S''= WHERE(causal mask, CONST(-inf), S')                   (optional)
      P  = softmax DAG of S'' over the last axis (f32)
      O  = MATMUL(CAST_narrow(P), V)
    -> one flash-attention kernel (bg_attention_ex, round_scores = the
       narrow rounding of S, causal from the mask buffer's provenance).

HIP_LINEAR     ADD(CAST_f32(MATMUL(A, B)) | MATMUL(A, B), bias) with B =
    [CAST](PERMUTE(W, (1, 0))) or a plain 2-D matrix, optionally followed by
    relu (WHERE(CMP gt(y, 0), y, 0), _functional.py:99-111) or the tanh-GELU
    graph of _functional.py:129-133 -> one GEMM with the rounding / bias /
    activation epilogue (bg_matmul_ex).

HIP_FUSED      any remaining elementwise sub-DAG (ADD MUL DIV NEG EXP LOG CMP
    WHERE CAST, CONST immediates), optionally ending in a REDUCE over the last
    axis -> one fused-kernel program (bg_fused_ex), e.g. C2's
    relu(a*b+c)*exp(-a*a) row sum in one pass over a, b, c.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Set, Tuple

import numpy as np

from .buffers import BufferTable
from .fusion import _match_softmax, consumers_of, fuse, substitute
from .ir import (
    OP_ADD, OP_BUFFER, OP_CAST, OP_CMP, OP_CONST, OP_DIV, OP_EXP, OP_HIP_ATTENTION, OP_HIP_LINEAR, OP_LAYER_NORM,
    OP_HIP_REDUCE_FUSED, OP_LOAD, OP_MATMUL, OP_MUL, OP_NEG, OP_PERMUTE, OP_REDUCE, OP_RESHAPE, OP_SLICE, OP_WHERE,
    UOp, toposort,
)
from .program import NotLowerable, ProgramTooLarge, compile_program, lowerable

NARROW = ("float16", "bfloat16")

# HIP_LINEAR activation codes (bg_matmul_desc.act)
ACT_NONE, ACT_RELU, ACT_GELU = 0, 1, 2


def _only_consumers(n: UOp, cons: Dict[int, List[UOp]], allowed: Set[int]) -> bool:
    return all(id(c) in allowed for c in cons.get(id(n), []))


def _const_value(n: UOp) -> Optional[float]:
    """Value of a CONST, possibly behind AMP's CAST (as float32 would hold it)."""
    if n.op == OP_CAST and n.inputs[0].op == OP_CONST and n.dtype == "float32":
        return float(np.float32(n.inputs[0].arg["value"]))
    if n.op == OP_CONST:
        return float(n.arg["value"])
    return None


def _buffer_of(n: UOp) -> Optional[UOp]:
    if n.op == OP_LOAD and n.inputs[0].op == OP_BUFFER:
        return n.inputs[0]
    if n.op == OP_BUFFER:
        return n
    return None


# ---- attention ---------------------------------------------------------------

def _match_attention(o: UOp, cons: Dict[int, List[UOp]], bt: BufferTable) -> Optional[Tuple[UOp, List[UOp]]]:
    if o.op != OP_MATMUL or len(o.inputs) != 2 or len(o.shape) < 3:
        return None
    p_in, v = o.inputs
    interior: List[UOp] = []
    if o.dtype in NARROW:
        if p_in.op != OP_CAST or p_in.dtype != o.dtype:
            return None
        p = p_in.inputs[0]
        interior.append(p_in)
    else:
        p = p_in
    if p.dtype != "float32":
        return None
    sm = _match_softmax(p, cons, set(), set())
    if sm is None:
        return None
    x, mx = sm[0], sm[1]
    axis = mx.arg.get("axis")
    if axis not in (-1, len(x.shape) - 1):
        return None
    interior.extend(sm[1:])
    causal = False
    s = x
    if s.op == OP_WHERE:
        mask, fill, inner = s.inputs
        mb = _buffer_of(mask)
        fv = _const_value(fill)
        if mb is None or fv is None or fv != float("-inf"):
            return None
        if bt.causal_mask(mb.arg) != (x.shape[-2], x.shape[-1]):
            return None
        causal = True
        interior.append(s)
        s = inner
    if s.op != OP_MUL:
        return None
    a, b = s.inputs
    scale = None
    for sc_node, sv in ((b, a), (a, b)):
        fb = _buffer_of(sc_node)
        if fb is not None and bt.fill_value(fb.arg) is not None:
            scale, s_val = bt.fill_value(fb.arg), sv
            break
        cv = _const_value(sc_node)
        if cv is not None:
            scale, s_val = cv, sv
            break
    if scale is None or scale <= 0:
        return None
    interior.append(s)
    round_scores = False
    if s_val.op == OP_CAST and s_val.dtype == "float32" and s_val.inputs[0].dtype in NARROW:
        interior.append(s_val)
        s_val = s_val.inputs[0]
        round_scores = True
    if s_val.op != OP_MATMUL:
        return None
    interior.append(s_val)
    q, kt = s_val.inputs
    k = None
    if kt.op == OP_PERMUTE:
        ax = tuple(kt.arg["axes"])
        r = len(kt.shape)
        if ax == tuple(range(r - 2)) + (r - 1, r - 2):
            k = kt.inputs[0]
            interior.append(kt)
    elif kt.op == OP_CAST and kt.inputs[0].op == OP_PERMUTE:
        perm = kt.inputs[0]
        ax = tuple(perm.arg["axes"])
        r = len(perm.shape)
        if ax == tuple(range(r - 2)) + (r - 1, r - 2):
            src = perm.inputs[0]
            k = src if src.dtype == kt.dtype else UOp(OP_CAST, (src,), src.shape, kt.dtype,
                                                          {"dtype": kt.dtype, "amp_inserted": True})
            interior.extend([kt, perm])
    if k is None:
        return None
    if not (q.dtype == k.dtype == v.dtype) or q.dtype not in NARROW + ("float32",):
        return None
    if q.dtype != "float32" and not round_scores:
        return None
    if len(q.shape) != 4 or q.shape[:2] != k.shape[:2] or k.shape != v.shape or q.shape[-1] != k.shape[-1]:
        return None
    allowed = {id(n) for n in interior} | {id(o)}
    for n in interior:
        if not _only_consumers(n, cons, allowed):
            return None
    fused = UOp(OP_HIP_ATTENTION, (q, k, v), o.shape, o.dtype,
                {"scale": float(scale), "causal": causal, "round_scores": round_scores})
    return fused, interior


# ---- linear ------------------------------------------------------------------

def _weight_operand(b: UOp) -> Tuple[UOp, bool, List[UOp]]:
    """(operand, trans_b, interior) for the B input of a linear MATMUL."""
    if b.op == OP_PERMUTE and tuple(b.arg["axes"]) == (1, 0):
        return b.inputs[0], True, [b]
    if b.op == OP_CAST and b.inputs[0].op == OP_PERMUTE and tuple(b.inputs[0].arg["axes"]) == (1, 0):
        w = b.inputs[0].inputs[0]
        cw = w if w.dtype == b.dtype else UOp(OP_CAST, (w,), w.shape, b.dtype, {"dtype": b.dtype, "amp_inserted": True})
        return cw, True, [b, b.inputs[0]]
    return b, False, []


def _match_gelu(y: UOp, cons: Dict[int, List[UOp]]) -> Optional[Tuple[UOp, List[UOp]]]:
    """The tanh-GELU graph built by _functional.gelu over `y`, after AMP
    (float64 constants behind CASTs to float32).  Returns (root, interior)."""
    def is_c(n: UOp, v: float) -> bool:
        cv = _const_value(n)
        return cv is not None and np.float32(cv) == np.float32(v)

    def mul_c(n: UOp, v: float) -> Optional[UOp]:
        if n.op == OP_MUL:
            a, b = n.inputs
            if is_c(a, v):
                return b
            if is_c(b, v):
                return a
        return None

    nodes: List[UOp] = []
    ys = cons.get(id(y), [])
    t1 = next((c for c in ys if mul_c(c, 0.5) is y), None)            # 0.5 * y
    m1 = next((c for c in ys if mul_c(c, 0.044715) is y), None)       # 0.044715 * y
    if t1 is None or m1 is None:
        return None
    c2 = cons.get(id(m1), [])
    if len(c2) != 1 or c2[0].op != OP_MUL or set(map(id, c2[0].inputs)) != {id(m1), id(y)}:
        return None
    m2 = c2[0]
    c3 = cons.get(id(m2), [])
    if len(c3) != 1 or c3[0].op != OP_MUL or set(map(id, c3[0].inputs)) != {id(m2), id(y)}:
        return None
    m3 = c3[0]
    c4 = cons.get(id(m3), [])
    if len(c4) != 1 or c4[0].op != OP_ADD or set(map(id, c4[0].inputs)) != {id(m3), id(y)}:
        return None
    inner = c4[0]
    c5 = cons.get(id(inner), [])
    if len(c5) != 1 or mul_c(c5[0], float((2.0 / np.pi) ** 0.5)) is not inner:
        return None
    u = c5[0]
    uc = cons.get(id(u), [])
    e_pos = next((c for c in uc if c.op == OP_EXP), None)
    nu = next((c for c in uc if c.op == OP_NEG), None)
    if e_pos is None or nu is None or len(uc) != 2:
        return None
    nc = cons.get(id(nu), [])
    if len(nc) != 1 or nc[0].op != OP_EXP:
        return None
    e_neg = nc[0]
    enc = cons.get(id(e_neg), [])
    neg_en = next((c for c in enc if c.op == OP_NEG), None)
    den = next((c for c in enc if c.op == OP_ADD), None)
    if neg_en is None or den is None or len(enc) != 2 or set(map(id, den.inputs)) != {id(e_pos), id(e_neg)}:
        return None
    nn = cons.get(id(neg_en), [])
    if len(nn) != 1 or nn[0].op != OP_ADD or set(map(id, nn[0].inputs)) != {id(e_pos), id(neg_en)}:
        return None
    num = nn[0]
    epc = cons.get(id(e_pos), [])
    if {id(c) for c in epc} != {id(num), id(den)}:
        return None
    dc = cons.get(id(den), [])
    numc = cons.get(id(num), [])
    if len(dc) != 1 or len(numc) != 1 or dc[0] is not numc[0] or dc[0].op != OP_DIV or dc[0].inputs != (num, den):
        return None
    th = dc[0]
    tc = cons.get(id(th), [])
    if len(tc) != 1 or tc[0].op != OP_ADD:
        return None
    one_th = tc[0]
    other = one_th.inputs[0] if one_th.inputs[1] is th else one_th.inputs[1]
    if not is_c(other, 1.0):
        return None
    oc = cons.get(id(one_th), [])
    t1c = cons.get(id(t1), [])
    if len(oc) != 1 or len(t1c) != 1 or oc[0] is not t1c[0] or oc[0].op != OP_MUL:
        return None
    g = oc[0]
    if set(map(id, g.inputs)) != {id(t1), id(one_th)}:
        return None
    nodes = [t1, m1, m2, m3, inner, u, e_pos, nu, e_neg, neg_en, den, num, th, one_th]
    for cst in (t1, m1, u, one_th):
        for i in cst.inputs:
            if i.op == OP_CAST and i.inputs[0].op == OP_CONST:
                nodes.append(i)
    # y itself feeds only the GELU graph
    allowed = {id(n) for n in nodes} | {id(g)}
    if not _only_consumers(y, cons, allowed):
        return None
    return g, nodes


def _match_linear(add: UOp, cons: Dict[int, List[UOp]]) -> Optional[Tuple[UOp, UOp, List[UOp]]]:
    """Returns (fused node, node it replaces, interior)."""
    if add.op != OP_ADD or add.dtype != "float32":
        return None
    for mm_side, bias in (add.inputs, add.inputs[::-1]):
        interior: List[UOp] = []
        round_out = False
        mm = mm_side
        if mm.op == OP_CAST and mm.dtype == "float32" and mm.inputs[0].op == OP_MATMUL and mm.inputs[0].dtype in NARROW:
            interior.append(mm)
            mm = mm.inputs[0]
            round_out = True
        if mm.op != OP_MATMUL:
            continue
        if not round_out and mm.dtype != "float32":
            continue
        a, b = mm.inputs
        if len(b.shape) != 2 or len(a.shape) < 2 or a.dtype != b.dtype:
            continue
        n = mm.shape[-1]
        if bias.dtype != "float32" or bias.numel != n or (bias.shape and bias.shape[-1] != n):
            continue
        w, trans_b, w_int = _weight_operand(b)
        interior.extend([mm] + w_int)
        allowed = {id(x) for x in interior} | {id(add)}
        if not all(_only_consumers(x, cons, allowed) for x in interior):
            continue
        act, out = ACT_NONE, add
        act_nodes: List[UOp] = []
        ac = cons.get(id(add), [])
        if len(ac) == 2:
            cmp_n = next((c for c in ac if c.op == OP_CMP), None)
            wh = next((c for c in ac if c.op == OP_WHERE), None)
            if (cmp_n is not None and wh is not None and cmp_n.arg.get("op") == "gt" and cmp_n.inputs[0] is add
                    and _const_value(cmp_n.inputs[1]) == 0.0 and wh.inputs[0] is cmp_n and wh.inputs[1] is add
                    and _const_value(wh.inputs[2]) == 0.0 and len(cons.get(id(cmp_n), [])) == 1):
                act, out, act_nodes = ACT_RELU, wh, [cmp_n]
        if act == ACT_NONE:
            g = _match_gelu(add, cons)
            if g is not None:
                act, out, act_nodes = ACT_GELU, g[0], g[1]
        fused = UOp(OP_HIP_LINEAR, (a, w, bias), out.shape, "float32",
                    {"trans_b": trans_b, "round_out": round_out, "act": act, "in_dtype": a.dtype})
        return fused, out, interior + [add] + act_nodes
    return None


def _fold_residual_adds(root: UOp) -> UOp:
    """ADD(HIP_LINEAR(...), r) with r float32 of the linear's own shape (a
    residual stream, `x + linear(h)`) becomes one HIP_LINEAR whose epilogue
    adds r after the bias and activation (bg_matmul_ex2).  f32 addition is
    commutative, so either operand order gives the reference's bits."""
    cons = consumers_of(root)
    subs: Dict[int, UOp] = {}
    for n in toposort(root):
        if n.op != OP_ADD or n.dtype != "float32":
            continue
        for lin, r in (n.inputs, n.inputs[::-1]):
            if (lin.op == OP_HIP_LINEAR and lin.dtype == "float32" and len(lin.inputs) == 3
                    and len(cons.get(id(lin), [])) == 1
                    and r.dtype == "float32" and tuple(r.shape) == tuple(lin.shape) and r is not lin):
                subs[id(n)] = UOp(OP_HIP_LINEAR, lin.inputs + (r,), n.shape, "float32", {**lin.arg, "residual": True})
                break
    return substitute(root, subs)


# ---- dtype refresh ---------------------------------------------------------------

_PASS_THROUGH = frozenset({"LOAD", "RESHAPE", "PERMUTE", "SLICE", "BROADCAST_TO"})


def refresh_dtypes(root: UOp) -> UOp:
    """Give pass-through ops the dtype their input actually carries and drop
    CASTs that became no-ops.  After cast insertion a PERMUTE / RESHAPE /
    SLICE keeps the dtype it was built with while its input turned narrow;
    the reference realizer follows numpy's array dtype there (the value is
    what the array holds), so rewriting the IR to the carried dtype changes
    no value and lets later rewrites see the real layout."""
    new: Dict[int, UOp] = {}
    for n in toposort(root):
        if not n.inputs:
            new[id(n)] = n
            continue
        ins = tuple(new.get(id(i), i) for i in n.inputs)
        dtype = n.dtype
        if n.op in _PASS_THROUGH:
            dtype = ins[0].dtype
        elif n.op == OP_WHERE and not (isinstance(n.arg, dict) and n.arg.get("autocast_hint")):
            from .tensor import promote
            dtype = promote(ins[1].dtype, ins[2].dtype)
        if n.op == OP_CAST and ins[0].dtype == n.dtype:
            new[id(n)] = ins[0]
            continue
        if dtype == n.dtype and all(a is b for a, b in zip(ins, n.inputs)):
            new[id(n)] = n
        else:
            new[id(n)] = UOp(n.op, ins, n.shape, dtype, n.arg)
    return new[id(root)]


# ---- head split / merge as strided views of the QKV GEMM -------------------------

def _head_split(x: UOp, narrow: str):
    """x = CAST_narrow(PERMUTE(0,2,1,3)(RESHAPE(B,S,H,D)(SLICE(L, last axis))))
    -> (L, start, interior nodes) or None."""
    if x.op != OP_CAST or x.dtype != narrow:
        return None
    p = x.inputs[0]
    if p.op != OP_PERMUTE or tuple(p.arg["axes"]) != (0, 2, 1, 3):
        return None
    r = p.inputs[0]
    if r.op != OP_RESHAPE or len(r.shape) != 4:
        return None
    sl = r.inputs[0]
    if sl.op != OP_SLICE:
        return None
    src = sl.inputs[0]
    slices = sl.arg["slices"]
    if len(src.shape) != 3 or any(tuple(t) != (0, d, 1) for t, d in zip(slices[:-1], src.shape[:-1])):
        return None
    start, stop, step = slices[-1]
    b, s, h, d = r.shape
    if step != 1 or stop - start != h * d or (b, s) != src.shape[:2]:
        return None
    return src, int(start), [x, p, r, sl]


def _rewrite_attention_views(root: UOp) -> UOp:
    cons = consumers_of(root)
    subs: Dict[int, UOp] = {}
    for att in toposort(root):
        if att.op != OP_HIP_ATTENTION or not att.arg.get("round_scores") or att.dtype not in NARROW:
            continue
        parts = [_head_split(x, att.dtype) for x in att.inputs]
        if any(p is None for p in parts) or len({id(p[0]) for p in parts}) != 1:
            continue
        lin = parts[0][0]
        if lin.op != OP_HIP_LINEAR or lin.dtype != "float32":
            continue
        interior = [n for p in parts for n in p[2]]
        allowed = {id(n) for n in interior} | {id(att)}
        if not all(_only_consumers(n, cons, allowed) for n in interior + [lin]):
            continue
        b, s, f = lin.shape
        _, h, _, d = att.inputs[0].shape
        lin16 = UOp(OP_HIP_LINEAR, lin.inputs, lin.shape, att.dtype, {**lin.arg, "out_dtype": att.dtype})
        views = [(p[1], s * f, d, f) for p in parts]
        arg = {**att.arg, "views": views, "o_layout": "bhsd"}
        out_node = att
        ac = cons.get(id(att), [])
        if len(ac) == 1 and ac[0].op == OP_PERMUTE and tuple(ac[0].arg["axes"]) == (0, 2, 1, 3):
            perm = ac[0]
            pc = cons.get(id(perm), [])
            if len(pc) == 1 and pc[0].op == OP_RESHAPE and pc[0].shape == (b, s, h * d):
                new_att = UOp(OP_HIP_ATTENTION, (lin16, lin16, lin16), (b, s, h, d), att.dtype,
                              {**arg, "o_layout": "bshd"})
                subs[id(pc[0])] = UOp(OP_RESHAPE, (new_att,), pc[0].shape, att.dtype, pc[0].arg)
                continue
        subs[id(out_node)] = UOp(OP_HIP_ATTENTION, (lin16, lin16, lin16), att.shape, att.dtype, arg)
    return substitute(root, subs)


def _rewrite_narrow_stores(root: UOp) -> UOp:
    """A linear or LayerNorm whose only reader casts it to a narrow dtype
    stores that dtype directly (the cast's rounding is the store's rounding;
    both compute in float32 up to the store)."""
    cons = consumers_of(root)
    subs: Dict[int, UOp] = {}
    for n in toposort(root):
        if n.op not in (OP_HIP_LINEAR, OP_LAYER_NORM) or n.dtype != "float32":
            continue
        c = cons.get(id(n), [])
        if len(c) == 1 and c[0].op == OP_CAST and c[0].dtype in NARROW:
            arg = {**n.arg, "out_dtype": c[0].dtype} if n.op == OP_HIP_LINEAR else n.arg
            subs[id(c[0])] = UOp(n.op, n.inputs, n.shape, c[0].dtype, arg)
    return substitute(root, subs)


def _is_seed_cast(n: UOp) -> bool:
    """CAST of a seed buffer: left to the walker, which caches the result."""
    return n.op == OP_CAST and _buffer_of(n.inputs[0]) is not None


# ---- elementwise DAGs (+ last-axis reduce) --------------------------------------

def _grow_dag(top: UOp, cons: Dict[int, List[UOp]], taken: Set[int]) -> List[UOp]:
    """Largest lowerable sub-DAG under `top` whose interior nodes are read
    only inside it; topological order, top last."""
    inside: Set[int] = {id(top)}
    members = [top]
    frontier = [top]
    while frontier:
        n = frontier.pop()
        for i in n.inputs:
            if id(i) in inside or id(i) in taken or not lowerable(i) or i.op == OP_CONST or _is_seed_cast(i):
                continue
            if all(id(c) in inside for c in cons.get(id(i), [])):
                inside.add(id(i))
                members.append(i)
                frontier.append(i)
    # a member whose consumers are not all inside (possible when a later
    # member adds a consumer path) is not a valid interior: drop and retry
    order = [n for n in toposort(top) if id(n) in inside]
    return order


def hip_fuse(root: UOp, bt: BufferTable) -> UOp:
    root = refresh_dtypes(root)
    # 1. attention
    cons = consumers_of(root)
    subs: Dict[int, UOp] = {}
    for n in toposort(root):
        m = _match_attention(n, cons, bt)
        if m is not None:
            subs[id(n)] = m[0]
    root = substitute(root, subs)
    # 2. linear (+ activation)
    cons = consumers_of(root)
    subs = {}
    taken: Set[int] = set()
    for n in toposort(root):
        if id(n) in taken:
            continue
        m = _match_linear(n, cons)
        if m is None:
            continue
        fused, out, interior = m
        if any(id(x) in taken for x in interior):
            continue
        subs[id(out)] = fused
        taken.update(id(x) for x in interior)
        taken.add(id(out))
    root = substitute(root, subs)
    root = _fold_residual_adds(root)
    root = _rewrite_attention_views(root)
    root = _rewrite_narrow_stores(root)
    # 3. softmax outside attention: the reference matcher
    root = fuse(root, include_elementwise=False)
    # 4. elementwise DAGs, with a last-axis reduction where one ends in REDUCE
    cons = consumers_of(root)
    subs = {}
    taken = set()
    for n in reversed(toposort(root)):
        if id(n) in taken:
            continue
        if (n.op == OP_REDUCE and isinstance(n.arg, dict) and n.arg.get("op") in ("sum", "mean", "max")
                and n.inputs and len(n.inputs[0].shape) >= 1 and n.dtype in ("float32", "float16", "bfloat16")):
            src = n.inputs[0]
            axis = n.arg.get("axis")
            nd = len(src.shape)
            last = axis is not None and not isinstance(axis, (tuple, list)) and axis % max(nd, 1) == nd - 1
            if last and lowerable(src) and id(src) not in taken and len(cons.get(id(src), [])) == 1:
                dag = _grow_dag(src, cons, taken)
                try:
                    prog = compile_program(dag, src)
                except (NotLowerable, ProgramTooLarge):
                    prog = None
                if prog is not None:
                    subs[id(n)] = UOp(OP_HIP_REDUCE_FUSED, tuple(prog.inputs), n.shape, n.dtype,
                                      {"program": prog, "reduce": n.arg["op"], "keepdims": bool(n.arg.get("keepdims"))})
                    taken.update(id(x) for x in dag)
                    taken.add(id(n))
                    continue
        if lowerable(n) and n.op != OP_CONST and not _is_seed_cast(n):
            dag = _grow_dag(n, cons, taken)
            if len(dag) == 1 and n.op == OP_CAST and n.inputs[0].op == OP_CONST:
                continue  # constant folding is done by the consumer's program
            try:
                prog = compile_program(dag, n)
            except (NotLowerable, ProgramTooLarge):
                continue
            subs[id(n)] = UOp(OP_HIP_REDUCE_FUSED, tuple(prog.inputs), n.shape, n.dtype,
                              {"program": prog, "reduce": None, "keepdims": False})
            taken.update(id(x) for x in dag)
    return substitute(root, subs)


__all__ = ["hip_fuse", "ACT_NONE", "ACT_RELU", "ACT_GELU"]
