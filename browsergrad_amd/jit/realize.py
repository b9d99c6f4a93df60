"""The walker: realize a UOp graph through the HIP bridge.

Mirrors packages/browsergrad-jit/src/python/_realize_webgpu.py:
  * realize_hip           <- realize_webgpu (:374-473): toposort, last-use
    release of owned handles, BUFFER / LOAD handles owned by the
    GpuBufferTable across calls, root materialised once then released,
    JitNotImplementedError for unsupported ops, RealizationError wrapping any
    other handler failure with op / shape / dtype.
  * realize_tensor_plan_hip / _resident / materialize_gpu_buffer <- the plan
    route (:476-589): the graph becomes a tensor plan (gpu_plan.py) run by
    the bridge's run_tensor_plan[_semantic][_resident].
  * register_hip_bridge / unregister / get_registered_* <- the bridge
    registry (:597-658).

The pipeline before the walk is the reference's (cast insertion, then
fusion) with this build's own rewrites (hip_fusion.py) in between, which map
SDPA, linear layers and elementwise(+reduce) DAGs onto single kernels.  With
`hip_rewrites=False` the walk dispatches the reference's op set one kernel
per (fused) op.

Handlers beyond the reference whitelist (_realize_webgpu.py:347-364) cover
the ops the configs need on the device: single elementwise ops, CMP / WHERE,
REDUCE, RESHAPE, PERMUTE, BROADCAST_TO, LAYER_NORM, FUSED_SOFTMAX, batched
MATMUL and the HIP_* rewrites.  There is no CPU fallback: a graph the device
path cannot run raises.
"""
from __future__ import annotations

import json
from typing import Any, Callable, Dict, List, Optional, Tuple

import numpy as np

from .. import _native as N
from ..errors import JitNotImplementedError, KernelError
from . import config
from .amp import insert_cast_pass
from .attention_forward import validate_attention_forward_node
from .buffers import BufferTable, GpuBufferTable
from .fusion import fuse, substitute
from .gpu_plan import GpuPlanUnsupported, build_gpu_execution_plan, build_gpu_execution_submission
from .hip_fusion import hip_fuse, refresh_dtypes
from .ir import (
    CONV_OPS,
    OP_ADD, OP_ATTENTION_FORWARD, OP_BROADCAST_TO, OP_BUFFER, OP_CAST, OP_CMP, OP_CONST, OP_CUSTOM, OP_DIV,
    OP_EXP, OP_FUSED_ELEMENTWISE, OP_FUSED_SOFTMAX, OP_HIP_ATTENTION, OP_HIP_LINEAR, OP_HIP_REDUCE_FUSED,
    OP_CAUSAL_MASK, OP_LAYER_NORM, OP_LOAD, OP_LOG, OP_MATMUL, OP_MUL, OP_NEG, OP_PERMUTE, OP_REDUCE, OP_RESHAPE,
    OP_SLICE, OP_WHERE,
    UOp, toposort,
)
from .program import NotLowerable, ProgramTooLarge, broadcast_strides, compile_program


class RealizationError(RuntimeError):
    """The reference's _errors.RealizationError."""


_RED = {"sum": N.RED_SUM, "mean": N.RED_MEAN, "max": N.RED_MAX, "min": N.RED_MIN}


def _np_dtype(name: str) -> np.dtype:
    if name == "bfloat16":
        return np.dtype(np.uint16)
    return np.dtype(name)


class _Walk:
    """State of one realize call: value table + owned handles."""

    def __init__(self, br: Any, gbt: GpuBufferTable, bt: BufferTable) -> None:
        self.br = br
        self.gbt = gbt
        self.bt = bt
        self.vt: Dict[int, int] = {}
        self.borrowed: set = set()  # handles owned by the GpuBufferTable

    def h(self, u: UOp) -> int:
        return self.vt[id(u)]

    def dtype_of(self, u: UOp) -> str:
        """The dtype the value actually holds.  After cast insertion,
        pass-through ops (PERMUTE, RESHAPE, SLICE, ...) keep the dtype they
        were built with while their input became narrow (the reference's
        realizer follows numpy's array dtype there, _amp.py:245-255), so the
        handle, not the IR, is authoritative."""
        h = self.vt.get(id(u))
        if h is None:
            return u.dtype
        return self.br.handle_info(h)["dtype"]

    # -- helpers
    def run_program(self, prog, inputs: Tuple[UOp, ...], reduce: Optional[str] = None,
                    keepdims: bool = False) -> int:
        """`inputs`: the node's own (possibly rewired) inputs, in the
        program's external-input order."""
        ins = [self.h(u) for u in inputs]
        shape = prog.shape or (1,)
        strides = None
        if not all(tuple(u.shape) == tuple(prog.shape) for u in inputs):
            strides = [broadcast_strides(u.shape, shape) for u in inputs]
        out = self.br.fused_ex(ins, prog.ops, shape, prog.out_dtype, in_strides=strides, imms=prog.imms,
                               reduce=_RED[reduce] if reduce else N.RED_NONE, keepdims=keepdims)
        return out

    def permute(self, h: int, shape: Tuple[int, ...], axes: Tuple[int, ...]) -> int:
        cst = [1] * len(shape)
        for i in range(len(shape) - 2, -1, -1):
            cst[i] = cst[i + 1] * shape[i + 1]
        return self.br.copy_strided(h, 0, [shape[a] for a in axes], [cst[a] for a in axes])


# ---- handlers -----------------------------------------------------------------

def _h_buffer(n: UOp, w: _Walk) -> int:
    bid = n.arg
    handle = w.gbt.get(bid)
    if handle is not None:
        return handle
    arr = w.bt.get(bid)
    if n.dtype == "bfloat16":
        raise JitNotImplementedError("HIP walker: bfloat16 seed buffers are uploaded as float32 then cast")
    return w.gbt.upload(bid, np.ascontiguousarray(arr), tuple(arr.shape), arr.dtype.name)


def _h_load(n: UOp, w: _Walk) -> int:
    return w.h(n.inputs[0])


def _h_const(n: UOp, w: _Walk) -> Optional[int]:
    if n.dtype not in ("float32", "float16", "bool"):
        # No device value: the consumers are fused programs, which read a
        # CONST as an immediate (program.py); anything else fails there.
        return None
    arr = np.asarray(n.arg["value"], dtype=_np_dtype(n.dtype))
    return w.br.upload(arr.tobytes(), tuple(arr.shape) or (1,), n.dtype)


def _h_elementwise(n: UOp, w: _Walk) -> int:
    try:
        prog = compile_program([n], n)
    except (NotLowerable, ProgramTooLarge) as e:
        raise JitNotImplementedError(f"HIP walker: {n.op} ({n.dtype}) has no device lowering: {e}") from e
    return w.run_program(prog, tuple(prog.inputs))


def _h_cast(n: UOp, w: _Walk) -> int:
    src = n.inputs[0]
    if src.op == OP_CONST or src.dtype == "bool" or n.dtype == "bool":
        return _h_elementwise(n, w)
    actual = w.dtype_of(src)
    if actual == n.dtype:  # astype to the dtype the array already has
        return w.br.reshape(w.h(src), n.shape or (1,))
    seed = src.inputs[0] if src.op == OP_LOAD and src.inputs[0].op == OP_BUFFER else None
    if seed is not None:
        # A seed buffer's cast is kept resident beside it (weights are cast
        # once per session, like the upload itself).
        key = f"{seed.arg}::{n.dtype}"
        h = w.gbt.get(key)
        if h is None:
            h = w.br.cast(w.h(src), actual, n.dtype, n.shape)
            w.gbt.register(key, h)
        w.borrowed.add(h)
        return h
    return w.br.cast(w.h(src), actual, n.dtype, n.shape)


def _h_matmul(n: UOp, w: _Walk) -> int:
    a, b = n.inputs
    da, db = w.dtype_of(a), w.dtype_of(b)
    if len(a.shape) == 2 and len(b.shape) == 2 and da == db == n.dtype == "float32":
        m, k = a.shape
        return w.br.matmul(w.h(a), w.h(b), m, k, b.shape[1], n.dtype)  # reference method
    m, k, nn = a.shape[-2], a.shape[-1], b.shape[-1]
    batch = int(np.prod(n.shape[:-2])) if len(n.shape) > 2 else 1
    ba = int(np.prod(a.shape[:-2])) if len(a.shape) > 2 else 1
    bb = int(np.prod(b.shape[:-2])) if len(b.shape) > 2 else 1
    if da != db:
        raise RealizationError(f"HIP matmul: operand dtypes differ ({da}, {db})")
    if (ba not in (1, batch)) or (bb not in (1, batch)) or (ba == 1 and bb == 1 and batch != 1):
        raise JitNotImplementedError(f"HIP matmul: batch broadcast {a.shape} @ {b.shape} not supported")
    if bb == 1 and ba == batch and len(b.shape) == 2:
        # batch folds into M (contiguous A)
        hnd = w.br.matmul_ex(w.h(a), w.h(b), m=m * batch, n=nn, k=k, in_dtype=da, out_dtype=n.dtype)
    else:
        hnd = w.br.matmul_ex(w.h(a), w.h(b), m=m, n=nn, k=k, batch=batch,
                             stride_a=0 if ba == 1 else m * k, stride_b=0 if bb == 1 else k * nn,
                             in_dtype=da, out_dtype=n.dtype)
    if _info_shape(w, hnd) == n.shape:
        return hnd
    out = w.br.reshape(hnd, n.shape)
    w.br.release(hnd)
    return out


def _info_shape(w: _Walk, h: int) -> Tuple[int, ...]:
    return tuple(w.br.handle_info(h)["shape"])


def _h_reduce(n: UOp, w: _Walk) -> int:
    x = n.inputs[0]
    op = n.arg["op"]
    if op not in _RED:
        raise JitNotImplementedError(f"HIP walker: REDUCE {op!r} has no device kernel")
    rank = len(x.shape)
    axis = n.arg.get("axis")
    axes = tuple(range(rank)) if axis is None else ((axis,) if isinstance(axis, int) else tuple(axis))
    red = sorted(a % rank for a in axes) if rank else []
    keep = [a for a in range(rank) if a not in red]
    hx = w.h(x)
    owned = None
    if red != list(range(rank - len(red), rank)):
        hx = owned = w.permute(hx, x.shape, tuple(keep + red))
    cols = int(np.prod([x.shape[a] for a in red])) if red else 1
    rows = x.numel // max(cols, 1)
    out = w.br.reduce_last(hx, rows, cols, _RED[op])
    if owned is not None:
        w.br.release(owned)
    res = w.br.reshape(out, n.shape or (1,))
    w.br.release(out)
    return res


def _h_reshape(n: UOp, w: _Walk) -> int:
    return w.br.reshape(w.h(n.inputs[0]), n.shape or (1,))


def _h_permute(n: UOp, w: _Walk) -> int:
    x = n.inputs[0]
    return w.permute(w.h(x), x.shape, tuple(n.arg["axes"]))


def _h_slice(n: UOp, w: _Walk) -> int:
    x = n.inputs[0]
    cst = [1] * len(x.shape)
    for i in range(len(x.shape) - 2, -1, -1):
        cst[i] = cst[i + 1] * x.shape[i + 1]
    sl = n.arg["slices"]
    offset = sum(int(s[0]) * c for s, c in zip(sl, cst))
    strides = [int(s[2]) * c for s, c in zip(sl, cst)]
    return w.br.copy_strided(w.h(x), offset, n.shape, strides)


def _h_broadcast_to(n: UOp, w: _Walk) -> int:
    x = n.inputs[0]
    return w.br.copy_strided(w.h(x), 0, n.shape, broadcast_strides(x.shape, n.shape))


def _h_layer_norm(n: UOp, w: _Walk) -> int:
    x, wt, b = n.inputs
    a = n.arg
    out = w.br.layer_norm(w.h(x), w.h(wt), w.h(b), int(a["rows"]), int(a["cols"]), float(a.get("eps", 1e-5)),
                          n.dtype)
    return out


def _conv_desc(op: str, arg: dict) -> Tuple[str, dict]:
    """(conv_ex op, geometry) of a CONV* node from the plan's arg fields."""
    kind = "forward"
    for suffix, name in (("_BACKWARD_INPUT", "backward_input"), ("_BACKWARD_WEIGHT", "backward_weight"),
                         ("_BACKWARD_BIAS", "backward_bias")):
        if op.endswith(suffix):
            kind, op = name, op[: -len(suffix)]
    transposed = op == "CONV_TRANSPOSE2D"
    r = 1 if op == "CONV1D" else 3 if op == "CONV3D" else 2
    a = {k: int(v) for k, v in arg.items() if not isinstance(v, bool)}
    if r == 1:
        geo = dict(in_size=(a["l_in"],), out_size=(a["l_out"],), k=(a["k"],), stride=(a["stride"],),
                   pad=(a["padding"],), dilation=(a["dilation"],))
    else:
        axes = ("h", "w") if r == 2 else ("d", "h", "w")
        geo = dict(in_size=tuple(a[x] for x in axes), out_size=tuple(a[f"out_{x}"] for x in axes),
                   k=tuple(a[f"k{x}"] for x in axes), stride=tuple(a[f"stride_{x}"] for x in axes),
                   pad=tuple(a[f"pad_{x}"] for x in axes), dilation=tuple(a[f"dilation_{x}"] for x in axes))
        if transposed:
            geo["output_pad"] = tuple(a[f"output_pad_{x}"] for x in axes)
    geo.update(n=a["n"], c_in=a["c_in"], c_out=a["c_out"], groups=a["groups"], transposed=transposed)
    return kind, geo


def _h_conv(n: UOp, w: _Walk) -> int:
    """CONV1D / CONV2D / CONV3D / CONV_TRANSPOSE2D and their backward forms
    (_realize.py:413-1005) on bg_conv_ex."""
    kind, geo = _conv_desc(n.op, n.arg)
    hs = [w.h(i) for i in n.inputs]
    a = hs[0]
    b = hs[1] if len(hs) > 1 else 0
    bias = hs[2] if kind == "forward" and len(hs) > 2 else 0
    return w.br.conv_ex(kind, a, b, bias, **geo)


def _h_fused_softmax(n: UOp, w: _Walk) -> int:
    x = n.inputs[0]
    axis = n.arg.get("axis")
    rank = len(x.shape)
    axis = rank - 1 if axis is None else axis % rank
    if axis != rank - 1:
        perm = tuple(a for a in range(rank) if a != axis) + (axis,)
        hp = w.permute(w.h(x), x.shape, perm)
        pshape = tuple(x.shape[a] for a in perm)
        hs = w.br.softmax_last(hp, x.numel // x.shape[axis], x.shape[axis], n.dtype)
        w.br.release(hp)
        inv = tuple(int(i) for i in np.argsort(perm))
        out = w.permute(hs, pshape, inv)
        w.br.release(hs)
        return out
    return w.br.softmax_last(w.h(x), x.numel // max(x.shape[-1], 1), x.shape[-1], n.dtype)


def _h_fused_elementwise(n: UOp, w: _Walk) -> int:
    ins = [w.h(i) for i in n.inputs]
    if all(i.numel == n.numel for i in n.inputs) and n.dtype == "float32" and all(i.dtype == "float32"
                                                                                   for i in n.inputs):
        return w.br.fused_elementwise(ins, [list(o) for o in n.arg["ops"]], n.shape or (1,), n.dtype)
    ops = [(o[0], int(o[1]), int(o[2]) if o[2] is not None else int(o[1]), 0) for o in n.arg["ops"]]
    rounds = {"float16": "ROUND_F16", "bfloat16": "ROUND_BF16"}
    if n.dtype in rounds:  # per-op rounding in the narrow dtype
        prog: List[Tuple[str, int, int, int]] = []
        remap: Dict[int, int] = {}
        for i, (code, a, b, c) in enumerate(ops):
            a2 = remap.get(a, a) if a >= 0 else a
            b2 = remap.get(b, b) if b >= 0 else b
            prog.append((code, a2, b2, c))
            prog.append((rounds[n.dtype], len(prog) - 1, 0, 0))
            remap[i] = len(prog) - 1
        ops = prog
    strides = [broadcast_strides(i.shape, n.shape) for i in n.inputs]
    return w.br.fused_ex(ins, ops, n.shape or (1,), n.dtype, in_strides=strides)


def _h_attention_forward(n: UOp, w: _Walk) -> int:
    """ATTENTION_FORWARD (_realize_webgpu.py:280-302): the node must pass the
    typed contract; then the bridge's attention with no mask."""
    c = validate_attention_forward_node(n)
    q, k, v = n.inputs
    return w.br.flash_attention(w.h(q), w.h(k), w.h(v), None, c.batch, c.heads, c.query_length, c.key_length,
                                c.depth, c.scale, n.dtype)


def _round_scores(arg: dict) -> bool:
    """The graph rounds S (arg round_scores); the kernel is asked to repeat
    that rounding only under config.exact_attention_score_rounding, and
    otherwise keeps S in f32 (within the 16-bit tolerance of the graph)."""
    return bool(arg["round_scores"]) and config.attention_rounds_scores()


def _h_hip_attention(n: UOp, w: _Walk) -> int:
    q, k, v = n.inputs
    a = n.arg
    views = a.get("views")
    if views is None:
        b, h, sq, d = q.shape
        sk = k.shape[2]
        return w.br.attention_ex(w.h(q), w.h(k), w.h(v), batch=b, heads=h, sq=sq, sk=sk, d=d, scale=a["scale"],
                                 causal=a["causal"], in_dtype=q.dtype, out_dtype=n.dtype,
                                 round_scores=_round_scores(a))
    # Q / K / V are strided views of one [B, S, 3E] buffer; the output is
    # written [B, H, S, D] or, with o_layout "bshd", [B, S, H, D].
    b, s = q.shape[0], q.shape[1]
    if a["o_layout"] == "bshd":
        _, _, h, d = n.shape
        o_strides = (s * h * d, d, h * d)
    else:
        _, h, _, d = n.shape
        o_strides = (0, 0, 0)
    out = w.br.attention_ex(w.h(q), w.h(k), w.h(v), batch=b, heads=h, sq=s, sk=s, d=d, scale=a["scale"],
                            causal=a["causal"], in_dtype=q.dtype, out_dtype=n.dtype,
                            round_scores=_round_scores(a), q_view=tuple(views[0]), k_view=tuple(views[1]),
                            v_view=tuple(views[2]), o_strides=o_strides)
    if a["o_layout"] == "bshd":
        view = w.br.reshape(out, n.shape)
        w.br.release(out)
        return view
    return out


def _h_hip_linear(n: UOp, w: _Walk) -> int:
    a, wt, bias = n.inputs[:3]
    arg = n.arg
    k = a.shape[-1]
    m = a.numel // k
    nn = wt.shape[0] if arg["trans_b"] else wt.shape[1]
    extra = {"residual": w.h(n.inputs[3])} if arg.get("residual") else {}
    hnd = w.br.matmul_ex(w.h(a), w.h(wt), m=m, n=nn, k=k, trans_b=arg["trans_b"], in_dtype=arg["in_dtype"],
                         out_dtype=arg.get("out_dtype", "float32"), bias=w.h(bias), round_out=arg["round_out"],
                         act=arg["act"], **extra)
    out = w.br.reshape(hnd, n.shape)
    w.br.release(hnd)
    return out


def _h_hip_fused(n: UOp, w: _Walk) -> int:
    return w.run_program(n.arg["program"], n.inputs, n.arg["reduce"], n.arg["keepdims"])


def _h_custom(n: UOp, w: _Walk) -> int:
    raise JitNotImplementedError("HIP walker: CUSTOM ops (user WGSL kernels) have no HIP meaning")


_DISPATCH: Dict[str, Callable[[UOp, _Walk], int]] = {
    OP_BUFFER: _h_buffer,
    OP_LOAD: _h_load,
    OP_CONST: _h_const,
    OP_CAST: _h_cast,
    OP_MATMUL: _h_matmul,
    OP_FUSED_ELEMENTWISE: _h_fused_elementwise,
    OP_ATTENTION_FORWARD: _h_attention_forward,
    OP_CUSTOM: _h_custom,
    # beyond the reference whitelist
    OP_ADD: _h_elementwise, OP_MUL: _h_elementwise, OP_DIV: _h_elementwise, OP_NEG: _h_elementwise,
    OP_EXP: _h_elementwise, OP_LOG: _h_elementwise, OP_CMP: _h_elementwise, OP_WHERE: _h_elementwise,
    OP_REDUCE: _h_reduce,
    OP_RESHAPE: _h_reshape,
    OP_PERMUTE: _h_permute,
    OP_SLICE: _h_slice,
    OP_BROADCAST_TO: _h_broadcast_to,
    OP_LAYER_NORM: _h_layer_norm,
    OP_FUSED_SOFTMAX: _h_fused_softmax,
    OP_HIP_ATTENTION: _h_hip_attention,
    OP_HIP_LINEAR: _h_hip_linear,
    OP_HIP_REDUCE_FUSED: _h_hip_fused,
    **{op: _h_conv for op in CONV_OPS},
}


def supported_opcodes() -> frozenset:
    return frozenset(_DISPATCH)


def prepare(root: UOp, bt: BufferTable, *, hip_rewrites: bool = True) -> UOp:
    """Cast insertion, this build's rewrites, then the reference's fusion
    (both skipped while fusion is disabled, config.use_fusion /
    BG_DISABLE_FUSION, as _realize.py:1891 skips _fusion.fuse)."""
    root = insert_cast_pass(root)
    if not config.fusion_enabled():
        return root
    if hip_rewrites:
        root = hip_fuse(root, bt)
    return fuse(root)


def walk(root: UOp, bt: BufferTable, gbt: GpuBufferTable, *, materialize: bool = True) -> Any:
    """Dispatch a prepared graph; returns the ndarray (materialize=True) or
    the root handle (owned by the caller)."""
    br = gbt.bridge
    order = toposort(root)
    last: Dict[int, int] = {}
    for i, n in enumerate(order):
        for inp in n.inputs:
            last[id(inp)] = i
    w = _Walk(br, gbt, bt)
    owned: Dict[int, int] = {}
    try:
        for i, n in enumerate(order):
            fn = _DISPATCH.get(n.op)
            if fn is None:
                raise JitNotImplementedError(
                    f"HIP realizer: opcode {n.op!r} is not supported. Supported set: {sorted(supported_opcodes())}.")
            try:
                hnd = fn(n, w)
            except (JitNotImplementedError, RealizationError):
                raise
            except Exception as e:  # noqa: BLE001 - wrapped like _realize_webgpu.py:415-424
                raise RealizationError(f"HIP realizer: {n.op} (shape={n.shape}, dtype={n.dtype}) failed: {e}") from e
            w.vt[id(n)] = hnd
            if n.op not in (OP_BUFFER, OP_LOAD) and hnd is not None and hnd not in w.borrowed:
                owned[id(n)] = hnd
            for inp in n.inputs:
                if last.get(id(inp)) == i and id(inp) in owned and inp is not root:
                    br.release(owned.pop(id(inp)))
                    w.vt.pop(id(inp), None)
        # values nobody reads (dead code) other than the root
        for k in [k for k in owned if k != id(root)]:
            br.release(owned.pop(k))
        hroot = w.vt[id(root)]
        if not materialize:
            if root.op in (OP_BUFFER, OP_LOAD):
                return br.reshape(hroot, root.shape or (1,))
            owned.pop(id(root), None)
            return hroot
        dtype = w.dtype_of(root)
        data = br.materialize(hroot, tuple(root.shape), dtype)
        arr = np.frombuffer(data, dtype=_np_dtype(dtype))
        return np.array(arr.reshape(root.shape) if root.shape else arr.reshape(()), copy=True)
    finally:
        for hnd in owned.values():
            br.release(hnd)


# ---- registry (_realize_webgpu.py:597-658) ---------------------------------------

_BRIDGE: Optional[Any] = None
_GBT: Optional[GpuBufferTable] = None


def register_hip_bridge(bridge: Any) -> None:
    global _BRIDGE, _GBT
    if _GBT is not None and bridge is not _BRIDGE:
        _GBT.release_all()
    _BRIDGE = bridge
    _GBT = GpuBufferTable(bridge) if bridge is not None else None


def unregister_hip_bridge() -> None:
    global _BRIDGE, _GBT
    if _GBT is not None:
        _GBT.release_all()
    _BRIDGE = None
    _GBT = None


def get_registered_bridge() -> Optional[Any]:
    return _BRIDGE


def get_registered_gpu_buffer_table() -> Optional[GpuBufferTable]:
    return _GBT


def is_available() -> bool:
    return _BRIDGE is not None


def _table(gbt: Optional[GpuBufferTable]) -> GpuBufferTable:
    t = gbt if gbt is not None else _GBT
    if t is None:
        raise JitNotImplementedError("HIP realizer: no bridge registered (register_hip_bridge(HipRealizerBridge()))")
    return t


def realize_hip(root: UOp, buffers: BufferTable, gpu_buffer_table: Optional[GpuBufferTable] = None, *,
                hip_rewrites: bool = True) -> np.ndarray:
    gbt = _table(gpu_buffer_table)
    return walk(prepare(root, buffers, hip_rewrites=hip_rewrites), buffers, gbt)


# ---- plan route (_realize_webgpu.py:476-589) -------------------------------------------

def _plan_leaves(root: UOp, bt: BufferTable) -> UOp:
    """Leaves the plan can state by value: a LOAD of a full() buffer becomes a
    CONST of its shape (same values, no upload), a LOAD of a causal-mask
    buffer a CAUSAL_MASK step (same values; lets the executor's plan-level
    fuser recognise masked attention without reading the mask)."""
    subs = {}
    for n in toposort(root):
        if n.op != OP_LOAD or not n.inputs or n.inputs[0].op != OP_BUFFER:
            continue
        bid = n.inputs[0].arg
        fill = bt.fill_value(bid)
        if fill is not None:
            subs[id(n)] = UOp(OP_CONST, (), n.shape, n.dtype, {"value": float(fill)})
            continue
        cm = bt.causal_mask(bid)
        if cm is not None:
            subs[id(n)] = UOp(OP_CAUSAL_MASK, (), n.shape, "bool", {"rows": cm[0], "cols": cm[1]})
    return substitute(root, subs) if subs else root


def _plan_submission(root: UOp, bt: BufferTable) -> Tuple[dict, dict, str]:
    """The plan and its semantic side table.  A PERMUTE the side table cannot
    carry (rank other than 2 or 3, or not float32, as in attention's head
    split and K transpose) sends the whole plan down the legacy route: every
    PERMUTE keeps its axes in arg and no requests travel."""
    # Views after cast insertion declare the dtype they were built with while
    # their input turned narrow; the plan states the dtype the data has.
    graph = _plan_leaves(refresh_dtypes(insert_cast_pass(root)), bt)
    try:
        sub = build_gpu_execution_submission(graph)
    except GpuPlanUnsupported as e:
        if "GPU semantic request" not in str(e):
            raise
        plan = build_gpu_execution_plan(graph).summary()
        req = {"requests": []}
        return plan, req, ""
    plan = sub.plan_summary()
    req = sub.semantic_request_summary()
    return plan, req, json.dumps(req, ensure_ascii=True, separators=(",", ":"), sort_keys=True)


def _plan_root_dtype(plan: dict) -> str:
    """dtype of the plan's root after cast insertion (an autocast graph's
    output may be narrower than the graph as built)."""
    return next(st["dtype"] for st in plan["steps"] if st["value_id"] == plan["root_id"])


def _plan_inputs(plan: dict, bt: BufferTable, gbt: GpuBufferTable) -> list:
    inputs = []
    for st in plan["steps"]:
        if st["op"] != OP_BUFFER:
            continue
        bid = st["arg"]
        h = gbt.get(bid)
        if h is not None and not bt.is_materialized(bid):
            inputs.append({"value_id": int(st["value_id"]), "handle": h})
        else:
            arr = bt.get(bid)
            if arr.dtype.name != st["dtype"]:
                raise RealizationError(f"HIP tensor plan: buffer {st['value_id']} dtype mismatch: "
                                       f"plan={st['dtype']} table={arr.dtype.name}")
            inputs.append({"value_id": int(st["value_id"]), "data": np.ascontiguousarray(arr).tobytes()})
    return inputs


def realize_tensor_plan_hip(root: UOp, buffers: BufferTable,
                            gpu_buffer_table: Optional[GpuBufferTable] = None) -> np.ndarray:
    """PERMUTE steps travel in the semantic side table when it can carry them
    (run_tensor_plan_semantic, as _realize_webgpu.py:476-522 requires);
    plans with a PERMUTE it cannot carry (attention's rank-4 head split and
    K transpose) run on the legacy route with the axes in the step arg."""
    gbt = _table(gpu_buffer_table)
    plan, req, req_json = _plan_submission(root, buffers)
    inputs = _plan_inputs(plan, buffers, gbt)
    dtype = _plan_root_dtype(plan)
    if req["requests"]:
        data = gbt.bridge.run_tensor_plan_semantic(plan, req_json, inputs, dtype)
    else:
        data = gbt.bridge.run_tensor_plan(plan, inputs, dtype)
    arr = np.frombuffer(data, dtype=_np_dtype(dtype))
    return np.array(arr.reshape(root.shape) if root.shape else arr.reshape(()), copy=True)


def realize_tensor_plan_hip_resident(root: UOp, buffers: BufferTable,
                                     gpu_buffer_table: Optional[GpuBufferTable] = None) -> str:
    gbt = _table(gpu_buffer_table)
    plan, req, req_json = _plan_submission(root, buffers)
    inputs = _plan_inputs(plan, buffers, gbt)
    dtype = _plan_root_dtype(plan)
    if req["requests"]:
        h = gbt.bridge.run_tensor_plan_resident_semantic(plan, req_json, inputs, dtype)
    else:
        h = gbt.bridge.run_tensor_plan_resident(plan, inputs, dtype)
    bid = buffers.new_unmaterialized_buffer(root.shape, dtype)
    gbt.register(bid, h)
    return bid


def materialize_gpu_buffer(buffer_id: str, *, shape: Tuple[int, ...], dtype: str, buffers: BufferTable,
                           gpu_buffer_table: Optional[GpuBufferTable] = None) -> np.ndarray:
    gbt = _table(gpu_buffer_table)
    h = gbt.get(buffer_id)
    if h is None:
        raise RealizationError(f"HIP buffer {buffer_id!r} is not registered")
    data = gbt.bridge.materialize(h, tuple(shape), dtype)
    arr = np.frombuffer(data, dtype=_np_dtype(dtype))
    out = np.array(arr.reshape(shape) if shape else arr.reshape(()), copy=True)
    buffers.update(buffer_id, out)
    return out


__all__ = [
    "RealizationError", "realize_hip", "prepare", "walk", "supported_opcodes", "register_hip_bridge",
    "unregister_hip_bridge", "get_registered_bridge", "get_registered_gpu_buffer_table", "is_available",
    "realize_tensor_plan_hip", "realize_tensor_plan_hip_resident", "materialize_gpu_buffer",
]
