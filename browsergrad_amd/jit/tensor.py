"""Graph building: a minimal tensor proxy over the UOp IR.

Builds the same UOp graphs as the reference's tracing API for the ops on the
realizer path, so the AMP pass, fusion and the walker see what they would see
behind `bg.realize_webgpu` (packages/browsergrad-jit/src/python):

  * binary ops broadcast with numpy rules and take numpy's promoted dtype
    (_tensor_proxy.py:449-464, 699-723); Python scalars become 0-d CONST
    leaves of numpy's dtype for them (float -> float64, _tensor_proxy.py:
    2098-2110); `a - b` is ADD(a, NEG(b)) (:731-732)
  * comparisons build CMP -> bool (:857-882); `where` builds WHERE with
    arg None (:2449-2470)
  * reductions build REDUCE {op, axis, keepdims} (:1178-1257)
  * permute / transpose / .T build PERMUTE {axes}; reshape builds RESHAPE
    {new_shape} (:1598-1735)
  * inside `autocast()` every op the AMP policy covers is stamped with
    arg["autocast_hint"] (:425-446)
  * functional forms follow _functional.py: relu (:99-111), tanh (:122-126),
    gelu (:129-133), softmax (:149-166), linear (:741-749), layer_norm
    (:752-812), scaled_dot_product_attention (:1505-1533)

Seed data lives in a BufferTable (buffers.py); every `from_numpy` is
LOAD(BUFFER(id)).
"""
from __future__ import annotations

import contextlib
import threading
from typing import Any, Optional, Sequence, Tuple

import numpy as np

from ..errors import JitNotImplementedError
from .buffers import BufferTable
from .ir import (
    OP_ADD, OP_CAST, OP_CMP, OP_CONST, OP_DIV, OP_EXP, OP_LAYER_NORM, OP_LOG, OP_MATMUL, OP_MUL,
    OP_NEG, OP_PERMUTE, OP_REDUCE, OP_RESHAPE, OP_SLICE, OP_WHERE, ShapeError, UOp, buffer, load,
)

_TLS = threading.local()


def active_autocast() -> Optional[str]:
    return getattr(_TLS, "amp_dtype", None)


@contextlib.contextmanager
def autocast(dtype: str = "float16", enabled: bool = True):
    """Tag ops built inside the block for the cast-insertion pass
    (_amp.py:82-150).  The reference accepts float16 only; "bfloat16" is an
    extension of this build (MI355X has native bf16 MFMA)."""
    if dtype not in ("float16", "bfloat16", "float32"):
        raise NotImplementedError(f"autocast dtype={dtype!r} not supported")
    prev = active_autocast()
    if enabled and dtype != "float32":
        _TLS.amp_dtype = dtype
    try:
        yield
    finally:
        _TLS.amp_dtype = prev


def _amp_arg(arg: Any = None) -> Any:
    active = active_autocast()
    if active is None:
        return arg
    if arg is None:
        return {"autocast_hint": active}
    if isinstance(arg, dict):
        return {**arg, "autocast_hint": active}
    return arg


def _np_dtype(name: str) -> np.dtype:
    return np.dtype(np.float32) if name == "bfloat16" else np.dtype(name)


def promote(a: str, b: str) -> str:
    """numpy.promote_types on dtype names; bfloat16 promotes like float16
    against wider floats and stays bfloat16 against itself."""
    if a == b:
        return a
    if "bfloat16" in (a, b):
        other = b if a == "bfloat16" else a
        return other if other in ("float32", "float64") else "float32"
    return np.promote_types(np.dtype(a), np.dtype(b)).name


def broadcast_shape(*shapes: Tuple[int, ...]) -> Tuple[int, ...]:
    try:
        return tuple(int(d) for d in np.broadcast_shapes(*shapes))
    except ValueError as e:
        raise ShapeError(f"shapes {shapes} are not broadcastable: {e}") from e


class Tensor:
    """A node of the graph being built plus the session it belongs to."""

    __slots__ = ("uop", "session")

    def __init__(self, uop: UOp, session: "Session") -> None:
        self.uop = uop
        self.session = session

    # -- metadata
    @property
    def shape(self) -> Tuple[int, ...]:
        return self.uop.shape

    @property
    def dtype(self) -> str:
        return self.uop.dtype

    @property
    def ndim(self) -> int:
        return len(self.uop.shape)

    def numel(self) -> int:
        return self.uop.numel

    def _wrap(self, uop: UOp) -> "Tensor":
        return Tensor(uop, self.session)

    def _lift(self, value: Any) -> "Tensor":
        return self.session.lift(value)

    # -- arithmetic (_tensor_proxy.py:699-771)
    def _binop(self, other: Any, op: str) -> "Tensor":
        rhs = self._lift(other)
        return self._wrap(UOp(op, (self.uop, rhs.uop), broadcast_shape(self.shape, rhs.shape),
                              promote(self.dtype, rhs.dtype), _amp_arg(None)))

    def __add__(self, o: Any) -> "Tensor":
        return self._binop(o, OP_ADD)

    def __radd__(self, o: Any) -> "Tensor":
        return self._lift(o).__add__(self)

    def __sub__(self, o: Any) -> "Tensor":
        return self.__add__(-self._lift(o))

    def __rsub__(self, o: Any) -> "Tensor":
        return self._lift(o).__sub__(self)

    def __mul__(self, o: Any) -> "Tensor":
        return self._binop(o, OP_MUL)

    def __rmul__(self, o: Any) -> "Tensor":
        return self._lift(o).__mul__(self)

    def __truediv__(self, o: Any) -> "Tensor":
        return self._binop(o, OP_DIV)

    def __rtruediv__(self, o: Any) -> "Tensor":
        return self._lift(o).__truediv__(self)

    def __neg__(self) -> "Tensor":
        return self._wrap(UOp(OP_NEG, (self.uop,), self.shape, self.dtype, _amp_arg(None)))

    def exp(self) -> "Tensor":
        return self._wrap(UOp(OP_EXP, (self.uop,), self.shape, self.dtype, _amp_arg(None)))

    def log(self) -> "Tensor":
        return self._wrap(UOp(OP_LOG, (self.uop,), self.shape, self.dtype, _amp_arg(None)))

    # -- comparisons (_tensor_proxy.py:857-882)
    def _cmp(self, o: Any, op: str) -> "Tensor":
        rhs = self._lift(o)
        return self._wrap(UOp(OP_CMP, (self.uop, rhs.uop), broadcast_shape(self.shape, rhs.shape), "bool",
                              {"op": op}))

    def __gt__(self, o: Any) -> "Tensor":
        return self._cmp(o, "gt")

    def __ge__(self, o: Any) -> "Tensor":
        return self._cmp(o, "ge")

    def __lt__(self, o: Any) -> "Tensor":
        return self._cmp(o, "lt")

    def __le__(self, o: Any) -> "Tensor":
        return self._cmp(o, "le")

    # -- matmul: numpy matmul shape rules (2-D, batched, broadcast batch)
    def __matmul__(self, o: Any) -> "Tensor":
        rhs = self._lift(o)
        a, b = self.shape, rhs.shape
        if len(a) < 2 or len(b) < 2:
            raise ShapeError(f"matmul needs rank >= 2 operands, got {a} @ {b}")
        if a[-1] != b[-2]:
            raise ShapeError(f"matmul inner dims mismatch: {a} @ {b}")
        batch = broadcast_shape(a[:-2], b[:-2])
        return self._wrap(UOp(OP_MATMUL, (self.uop, rhs.uop), batch + (a[-2], b[-1]),
                              promote(self.dtype, rhs.dtype), _amp_arg(None)))

    # -- reductions (_tensor_proxy.py:1178-1257)
    def _reduce(self, op: str, axis: Any = None, keepdims: bool = False) -> "Tensor":
        if axis is None:
            out = (1,) * self.ndim if keepdims else ()
        else:
            axes = (axis,) if isinstance(axis, int) else tuple(axis)
            red = tuple(a % self.ndim for a in axes)
            out = tuple((1 if keepdims else None) if i in red else d for i, d in enumerate(self.shape))
            out = tuple(d for d in out if d is not None)
        return self._wrap(UOp(OP_REDUCE, (self.uop,), out, self.dtype,
                              _amp_arg({"op": op, "axis": axis, "keepdims": keepdims})))

    def sum(self, axis: Any = None, keepdims: bool = False) -> "Tensor":
        return self._reduce("sum", axis, keepdims)

    def mean(self, axis: Any = None, keepdims: bool = False) -> "Tensor":
        return self._reduce("mean", axis, keepdims)

    def max(self, axis: Any = None, keepdims: bool = False) -> "Tensor":
        return self._reduce("max", axis, keepdims)

    # -- shape ops
    def reshape(self, *shape: Any) -> "Tensor":
        new = tuple(shape[0]) if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else tuple(shape)
        if -1 in new:
            known = int(np.prod([d for d in new if d != -1]))
            new = tuple(self.numel() // known if d == -1 else d for d in new)
        if int(np.prod(new)) != self.numel():
            raise ShapeError(f"reshape: shape {new} does not match numel {self.numel()}")
        return self._wrap(UOp(OP_RESHAPE, (self.uop,), tuple(int(d) for d in new), self.dtype,
                              {"new_shape": tuple(int(d) for d in new)}))

    def permute(self, *axes: int) -> "Tensor":
        if len(axes) == 1 and isinstance(axes[0], (tuple, list)):
            axes = tuple(axes[0])
        if len(axes) != self.ndim:
            raise ShapeError(f"permute: expected {self.ndim} axes for shape {self.shape}, got {len(axes)}")
        norm = tuple(a + self.ndim if a < 0 else a for a in axes)
        if sorted(norm) != list(range(self.ndim)):
            raise ShapeError(f"permute: {axes} is not a permutation")
        return self._wrap(UOp(OP_PERMUTE, (self.uop,), tuple(self.shape[a] for a in norm), self.dtype,
                              {"axes": norm}))

    def transpose(self, d0: int, d1: int) -> "Tensor":
        axes = list(range(self.ndim))
        d0 %= self.ndim
        d1 %= self.ndim
        axes[d0], axes[d1] = axes[d1], axes[d0]
        return self.permute(*axes)

    @property
    def T(self) -> "Tensor":  # noqa: N802 - numpy name
        return self.permute(*reversed(range(self.ndim)))

    def slice(self, dim: int, start: int, stop: int) -> "Tensor":
        """x[..., start:stop, ...] along `dim` (basic slicing, step 1)."""
        dim %= self.ndim
        start, stop, _ = slice(start, stop).indices(self.shape[dim])
        slices = tuple((start, stop, 1) if i == dim else (0, d, 1) for i, d in enumerate(self.shape))
        shape = tuple(max(stop - start, 0) if i == dim else d for i, d in enumerate(self.shape))
        return self._wrap(UOp(OP_SLICE, (self.uop,), shape, self.dtype, {"slices": slices}))

    def cast(self, dtype: str) -> "Tensor":
        return self._wrap(UOp(OP_CAST, (self.uop,), self.shape, dtype, {"dtype": dtype}))

    def numpy(self) -> np.ndarray:
        """Realize through the registered HIP bridge (realize.realize_hip)."""
        from .realize import realize_hip
        return realize_hip(self.uop, self.session.buffers)


class Session:
    """Owns the BufferTable that BUFFER leaves refer to."""

    def __init__(self, buffers: Optional[BufferTable] = None) -> None:
        self.buffers = buffers if buffers is not None else BufferTable()

    def from_numpy(self, arr: np.ndarray, name: Optional[str] = None) -> Tensor:
        arr = np.asarray(arr)
        bid = self.buffers.new_buffer(arr, name=name)
        return Tensor(load(buffer(bid, tuple(int(d) for d in arr.shape), arr.dtype.name)), self)

    def full(self, shape: Sequence[int], value: float, dtype: str = "float32") -> Tensor:
        """np.full(...) uploaded as a buffer; the table keeps the fill value
        so passes can recognise a broadcast scalar without reading it."""
        bid = self.buffers.new_full(tuple(int(d) for d in shape), value, dtype)
        return Tensor(load(buffer(bid, tuple(int(d) for d in shape), dtype)), self)

    def lift(self, value: Any) -> Tensor:
        if isinstance(value, Tensor):
            return value
        if isinstance(value, (bool, int, float, np.floating, np.integer)):
            dt = np.asarray(value).dtype.name
            return Tensor(UOp(OP_CONST, (), (), dt, {"value": value}), self)
        if isinstance(value, np.ndarray):
            return self.from_numpy(value)
        raise TypeError(f"cannot lift {type(value).__name__} into the graph")

    def const(self, value: float, dtype: str) -> Tensor:
        return Tensor(UOp(OP_CONST, (), (), dtype, {"value": value}), self)


# ---- functional forms (_functional.py) --------------------------------------

def where(cond: Tensor, a: Any, b: Any) -> Tensor:
    s = cond.session
    lhs, rhs = s.lift(a), s.lift(b)
    if cond.dtype != "bool":
        raise ShapeError(f"where: condition dtype must be bool, got {cond.dtype!r}")
    return Tensor(UOp(OP_WHERE, (cond.uop, lhs.uop, rhs.uop), broadcast_shape(cond.shape, lhs.shape, rhs.shape),
                      promote(lhs.dtype, rhs.dtype), None), s)


def relu(x: Tensor) -> Tensor:
    zero = x.session.const(0.0, x.dtype)
    return where(x > zero, x, zero)


def tanh(x: Tensor) -> Tensor:
    e_pos = x.exp()
    e_neg = (-x).exp()
    return (e_pos - e_neg) / (e_pos + e_neg)


def gelu(x: Tensor) -> Tensor:
    c = (2.0 / np.pi) ** 0.5
    s = x.session
    return 0.5 * x * (s.lift(1.0) + tanh(s.lift(c) * (x + 0.044715 * x * x * x)))


def softmax(x: Tensor, dim: int = -1) -> Tensor:
    x_max = x.max(axis=dim, keepdims=True)
    shifted = x - x_max
    e = shifted.exp()
    s = e.sum(axis=dim, keepdims=True)
    return e / s


def linear(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None) -> Tensor:
    out = x @ weight.T
    if bias is not None:
        out = out + bias
    return out


def layer_norm(x: Tensor, normalized_shape: Any, weight: Optional[Tensor] = None, bias: Optional[Tensor] = None,
               eps: float = 1e-5) -> Tensor:
    ns = (int(normalized_shape),) if isinstance(normalized_shape, int) else tuple(int(v) for v in normalized_shape)
    if x.shape[-len(ns):] != ns:
        raise ShapeError(f"layer_norm: input trailing shape {x.shape[-len(ns):]} does not match {ns}")
    cols = int(np.prod(ns))
    rows = x.numel() // cols
    s = x.session
    w = weight if weight is not None else s.from_numpy(np.ones(ns, dtype=np.float32))
    b = bias if bias is not None else s.from_numpy(np.zeros(ns, dtype=np.float32))
    arg = {"normalized_shape": ns, "rows": rows, "cols": cols, "eps": float(eps)}
    return Tensor(UOp(OP_LAYER_NORM, (x.uop, w.uop, b.uop), x.shape, x.dtype, arg), s)


def scaled_dot_product_attention(q: Tensor, k: Tensor, v: Tensor, is_causal: bool = False,
                                 scale: Optional[float] = None) -> Tensor:
    s_val = (1.0 / np.sqrt(q.shape[-1])) if scale is None else float(scale)
    scores = q @ k.transpose(-1, -2)
    scale_t = q.session.full(scores.shape, s_val, "float32")
    scores = scores * scale_t
    if is_causal:
        lq, lk = scores.shape[-2], scores.shape[-1]
        mask = q.session.buffers.new_causal_mask(lq, lk)
        mask_t = Tensor(load(buffer(mask, (lq, lk), "bool")), q.session)
        fill = q.session.const(float("-inf"), scores.dtype)
        scores = Tensor(UOp(OP_WHERE, (mask_t.uop, fill.uop, scores.uop), scores.shape, scores.dtype,
                            "masked_fill"), q.session)
    attn = softmax(scores, dim=-1)
    return attn @ v


def attention_forward(q: Tensor, k: Tensor, v: Tensor) -> Tensor:
    """Typed dense rank-4 float32 attention forward (bg.kernels.attention_forward,
    packages/browsergrad-jit/src/python/index.ts:212-245): the contract is
    inferred (shape / dtype / ceilings) and the ATTENTION_FORWARD node carries
    the canonical scale and mask "none"."""
    from .attention_forward import infer_attention_forward_contract, validate_attention_forward_node
    from .ir import OP_ATTENTION_FORWARD
    if any(type(t) is not Tensor for t in (q, k, v)):
        raise TypeError("bg.kernels.attention_forward requires Tensor inputs for query, key, and value")
    if k.session is not q.session or v.session is not q.session:
        raise ShapeError("bg.kernels.attention_forward inputs must belong to one session")
    c = infer_attention_forward_contract(q.uop, k.uop, v.uop)
    uop = UOp(OP_ATTENTION_FORWARD, (q.uop, k.uop, v.uop), c.output_shape, "float32",
              {"scale": c.scale, "mask": "none"})
    validate_attention_forward_node(uop)
    return Tensor(uop, q.session)


def flash_attention(q: Tensor, k: Tensor, v: Tensor, mask: Any = None, scale: Any = None) -> Tensor:
    """Compatibility alias of attention_forward (index.ts:248-265): masks and
    custom scales are refused."""
    if mask is not None or scale is not None:
        raise JitNotImplementedError(
            "bg.kernels.flash_attention now aliases the exact typed attention_forward v1 profile and accepts "
            "neither additive masks nor custom scale. Use torch.nn.functional.scaled_dot_product_attention for "
            "those semantics.")
    return attention_forward(q, k, v)


def _tup(v: Any, r: int) -> Tuple[int, ...]:
    return tuple(int(a) for a in v) if isinstance(v, (tuple, list)) else (int(v),) * r


def _conv_nd(x: Tensor, w: Tensor, bias: Optional[Tensor], stride: Any, padding: Any, dilation: Any,
             groups: int, r: int) -> Tensor:
    """CONV1D / CONV2D / CONV3D graph node with the reference plan's arg
    fields (tensor_plan.ts:715-790) and has_bias (_realize.py:413-583)."""
    if x.dtype != "float32" or w.dtype != "float32":
        raise ShapeError(f"conv{r}d: float32 tensors only (got {x.dtype}, {w.dtype})")
    if len(x.shape) != r + 2 or len(w.shape) != r + 2:
        raise ShapeError(f"conv{r}d: input and weight must have rank {r + 2}")
    n, c = x.shape[:2]
    o, cpg = w.shape[:2]
    k = w.shape[2:]
    s, p, d = _tup(stride, r), _tup(padding, r), _tup(dilation, r)
    if c % groups or o % groups or cpg != c // groups:
        raise ShapeError(f"conv{r}d: weight {w.shape} does not match {c} channels in {groups} groups")
    ins = x.shape[2:]
    out = tuple((ins[i] + 2 * p[i] - d[i] * (k[i] - 1) - 1) // s[i] + 1 for i in range(r))
    if any(v <= 0 for v in out):
        raise ShapeError(f"conv{r}d: output size {out} is not positive")
    if r == 1:
        arg = {"n": n, "c_in": c, "l_in": ins[0], "c_out": o, "k": k[0], "stride": s[0], "padding": p[0],
               "dilation": d[0], "groups": groups, "l_out": out[0]}
    else:
        axes = ("h", "w") if r == 2 else ("d", "h", "w")
        arg = {"n": n, "c_in": c, "c_out": o, "groups": groups}
        for i, a in enumerate(axes):
            arg.update({a: ins[i], f"k{a}": k[i], f"stride_{a}": s[i], f"pad_{a}": p[i], f"dilation_{a}": d[i],
                        f"out_{a}": out[i]})
    arg["has_bias"] = bias is not None
    inputs = (x.uop, w.uop) + ((bias.uop,) if bias is not None else ())
    return x._wrap(UOp(f"CONV{r}D", inputs, (n, o) + out, "float32", arg))


def conv1d(x: Tensor, w: Tensor, bias: Optional[Tensor] = None, stride: Any = 1, padding: Any = 0,
           dilation: Any = 1, groups: int = 1) -> Tensor:
    return _conv_nd(x, w, bias, stride, padding, dilation, groups, 1)


def conv2d(x: Tensor, w: Tensor, bias: Optional[Tensor] = None, stride: Any = 1, padding: Any = 0,
           dilation: Any = 1, groups: int = 1) -> Tensor:
    return _conv_nd(x, w, bias, stride, padding, dilation, groups, 2)


def conv3d(x: Tensor, w: Tensor, bias: Optional[Tensor] = None, stride: Any = 1, padding: Any = 0,
           dilation: Any = 1, groups: int = 1) -> Tensor:
    return _conv_nd(x, w, bias, stride, padding, dilation, groups, 3)


__all__ = [
    "conv1d", "conv2d", "conv3d",
    "Tensor", "Session", "autocast", "active_autocast", "promote", "broadcast_shape",
    "where", "relu", "tanh", "gelu", "softmax", "linear", "layer_norm", "scaled_dot_product_attention",
    "attention_forward", "flash_attention",
]
