"""Graph-level NumPy realizer over browsergrad_amd.jit's UOp IR (test infrastructure).

Restates the reference CPU realizer packages/browsergrad-jit/src/python/
_realize.py (`realize`, :1854-1923) handler by handler:

  CONST  np.asarray(value, dtype)                          :187-189
  CAST   astype(arg dtype)                                 :210-212
  ADD MUL DIV NEG EXP LOG                                  :215-243
  CMP    np.equal / less / ...                             :376-393
  MATMUL float16 operands -> f32 @ f32 -> node dtype       :395-412
  LAYER_NORM  mean, centered, var, 1/sqrt(var+eps), x_hat*w + b  :1008-1034
  REDUCE np.sum / max / min / mean with axis, keepdims      :1082-1111
  RESHAPE / PERMUTE                                        :1114-1121
  WHERE  np.where(cond, a, b) in the node dtype            :1453-1459
  FUSED_ELEMENTWISE  the op list in order                  :1557-1600
  FUSED_SOFTMAX  e = exp(x - max); e / sum(e)              :1603-1614
  ATTENTION_FORWARD  execute_attention_forward_arrays
                 (_framework_contracts.py:2881-2932)          :1440-1450

Only cast insertion (browsergrad_amd.jit.amp, which mirrors _amp.py) is
applied before evaluation; fusion does not change values.  Two restatement
choices, both documented at their call site:
  * binary ops between a 0-d operand and an array take the array's float
    dtype (numpy 1.26 value-based casting, the Pyodide 0.26.4 numpy the
    reference runs on); with numpy 2 (NEP 50) a float64 0-d constant would
    otherwise widen a float32 op;
  * bfloat16 (an extension with no reference) is carried as float32 arrays
    holding bf16-representable values, rounded after every bf16-typed op.
Never imported by the product path.
"""
from __future__ import annotations

from typing import Dict

import numpy as np

from browsergrad_amd.jit.amp import insert_cast_pass
from browsergrad_amd.jit.buffers import BufferTable
from browsergrad_amd.jit.ir import UOp, toposort

from .ops import attention_forward_f32, round_bf16

_CMP = {"eq": np.equal, "ne": np.not_equal, "lt": np.less, "le": np.less_equal, "gt": np.greater,
        "ge": np.greater_equal}
_RED = {"sum": np.sum, "max": np.max, "min": np.min, "mean": np.mean}


def _np(dtype: str) -> np.dtype:
    return np.dtype(np.float32) if dtype == "bfloat16" else np.dtype(dtype)


def _fix(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return round_bf16(np.asarray(x, dtype=np.float32))
    return np.asarray(x)


def _operands(n: UOp, vals) -> list:
    """numpy 1.26 value-based casting for 0-d operands against arrays."""
    arrs = [np.asarray(v) for v in vals]
    if len(arrs) == 2:
        a, b = arrs
        if a.ndim == 0 and b.ndim > 0 and a.dtype.kind == b.dtype.kind == "f":
            a = a.astype(b.dtype)
        elif b.ndim == 0 and a.ndim > 0 and a.dtype.kind == b.dtype.kind == "f":
            b = b.astype(a.dtype)
        arrs = [a, b]
    return arrs


def _conv(op: str, arg: dict, ins: list) -> np.ndarray:
    """The CONV* handlers (_realize.py:413-1005) through oracle.ops' conv
    restatements, with the plan's arg fields."""
    from . import ops as O
    kind = "FWD"
    for suffix in ("_BACKWARD_INPUT", "_BACKWARD_WEIGHT", "_BACKWARD_BIAS"):
        if op.endswith(suffix):
            kind, op = suffix, op[: -len(suffix)]
    a = {k: int(v) for k, v in arg.items() if not isinstance(v, bool)}
    if op == "CONV1D":
        ins_, out_, k_ = (a["l_in"],), (a["l_out"],), (a["k"],)
        s_, p_, d_ = (a["stride"],), (a["padding"],), (a["dilation"],)
    else:
        axes = ("h", "w") if op in ("CONV2D", "CONV_TRANSPOSE2D") else ("d", "h", "w")
        ins_ = tuple(a[x] for x in axes)
        out_ = tuple(a[f"out_{x}"] for x in axes)
        k_ = tuple(a[f"k{x}"] for x in axes)
        s_ = tuple(a[f"stride_{x}"] for x in axes)
        p_ = tuple(a[f"pad_{x}"] for x in axes)
        d_ = tuple(a[f"dilation_{x}"] for x in axes)
    g = a["groups"]
    if kind == "_BACKWARD_BIAS":
        return O.conv_backward_bias(ins[0])
    if op == "CONV_TRANSPOSE2D":
        if kind == "FWD":
            return O.conv_transpose_forward(ins[0], ins[1], ins[2] if len(ins) > 2 else None, s_, p_, d_, g, out_)
        if kind == "_BACKWARD_INPUT":
            return O.conv_transpose_backward_input(ins[0], ins[1], s_, p_, d_, g, ins_)
        return O.conv_transpose_backward_weight(ins[0], ins[1], k_, s_, p_, d_, g)
    if kind == "FWD":
        return O.conv_forward(ins[0], ins[1], ins[2] if len(ins) > 2 else None, s_, p_, d_, g, out_)
    if kind == "_BACKWARD_INPUT":
        return O.conv_backward_input(ins[0], ins[1], s_, p_, d_, g, ins_)
    return O.conv_backward_weight(ins[0], ins[1], k_, s_, p_, d_, g)


def evaluate(root: UOp, bt: BufferTable, *, amp: bool = True) -> np.ndarray:
    if amp:
        root = insert_cast_pass(root)
    vt: Dict[int, np.ndarray] = {}
    for n in toposort(root):
        ins = [vt[id(i)] for i in n.inputs]
        op = n.op
        if op == "BUFFER":
            arr = bt.get(n.arg)
            out = arr.astype(np.float32) if n.dtype == "bfloat16" else arr
        elif op == "LOAD":
            out = ins[0]
        elif op == "CONST":
            out = np.asarray(n.arg["value"], dtype=_np(n.dtype))
            out = _fix(out, n.dtype)
        elif op == "CAST":
            out = _fix(ins[0].astype(_np(n.arg["dtype"] if isinstance(n.arg, dict) else n.dtype)), n.dtype)
        elif op in ("ADD", "MUL", "DIV"):
            a, b = _operands(n, ins)
            r = a + b if op == "ADD" else a * b if op == "MUL" else a / b
            out = _fix(r.astype(r.dtype if op != "DIV" else _np(n.dtype), copy=False), n.dtype)
        elif op == "NEG":
            out = _fix(-ins[0], n.dtype)
        elif op == "EXP":
            out = _fix(np.exp(ins[0]), n.dtype)
        elif op == "LOG":
            out = _fix(np.log(ins[0]), n.dtype)
        elif op == "CMP":
            a, b = _operands(n, ins)
            out = _CMP[n.arg["op"]](a, b)
        elif op == "WHERE":
            out = np.array(np.where(ins[0], ins[1], ins[2]), dtype=_np(n.dtype)).reshape(n.shape)
            out = _fix(out, n.dtype)
        elif op == "MATMUL":
            a, b = ins
            if a.dtype == np.float16 or b.dtype == np.float16 or n.dtype == "bfloat16":
                out = _fix((a.astype(np.float32) @ b.astype(np.float32)).astype(_np(n.dtype)), n.dtype)
            else:
                out = a @ b
        elif op == "REDUCE":
            fn = _RED[n.arg["op"]]
            out = np.asarray(fn(ins[0], axis=n.arg.get("axis"), keepdims=bool(n.arg.get("keepdims"))),
                             dtype=_np(n.dtype))
        elif op == "RESHAPE":
            out = ins[0].reshape(n.arg["new_shape"])
        elif op == "PERMUTE":
            out = np.transpose(ins[0], axes=n.arg["axes"])
        elif op == "SLICE":
            out = ins[0][tuple(slice(s[0], s[1], s[2]) for s in n.arg["slices"])]
        elif op == "BROADCAST_TO":
            out = np.broadcast_to(ins[0], n.shape)
        elif op.startswith("CONV"):
            out = _conv(op, n.arg, ins)
        elif op == "LAYER_NORM":
            x, w, b = ins
            rows, cols = int(n.arg["rows"]), int(n.arg["cols"])
            eps = float(n.arg.get("eps", 1e-5))
            x2 = x.reshape(rows, cols).astype(np.float32, copy=False)
            mean = x2.mean(axis=1, keepdims=True)
            centered = x2 - mean
            var = (centered * centered).mean(axis=1, keepdims=True)
            inv_std = 1.0 / np.sqrt(var + eps)
            x_hat = centered * inv_std
            y = x_hat * w.reshape(1, cols).astype(np.float32) + b.reshape(1, cols).astype(np.float32)
            out = y.reshape(x.shape).astype(_np(n.dtype), copy=False)
        elif op == "FUSED_SOFTMAX":
            x = ins[0]
            ax = n.arg["axis"]
            m = x.max(axis=ax, keepdims=True)
            e = np.exp(x - m)
            out = e / e.sum(axis=ax, keepdims=True)
        elif op == "ATTENTION_FORWARD":
            out = attention_forward_f32(ins[0], ins[1], ins[2], n.arg["scale"])
        elif op == "FUSED_ELEMENTWISE":
            steps = []
            for code, l, r in n.arg["ops"]:
                a = ins[-l - 1] if l < 0 else steps[l]
                if code in ("ADD", "MUL", "DIV"):
                    bb = ins[-r - 1] if r < 0 else steps[r]
                    steps.append(a + bb if code == "ADD" else a * bb if code == "MUL" else a / bb)
                elif code == "NEG":
                    steps.append(-a)
                elif code == "EXP":
                    steps.append(np.exp(a))
                else:
                    steps.append(np.log(a))
            out = steps[-1]
        else:
            raise NotImplementedError(f"oracle graph: {op} has no restatement")
        vt[id(n)] = out
    return np.asarray(vt[id(root)])


__all__ = ["evaluate"]
