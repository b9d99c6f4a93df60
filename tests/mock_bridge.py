"""A NumPy stand-in for HipRealizerBridge (test infrastructure, CPU only).

The reference tests its walker against a MockBridge that implements the
bridge protocol with array arithmetic
(packages/browsergrad-jit/tests-integration/webgpu_realizer.test.ts:24-1007).
This is the same idea for the HIP walker: every method the walker, the
residency logic and the GpuBufferTable call exists here with the C ABI's
handle semantics, so those parts of the front end run in the build
container with no GPU:

* handles are integers minted from 1 and never reused; an unknown or
  released handle raises KernelError naming the op (realizer.ts:995);
  release is idempotent (realizer.ts:1036-1041);
* a handle is flat storage plus a shape, like a device allocation:
  reshape shares the storage, copy_strided / attention views / GEMM
  leading dimensions index it with element strides exactly as the kernels
  do;
* arithmetic comes from oracle/ (the NumPy restatement of the reference
  CPU realizer), so results match the graph oracle within the parity
  tolerances; bfloat16 is held as its uint16 bit pattern.

Only the tests import this module.
"""
from __future__ import annotations

from typing import Any, Dict, Optional, Sequence, Tuple

import numpy as np
from numpy.lib.stride_tricks import as_strided

from browsergrad_amd import _native as N
from browsergrad_amd.errors import JitNotImplementedError, KernelError
from oracle import ops as O

_STORE = {"float32": np.float32, "float16": np.float16, "bfloat16": np.uint16, "bool": np.bool_,
          "uint8": np.uint8, "int32": np.int32, "int64": np.int64, "float64": np.float64}


def _to_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return O.bf16_bits_to_f32(a)
    return np.asarray(a).astype(np.float32)


def _from_f32(a: np.ndarray, dtype: str) -> np.ndarray:
    a = np.asarray(a, dtype=np.float32)
    if dtype == "bfloat16":
        return O.f32_to_bf16_bits(a)
    if dtype == "bool":
        return a != 0
    return a.astype(_STORE[dtype])


class _Rec:
    __slots__ = ("flat", "shape", "dtype")

    def __init__(self, flat: np.ndarray, shape: Tuple[int, ...], dtype: str) -> None:
        self.flat, self.shape, self.dtype = flat, tuple(int(d) for d in shape), dtype


class MockHipBridge:
    """Same method names and handle rules as browsergrad_amd.bridge.HipRealizerBridge."""

    def __init__(self, device: int = 0, profiling: bool = False) -> None:
        self.device = device
        self.profiling = profiling
        self.counters = {"upload": 0, "materialize": 0, "release": 0, "matmul": 0}
        self._next = 1
        self._h: Dict[int, _Rec] = {}
        self._allocated = 0
        self._released = 0

    # -- lifecycle -----------------------------------------------------------------
    def close(self) -> None:
        pass

    def __enter__(self) -> "MockHipBridge":
        return self

    def __exit__(self, *exc: Any) -> None:
        self.close()

    def synchronize(self) -> None:
        pass

    def set_profiling(self, on: bool) -> None:
        self.profiling = bool(on)

    def _mint(self, flat: np.ndarray, shape: Sequence[int], dtype: str) -> int:
        h = self._next
        self._next += 1
        self._h[h] = _Rec(np.ascontiguousarray(flat).reshape(-1), tuple(shape), dtype)
        self._allocated += self._h[h].flat.nbytes
        return h

    def _get(self, h: Any, what: str) -> _Rec:
        rec = self._h.get(int(h)) if h is not None else None
        if rec is None:
            raise KernelError(f"{what}: unknown or released handle {h}", N.BG_E_HANDLE)
        return rec

    def _arr(self, h: Any, what: str) -> np.ndarray:
        r = self._get(h, what)
        return r.flat.reshape(r.shape) if r.shape else r.flat.reshape(())

    # -- buffer lifecycle ------------------------------------------------------------
    def upload(self, data: Any, shape: Sequence[int], dtype: str) -> int:
        if dtype not in _STORE:
            raise KernelError(f"upload: dtype {dtype} not supported", N.BG_E_DTYPE)
        st = _STORE[dtype]
        if isinstance(data, np.ndarray):
            flat = np.ascontiguousarray(data).reshape(-1).view(st) if data.dtype != st else data.reshape(-1).copy()
        else:
            flat = np.frombuffer(bytes(data), dtype=st).copy()
        if flat.size != int(np.prod(shape, dtype=np.int64)):
            raise KernelError("upload: data length does not match shape", N.BG_E_SHAPE)
        self.counters["upload"] += 1
        return self._mint(flat, shape, dtype)

    def materialize(self, handle: int, shape: Sequence[int], dtype: str) -> bytes:
        r = self._get(handle, "materialize")
        self.counters["materialize"] += 1
        return r.flat.tobytes()

    def to_numpy(self, handle: int) -> np.ndarray:
        self.counters["materialize"] += 1
        return self._arr(handle, "materialize").copy()

    def release(self, handle: Any) -> None:
        if handle is None:
            return
        r = self._h.pop(int(handle), None)
        if r is not None:
            self._released += r.flat.nbytes
        self.counters["release"] += 1

    def handle_info(self, handle: int) -> dict:
        r = self._get(handle, "handle_info")
        return {"shape": r.shape, "dtype": r.dtype, "nbytes": int(r.flat.nbytes)}

    def reshape(self, handle: int, shape: Sequence[int]) -> int:
        r = self._get(handle, "reshape")
        if int(np.prod(shape, dtype=np.int64)) != r.flat.size:
            raise KernelError("reshape: element count differs", N.BG_E_SHAPE)
        h = self._next
        self._next += 1
        self._h[h] = _Rec(r.flat, tuple(shape), r.dtype)  # shares storage, as a device view does
        return h

    def copy_strided(self, src: int, offset: int, shape: Sequence[int], strides: Sequence[int]) -> int:
        r = self._get(src, "copy_strided")
        it = r.flat.itemsize
        base = r.flat[int(offset):]
        v = as_strided(base, shape=tuple(shape), strides=tuple(int(s) * it for s in strides))
        return self._mint(v.copy(), shape, r.dtype)

    # -- compute ------------------------------------------------------------------------
    def matmul(self, a: int, b: int, m: int, k: int, n: int, dtype: str) -> int:
        self.counters["matmul"] += 1
        x = self._arr(a, "matmul[A]").reshape(m, k)
        y = self._arr(b, "matmul[B]").reshape(k, n)
        return self._mint(O.matmul(x, y), (m, n), dtype)

    def matmul_ex(self, a: int, b: int, *, m: int, n: int, k: int, batch: int = 1, lda: Optional[int] = None,
                  ldb: Optional[int] = None, ldc: Optional[int] = None, stride_a: Optional[int] = None,
                  stride_b: Optional[int] = None, stride_c: Optional[int] = None, offset_a: int = 0,
                  offset_b: int = 0, trans_b: bool = False, in_dtype: str = "float32",
                  out_dtype: Optional[str] = None, bias: Optional[int] = None, round_out: bool = False,
                  act: int = N.ACT_NONE, residual: Optional[int] = None, a_dtype: Optional[str] = None,
                  b_dtype: Optional[str] = None) -> int:
        out_dtype = out_dtype or in_dtype
        lda = k if lda is None else lda
        ldb = (k if trans_b else n) if ldb is None else ldb
        ldc = n if ldc is None else ldc
        stride_a = m * lda if stride_a is None else stride_a
        stride_b = (n if trans_b else k) * ldb if stride_b is None else stride_b
        stride_c = m * ldc if stride_c is None else stride_c
        ra, rb = self._get(a, "matmul[A]"), self._get(b, "matmul[B]")
        if ra.dtype != (a_dtype or in_dtype) or rb.dtype != (b_dtype or in_dtype):
            raise KernelError(f"matmul: operands must be {in_dtype}", N.BG_E_DTYPE)

        def view(rec, off, sb, rows, ld, cols):
            it = rec.flat.itemsize
            v = as_strided(rec.flat[off:], shape=(batch, rows, cols), strides=(sb * it, ld * it, it))
            x = _to_f32(v, rec.dtype)
            if rec.dtype != in_dtype:  # operand cast in the pre-pass (round to nearest even)
                x = _to_f32(_from_f32(x, in_dtype), in_dtype)
            return x

        A = view(ra, offset_a, stride_a, m, lda, k)
        B = view(rb, offset_b, stride_b, n if trans_b else k, ldb, k if trans_b else n)
        if trans_b:
            B = np.swapaxes(B, 1, 2)
        acc = np.matmul(A, B).astype(np.float32)
        if round_out and in_dtype in ("float16", "bfloat16"):
            acc = _to_f32(_from_f32(acc, in_dtype), in_dtype)
        if bias:
            acc = (acc + self._arr(bias, "matmul[bias]").reshape(-1)).astype(np.float32)
        if act == N.ACT_RELU:
            acc = np.where(acc > 0, acc, np.float32(0)).astype(np.float32)
        elif act == N.ACT_GELU_TANH:
            acc = O.gelu_tanh_f32(acc)
        if residual:
            acc = (acc + self._arr(residual, "matmul[residual]").reshape(batch, m, n)).astype(np.float32)
        out_elems = (batch - 1) * stride_c + (m - 1) * ldc + n
        st = _STORE[out_dtype]
        flat = np.zeros(out_elems, dtype=st)
        it = flat.itemsize
        as_strided(flat, shape=(batch, m, n), strides=(stride_c * it, ldc * it, it))[...] = _from_f32(acc, out_dtype)
        return self._mint(flat, (batch, m, n) if batch > 1 else (m, n), out_dtype)

    def fused_elementwise(self, inputs: list, ops: list, shape: Sequence[int], dtype: str) -> int:
        xs = [_to_f32(self._arr(h, "fused_elementwise"), self._get(h, "fused_elementwise").dtype).reshape(shape)
              for h in inputs]
        y = O.fused_program(xs, [tuple(o) + (0,) * (4 - len(o)) for o in ops])
        return self._mint(_from_f32(np.broadcast_to(y, shape), dtype), shape, dtype)

    def fused_ex(self, inputs: Sequence[int], ops: Sequence[Tuple[str, int, int, int]], shape: Sequence[int],
                 out_dtype: str, *, in_strides: Optional[Sequence[Sequence[int]]] = None,
                 imms: Sequence[float] = (), reduce: int = N.RED_NONE, keepdims: bool = False) -> int:
        shape = tuple(int(d) for d in shape)
        xs = []
        for i, h in enumerate(inputs):
            r = self._get(h, "fused_elementwise[input]")
            if in_strides is None:
                v = r.flat.reshape(shape)
            else:
                it = r.flat.itemsize
                v = as_strided(r.flat, shape=shape, strides=tuple(int(s) * it for s in in_strides[i]))
            xs.append(_to_f32(v, r.dtype))
        y = np.broadcast_to(O.fused_program(xs, [tuple(o) for o in ops], [np.float32(v) for v in imms]), shape)
        y = y.astype(np.float32)
        if reduce != N.RED_NONE:
            fn = {N.RED_SUM: np.sum, N.RED_MAX: np.max, N.RED_MEAN: np.mean, N.RED_MIN: np.min}[reduce]
            y = fn(y, axis=-1, keepdims=keepdims).astype(np.float32)
        return self._mint(_from_f32(y, out_dtype), y.shape, out_dtype)

    def cast(self, handle: int, src_dtype: str, dst_dtype: str, shape: Sequence[int]) -> int:
        r = self._get(handle, "cast")
        if r.dtype != src_dtype:
            raise KernelError("cast: source dtype differs from the handle", N.BG_E_DTYPE)
        if dst_dtype == "float16" and src_dtype == "float32":
            flat = O.f32_to_f16(r.flat)
        else:
            flat = _from_f32(_to_f32(r.flat, src_dtype), dst_dtype)
        return self._mint(flat, shape, dst_dtype)

    def reduce_last(self, x: int, rows: int, cols: int, op: int, keepdims: bool = False) -> int:
        r = self._get(x, "reduce")
        a = _to_f32(r.flat, r.dtype).reshape(rows, cols)
        fn = {N.RED_SUM: np.sum, N.RED_MAX: np.max, N.RED_MEAN: np.mean, N.RED_MIN: np.min}[op]
        y = fn(a, axis=1).astype(np.float32)
        return self._mint(_from_f32(y, r.dtype), (rows, 1) if keepdims else (rows,), r.dtype)

    def softmax_last(self, x: int, rows: int, cols: int, out_dtype: str = "float32") -> int:
        r = self._get(x, "softmax")
        y = O.softmax_lastaxis(_to_f32(r.flat, r.dtype).reshape(rows, cols))
        return self._mint(_from_f32(y, out_dtype), r.shape, out_dtype)

    def layer_norm(self, x: int, weight: int, bias: int, rows: int, cols: int, eps: float,
                   out_dtype: str = "float32") -> int:
        r = self._get(x, "layer_norm[x]")
        y = O.layer_norm(_to_f32(r.flat, r.dtype).reshape(rows, cols), self._arr(weight, "layer_norm[weight]"),
                         self._arr(bias, "layer_norm[bias]"), eps)
        return self._mint(_from_f32(y, out_dtype), r.shape, out_dtype)

    def attention_ex(self, q: int, k: int, v: int, *, batch: int, heads: int, sq: int, sk: int, d: int,
                     scale: float, causal: bool = False, in_dtype: str = "float16",
                     out_dtype: Optional[str] = None, round_scores: bool = False,
                     q_view: Tuple[int, int, int, int] = (0, 0, 0, 0),
                     k_view: Tuple[int, int, int, int] = (0, 0, 0, 0),
                     v_view: Tuple[int, int, int, int] = (0, 0, 0, 0),
                     o_strides: Tuple[int, int, int] = (0, 0, 0)) -> int:
        out_dtype = out_dtype or in_dtype

        def view(h, vw, s, what):
            r = self._get(h, what)
            off, sb, sh, ss = vw
            if (sb, sh, ss) == (0, 0, 0):
                sb, sh, ss = heads * s * d, s * d, d
            it = r.flat.itemsize
            return as_strided(r.flat[off:], shape=(batch, heads, s, d), strides=(sb * it, sh * it, ss * it, it))

        qa, ka, va = view(q, q_view, sq, "attention[q]"), view(k, k_view, sk, "attention[k]"), view(v, v_view, sk,
                                                                                                    "attention[v]")
        if in_dtype == "float16":
            o = O.sdpa_amp(np.ascontiguousarray(qa), np.ascontiguousarray(ka), np.ascontiguousarray(va), scale,
                           causal).astype(np.float32)
        elif in_dtype == "bfloat16":
            o = O.bf16_bits_to_f32(O.sdpa_bf16(np.ascontiguousarray(qa), np.ascontiguousarray(ka),
                                               np.ascontiguousarray(va), scale, causal))
        else:
            mask = np.triu(np.ones((sq, sk), dtype=bool), k=1) if causal else None
            o = O.attention_f64(qa, ka, va, scale, causal=mask is not None).astype(np.float32)
        sb, sh, ss = o_strides
        if (sb, sh, ss) == (0, 0, 0):
            sb, sh, ss = heads * sq * d, sq * d, d
        out_elems = (batch - 1) * sb + (heads - 1) * sh + (sq - 1) * ss + d
        flat = np.zeros(out_elems, dtype=_STORE[out_dtype])
        it = flat.itemsize
        as_strided(flat, shape=(batch, heads, sq, d), strides=(sb * it, sh * it, ss * it, it))[...] = \
            _from_f32(o, out_dtype)
        return self._mint(flat, (batch, heads, sq, d), out_dtype)

    def flash_attention(self, q: int, k: int, v: int, mask: Optional[int], b: int, h: int, sq: int, sk: int,
                        d: int, scale: float, dtype: str) -> int:
        if mask:
            raise JitNotImplementedError("mock flash_attention: additive masks are not modelled")
        qa, ka, va = (self._arr(x, "flash_attention").reshape(b, h, -1, d) for x in (q, k, v))
        o = O.attention_forward_f32(qa, ka, va, scale)
        return self._mint(_from_f32(o, dtype), (b, h, sq, d), dtype)

    def conv_ex(self, *a: Any, **k: Any) -> int:
        raise JitNotImplementedError("mock bridge: convolutions are exercised on the GPU only")

    # -- observability ------------------------------------------------------------------
    def aliveHandleCount(self) -> int:  # noqa: N802 - reference name
        return len(self._h)

    alive_handle_count = aliveHandleCount

    def resourceSnapshot(self) -> dict:  # noqa: N802 - reference name
        owned = sum(r.flat.nbytes for r in self._h.values())
        return {"timingMode": "unavailable", "timestampQueryAvailable": False, "currentOwnedGpuBytes": owned,
                "totalAllocatedGpuBytes": self._allocated, "totalReleasedGpuBytes": self._released,
                "aliveHandleCount": len(self._h), "pendingProfileCount": 0}

    def flushProfiles(self) -> dict:  # noqa: N802 - reference name
        snap = self.resourceSnapshot()
        snap["passProfiles"] = []
        return snap


__all__ = ["MockHipBridge"]
