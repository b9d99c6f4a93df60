"""Seed-buffer tables: host arrays by id, and their resident GPU handles.

BufferTable is the host side (the reference's _buffer_table.BufferTable:
new_buffer / new_unmaterialized_buffer / get / is_materialized / update).
It additionally remembers how two kinds of seed buffers were made so the
walker can treat them symbolically instead of uploading them:

  * `new_full(shape, value)`  -- a broadcast scalar (SDPA's scale tensor,
    _functional.py:1518-1522, is np.full of the score shape: 2 GiB at the
    C4 size);
  * `new_causal_mask(lq, lk)` -- np.triu(ones, k=1) (_functional.py:1524-1527).

Their arrays are still produced on demand (get()) for consumers that need
the bytes.

GpuBufferTable mirrors _gpu_buffer_table.py:35-131 method for method:
register (refuses double registration), get, has, detach, replace, release,
release_all, upload (idempotent), stats {handles_alive, uploaded_bytes,
registered_ids}.
"""
from __future__ import annotations

import itertools
from typing import Any, Dict, Optional, Tuple

import numpy as np


class BufferTableError(RuntimeError):
    """The reference's _errors.BufferTableError."""


_IDS = itertools.count(1)


class BufferTable:
    def __init__(self) -> None:
        self._arrays: Dict[str, Optional[np.ndarray]] = {}
        self._meta: Dict[str, Tuple[Tuple[int, ...], str]] = {}
        self._fill: Dict[str, float] = {}
        self._causal: Dict[str, Tuple[int, int]] = {}

    def new_buffer(self, array: np.ndarray, name: Optional[str] = None) -> str:
        bid = f"{name or 'buf'}#{next(_IDS)}"
        arr = np.ascontiguousarray(array)
        self._arrays[bid] = arr
        self._meta[bid] = (tuple(arr.shape), arr.dtype.name)
        return bid

    def new_full(self, shape: Tuple[int, ...], value: float, dtype: str) -> str:
        bid = f"full#{next(_IDS)}"
        self._arrays[bid] = None
        self._meta[bid] = (tuple(shape), dtype)
        self._fill[bid] = float(value)
        return bid

    def new_causal_mask(self, lq: int, lk: int) -> str:
        bid = f"causal_mask#{next(_IDS)}"
        self._arrays[bid] = None
        self._meta[bid] = ((int(lq), int(lk)), "bool")
        self._causal[bid] = (int(lq), int(lk))
        return bid

    def new_unmaterialized_buffer(self, shape: Tuple[int, ...], dtype: str) -> str:
        bid = f"resident#{next(_IDS)}"
        self._arrays[bid] = None
        self._meta[bid] = (tuple(shape), dtype)
        return bid

    def _check(self, bid: str) -> None:
        if bid not in self._meta:
            raise BufferTableError(f"BufferTable: unknown buffer id {bid!r}")

    def get(self, bid: str) -> np.ndarray:
        self._check(bid)
        arr = self._arrays[bid]
        if arr is None:
            shape, dtype = self._meta[bid]
            if bid in self._fill:
                arr = np.full(shape, self._fill[bid], dtype=np.dtype(dtype))
            elif bid in self._causal:
                lq, lk = self._causal[bid]
                arr = np.triu(np.ones((lq, lk), dtype=bool), k=1)
            else:
                raise BufferTableError(f"BufferTable: buffer {bid!r} is resident on the GPU and not materialized")
            self._arrays[bid] = arr
        return arr

    def is_materialized(self, bid: str) -> bool:
        self._check(bid)
        return self._arrays[bid] is not None or bid in self._fill or bid in self._causal

    def update(self, bid: str, array: np.ndarray) -> None:
        self._check(bid)
        self._arrays[bid] = np.ascontiguousarray(array)

    def meta(self, bid: str) -> Tuple[Tuple[int, ...], str]:
        self._check(bid)
        return self._meta[bid]

    def fill_value(self, bid: str) -> Optional[float]:
        return self._fill.get(bid)

    def causal_mask(self, bid: str) -> Optional[Tuple[int, int]]:
        return self._causal.get(bid)


class GpuBufferTable:
    """Per-session registry buffer_id -> bridge handle (the bridge owns memory)."""

    __slots__ = ("_handles", "_bridge", "_total_uploaded_bytes", "_handles_alive")

    def __init__(self, bridge: Any) -> None:
        if bridge is None:
            raise BufferTableError("GpuBufferTable requires a non-None bridge. Register a bridge first.")
        self._handles: Dict[str, Any] = {}
        self._bridge = bridge
        self._total_uploaded_bytes = 0
        self._handles_alive = 0

    @property
    def bridge(self) -> Any:
        return self._bridge

    def register(self, buffer_id: str, handle: Any) -> None:
        if buffer_id in self._handles:
            raise BufferTableError(
                f"GpuBufferTable: buffer_id {buffer_id!r} is already registered with a handle. "
                f"The realizer should consult .get() before re-uploading.")
        self._handles[buffer_id] = handle
        self._handles_alive += 1

    def get(self, buffer_id: str) -> Optional[Any]:
        return self._handles.get(buffer_id)

    def has(self, buffer_id: str) -> bool:
        return buffer_id in self._handles

    def detach(self, buffer_id: str) -> Any:
        if buffer_id not in self._handles:
            raise BufferTableError(f"GpuBufferTable: cannot detach unknown buffer_id {buffer_id!r}")
        self._handles_alive -= 1
        return self._handles.pop(buffer_id)

    def replace(self, buffer_id: str, handle: Any) -> None:
        old = self._handles.pop(buffer_id, None)
        if old is not None:
            self._bridge.release(old)
            self._handles_alive -= 1
        self._handles[buffer_id] = handle
        self._handles_alive += 1

    def release(self, buffer_id: str) -> None:
        handle = self._handles.pop(buffer_id, None)
        if handle is None:
            return
        self._bridge.release(handle)
        self._handles_alive -= 1

    def release_all(self) -> None:
        for buffer_id in list(self._handles):
            self.release(buffer_id)

    def upload(self, buffer_id: str, data: Any, shape: tuple, dtype: str) -> Any:
        existing = self._handles.get(buffer_id)
        if existing is not None:
            return existing
        handle = self._bridge.upload(data, shape, dtype)
        self._handles[buffer_id] = handle
        self._handles_alive += 1
        self._total_uploaded_bytes += len(data) if isinstance(data, (bytes, bytearray)) else int(data.nbytes)
        return handle

    def stats(self) -> Dict[str, int]:
        return {
            "handles_alive": self._handles_alive,
            "uploaded_bytes": self._total_uploaded_bytes,
            "registered_ids": len(self._handles),
        }


__all__ = ["BufferTable", "BufferTableError", "GpuBufferTable"]
