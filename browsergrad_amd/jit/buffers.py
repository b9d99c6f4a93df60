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

GpuBufferTable keeps the interface of _gpu_buffer_table.py:35-131 (method
names, idempotent upload, stats keys) over its own bookkeeping.
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
    """Device residency of one session's seed buffers.

    Maps a buffer id to the bridge handle that holds its bytes on the GPU.
    The bridge owns the memory; the table decides when a handle is minted
    (the first ``upload`` of an id; later ones return the same handle) and
    when it is given back (``release`` / ``replace`` / ``release_all``).
    ``handles_alive`` and ``registered_ids`` are both the number of ids that
    currently hold a handle; ``uploaded_bytes`` counts host bytes sent over
    the table's life.  Interface of the reference's table
    (``_gpu_buffer_table.py:35-131``): the method names, an idempotent
    upload, a refused second ``register`` of one id, and the stats keys the
    residency tests read.
    """

    __slots__ = ("_bridge", "_resident", "_sent")

    def __init__(self, bridge: Any) -> None:
        if bridge is None:
            raise BufferTableError("a GpuBufferTable needs a bridge to hold its device handles, got None")
        self._bridge = bridge
        self._resident: Dict[str, Any] = {}
        self._sent = 0

    @property
    def bridge(self) -> Any:
        return self._bridge

    def _drop(self, buffer_id: str, give_back: bool) -> Any:
        handle = self._resident.pop(buffer_id)
        if give_back:
            self._bridge.release(handle)
        return handle

    def register(self, buffer_id: str, handle: Any) -> None:
        """Record a handle minted elsewhere (a resident plan result)."""
        held = self._resident.get(buffer_id)
        if held is not None:
            raise BufferTableError(
                f"buffer {buffer_id!r} is resident already (handle {held!r}); "
                "look it up with get() rather than registering a second handle")
        self._resident[buffer_id] = handle

    def get(self, buffer_id: str) -> Optional[Any]:
        return self._resident.get(buffer_id)

    def has(self, buffer_id: str) -> bool:
        return buffer_id in self._resident

    def ids(self) -> list:
        """The buffer ids that currently hold a handle."""
        return list(self._resident)

    def detach(self, buffer_id: str) -> Any:
        """Forget an id without releasing its handle; the caller owns it now."""
        if buffer_id not in self._resident:
            raise BufferTableError(f"buffer {buffer_id!r} holds no device handle, so there is nothing to detach")
        return self._drop(buffer_id, give_back=False)

    def replace(self, buffer_id: str, handle: Any) -> None:
        if buffer_id in self._resident:
            self._drop(buffer_id, give_back=True)
        self._resident[buffer_id] = handle

    def release(self, buffer_id: str) -> None:
        """Give an id's handle back to the bridge; unknown ids are ignored."""
        if buffer_id in self._resident:
            self._drop(buffer_id, give_back=True)

    def release_all(self) -> None:
        while self._resident:
            self._drop(next(iter(self._resident)), give_back=True)

    def upload(self, buffer_id: str, data: Any, shape: tuple, dtype: str) -> Any:
        """The id's handle, uploading ``data`` only the first time."""
        held = self._resident.get(buffer_id)
        if held is None:
            held = self._resident[buffer_id] = self._bridge.upload(data, shape, dtype)
            self._sent += len(data) if isinstance(data, (bytes, bytearray)) else int(data.nbytes)
        return held

    def stats(self) -> Dict[str, int]:
        n = len(self._resident)
        return {"handles_alive": n, "uploaded_bytes": self._sent, "registered_ids": n}


__all__ = ["BufferTable", "BufferTableError", "GpuBufferTable"]
