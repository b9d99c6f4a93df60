"""safetensors IO for the HIP realizer's graphs.

Mirrors the reference's reader / writer
(packages/browsergrad-jit/src/python/_safetensors.py): ``load_safetensors``
(:189-267) returns ``{name: Tensor}`` with the same header validation, dtype
table, ``dtype=`` cast, ``progress`` callback and errors (BF16 refused, HTTP
sources refused, header cap 100 MB); ``save_safetensors`` (:303-385) writes
the same byte layout (8-byte little-endian header length, compact JSON
header with ``data_offsets`` in insertion order, then the raw tensors).

Beyond the reference:

* a path source is memory-mapped instead of read whole, so the file is held
  by the page cache rather than copied into a Python ``bytes``;
* ``load_safetensors_resident`` uploads every tensor straight from the
  mapping into device memory (one host-to-device copy per tensor, no host
  copy) and registers the handle in a ``GpuBufferTable`` under the leaf's
  buffer id, so the walker runs on resident weights with no upload of its
  own;
* ``gpt2_block_params`` maps Hugging Face GPT-2 tensor names
  (``h.{i}.ln_1.weight``, ``h.{i}.attn.c_attn.weight`` in Conv1D [in, out]
  layout, ...) onto the parameter dict of ``configs.gpt2_block``.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from typing import Any, Callable, Dict, Optional, Tuple, Union

import numpy as np

from .tensor import Session, Tensor

# The format's dtype names and the NumPy names of this IR (_safetensors.py:52-66).
DTYPE_MAP: Dict[str, str] = {
    "F64": "float64", "F32": "float32", "F16": "float16",
    "I64": "int64", "I32": "int32", "I16": "int16", "I8": "int8",
    "U64": "uint64", "U32": "uint32", "U16": "uint16", "U8": "uint8",
    "BOOL": "bool",
}
_NAME_OF = {v: k for k, v in DTYPE_MAP.items()}

MAX_HEADER_BYTES = 100 * 1024 * 1024  # _safetensors.py:71-73

_DEFAULT_SESSION: Optional[Session] = None


def get_default_session() -> Session:
    """The implicit session tensors land in when no ``session=`` is given."""
    global _DEFAULT_SESSION
    if _DEFAULT_SESSION is None:
        _DEFAULT_SESSION = Session()
    return _DEFAULT_SESSION


# ---------------------------------------------------------------------------- parsing


def parse_header(buf: Any) -> Tuple[Dict[str, Any], int]:
    """(header dict, offset of the data section) of a safetensors buffer
    (_safetensors.py:82-117)."""
    n = len(buf)
    if n < 8:
        raise ValueError(f"safetensors: file is {n} bytes, too small to contain the 8-byte header-length prefix")
    (header_len,) = struct.unpack("<Q", bytes(buf[:8]))
    if header_len == 0:
        raise ValueError("safetensors: header length is zero")
    if header_len > MAX_HEADER_BYTES:
        raise ValueError(f"safetensors: header length {header_len} exceeds the {MAX_HEADER_BYTES}-byte ceiling. "
                         f"Refusing to parse — the file may be corrupted or malicious.")
    if 8 + header_len > n:
        raise ValueError(f"safetensors: header length {header_len} exceeds file size {n}")
    try:
        header = json.loads(bytes(buf[8:8 + header_len]).decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise ValueError(f"safetensors: header is not valid UTF-8 JSON: {e}") from e
    if not isinstance(header, dict):
        raise ValueError(f"safetensors: header is a {type(header).__name__}, expected dict")
    return header, 8 + header_len


def validate_entry(name: str, meta: Any) -> Tuple[str, Tuple[int, ...], int, int]:
    """(numpy dtype name, shape, start, end) of one header entry, checked
    against the format (_safetensors.py:120-186)."""
    if not isinstance(meta, dict):
        raise ValueError(f"safetensors: tensor {name!r} metadata is a {type(meta).__name__}, expected dict")
    code = meta.get("dtype")
    if not isinstance(code, str):
        raise ValueError(f"safetensors: tensor {name!r} missing string dtype (got {code!r})")
    if code == "BF16":
        # The reference defers BF16 to its mixed-precision milestone (PRD-010).
        raise NotImplementedError(
            f"safetensors: tensor {name!r} is BF16, which NumPy doesn't natively support (the reference "
            f"defers it to PRD-010). Re-export the file as F16 or F32.")
    if code not in DTYPE_MAP:
        raise ValueError(f"safetensors: tensor {name!r} has unknown dtype {code!r}; "
                         f"expected one of {sorted(DTYPE_MAP) + ['BF16']}")
    np_name = DTYPE_MAP[code]
    shape = meta.get("shape")
    if not isinstance(shape, list) or not all(isinstance(d, int) and not isinstance(d, bool) and d >= 0
                                              for d in shape):
        raise ValueError(f"safetensors: tensor {name!r} has invalid shape {shape!r}; "
                         f"expected list of non-negative ints")
    offsets = meta.get("data_offsets")
    if (not isinstance(offsets, list) or len(offsets) != 2
            or not all(isinstance(o, int) and not isinstance(o, bool) and o >= 0 for o in offsets)
            or offsets[0] > offsets[1]):
        raise ValueError(f"safetensors: tensor {name!r} has invalid data_offsets {offsets!r}; "
                         f"expected [start, end] with 0 <= start <= end")
    want = np.dtype(np_name).itemsize * int(np.prod(shape, dtype=np.int64))
    if offsets[1] - offsets[0] != want:
        raise ValueError(f"safetensors: tensor {name!r} byte range {offsets[1] - offsets[0]} doesn't match "
                         f"shape×dtype {want}")
    return np_name, tuple(shape), offsets[0], offsets[1]


def _resolve_source(source: Union[str, bytes, bytearray, memoryview]) -> Tuple[Any, str]:
    """A read-only buffer over the source and a label for errors
    (_safetensors.py:270-300; a path is memory-mapped)."""
    if isinstance(source, (bytes, bytearray)):
        return memoryview(source), "<bytes>"
    if isinstance(source, memoryview):
        return source, "<memoryview>"
    if isinstance(source, (str, os.PathLike)):
        path = os.fspath(source)
        if path.startswith("file://"):
            path = path[len("file://"):]
        if path.startswith(("http://", "https://")):
            raise NotImplementedError(
                f"safetensors: HTTP URL sources need the reference's runtime bridge (PRD-008.2); download to a "
                f"local file and pass the path. (got: {source!r})")
        if not os.path.exists(path):
            raise FileNotFoundError(f"safetensors: no such file: {path!r}")
        if os.path.getsize(path) == 0:
            return memoryview(b""), path
        with open(path, "rb") as f:
            return mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ), path
    raise TypeError(f"safetensors: source must be bytes / memoryview / file path, got {type(source).__name__}")


def _entries(buf: Any):
    header, data_start = parse_header(buf)
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        np_name, shape, start, end = validate_entry(name, meta)
        a, b = data_start + start, data_start + end
        if b > len(buf):
            raise ValueError(f"safetensors: tensor {name!r} extends past end of file ({b} > {len(buf)})")
        view = np.frombuffer(buf, dtype=np.dtype(np_name), count=(b - a) // np.dtype(np_name).itemsize, offset=a)
        yield name, view.reshape(shape), end, len(buf) - data_start


# ---------------------------------------------------------------------------- loading


def load_safetensors(source: Union[str, bytes, bytearray, memoryview], *, session: Optional[Session] = None,
                     progress: Optional[Callable[[str, int, int], None]] = None,
                     dtype: Optional[str] = None) -> Dict[str, Tensor]:
    """{name: Tensor} from a safetensors file or buffer (_safetensors.py:189-267).

    Every tensor is copied out of the source into the session's host
    BufferTable (the source may be released afterwards); ``dtype`` casts
    each tensor whose dtype differs; ``progress(name, bytes_loaded,
    bytes_total)`` fires once per tensor."""
    buf, _ = _resolve_source(source)
    session = session if session is not None else get_default_session()
    out: Dict[str, Tensor] = {}
    for name, view, end, total in _entries(buf):
        t = session.from_numpy(view.copy(), name)
        if dtype is not None and t.dtype != dtype:
            t = t.cast(dtype)
        out[name] = t
        if progress is not None:
            progress(name, end, total)
    return out


def load_safetensors_resident(source: Union[str, bytes, bytearray, memoryview], gpu_table: Any, *,
                              session: Optional[Session] = None,
                              progress: Optional[Callable[[str, int, int], None]] = None) -> Dict[str, Tensor]:
    """{name: Tensor} whose leaves are already resident on the device
    (extension).  Each tensor is uploaded from the source mapping into a
    device handle registered in ``gpu_table`` (a GpuBufferTable) under the
    leaf's buffer id; the host BufferTable keeps a read-only view of the
    mapping, not a copy, so a mapped file must stay unchanged while the
    session is in use."""
    buf, _ = _resolve_source(source)
    session = session if session is not None else get_default_session()
    bridge = gpu_table.bridge
    out: Dict[str, Tensor] = {}
    for name, view, end, total in _entries(buf):
        t = session.from_numpy(view, name)
        bid = t.uop.inputs[0].arg  # LOAD(BUFFER(bid))
        gpu_table.register(bid, bridge.upload(view, view.shape, view.dtype.name))
        out[name] = t
        if progress is not None:
            progress(name, end, total)
    return out


# ---------------------------------------------------------------------------- saving


def save_safetensors(tensors: Dict[str, Any], path: Optional[str] = None, *,
                     metadata: Optional[Dict[str, str]] = None) -> bytes:
    """The safetensors bytes of ``tensors`` (Tensor or ndarray values), also
    written to ``path`` when given (_safetensors.py:303-385)."""
    header: Dict[str, Any] = {}
    arrays = []
    cursor = 0
    for name, value in tensors.items():
        if isinstance(value, np.ndarray):
            arr = value
        elif hasattr(value, "numpy"):
            arr = value.numpy()
        else:
            raise TypeError(f"safetensors: value at {name!r} is a {type(value).__name__}, "
                            f"expected TensorProxy or np.ndarray")
        arr = np.ascontiguousarray(arr)
        code = _NAME_OF.get(arr.dtype.name)
        if code is None:
            raise ValueError(f"safetensors: cannot save dtype {arr.dtype.name!r} (no safetensors equivalent)")
        header[name] = {"dtype": code, "shape": list(arr.shape), "data_offsets": [cursor, cursor + arr.nbytes]}
        cursor += arr.nbytes
        arrays.append(arr)
    if metadata is not None:
        if not isinstance(metadata, dict) or not all(isinstance(k, str) and isinstance(v, str)
                                                     for k, v in metadata.items()):
            raise ValueError("safetensors: __metadata__ must be Dict[str, str]")
        header["__metadata__"] = metadata
    head = json.dumps(header, separators=(",", ":")).encode("utf-8")
    blob = b"".join([struct.pack("<Q", len(head)), head] + [a.tobytes() for a in arrays])
    if path is not None:
        with open(path, "wb") as f:
            f.write(blob)
    return blob


# ---------------------------------------------------------------------------- GPT-2 weights


def gpt2_block_params(tensors: Dict[str, Tensor], layer: int, prefix: str = "") -> Dict[str, Tensor]:
    """The parameter dict of ``configs.gpt2_block`` from Hugging Face GPT-2
    names (``{prefix}h.{layer}.ln_1.weight`` ...).  GPT-2 stores its
    projections as Conv1D weights [in, out]; the block's ``linear`` takes
    [out, in], so those are transposed (a PERMUTE the walker folds into the
    GEMM's operand layout)."""
    p = f"{prefix}h.{layer}."

    def get(name: str) -> Tensor:
        key = p + name
        if key not in tensors:
            raise KeyError(f"gpt2_block_params: missing tensor {key!r}")
        return tensors[key]

    def conv1d_weight(name: str) -> Tensor:
        return get(name).permute(1, 0)

    return {
        "ln1_w": get("ln_1.weight"), "ln1_b": get("ln_1.bias"),
        "w_qkv": conv1d_weight("attn.c_attn.weight"), "b_qkv": get("attn.c_attn.bias"),
        "w_o": conv1d_weight("attn.c_proj.weight"), "b_o": get("attn.c_proj.bias"),
        "ln2_w": get("ln_2.weight"), "ln2_b": get("ln_2.bias"),
        "w_up": conv1d_weight("mlp.c_fc.weight"), "b_up": get("mlp.c_fc.bias"),
        "w_down": conv1d_weight("mlp.c_proj.weight"), "b_down": get("mlp.c_proj.bias"),
    }


__all__ = ["load_safetensors", "load_safetensors_resident", "save_safetensors", "parse_header", "validate_entry",
           "gpt2_block_params", "get_default_session", "DTYPE_MAP", "MAX_HEADER_BYTES"]
