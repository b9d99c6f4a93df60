"""safetensors IO for the HIP realizer's graphs.

Offers the reference's entry points
(packages/browsergrad-jit/src/python/_safetensors.py): ``load_safetensors``
(:189-267) returns ``{name: Tensor}`` with the same dtype table, ``dtype=``
cast, ``progress`` callback and the two refusals its tests pin (BF16 ->
NotImplementedError naming PRD-010, HTTP sources -> NotImplementedError
naming PRD-008.2; safetensors.test.ts:127-171); ``save_safetensors``
(:303-385) writes files any safetensors reader loads.

The parser and the writer are written from the format description of the
safetensors project (length prefix, JSON header, tiled data buffer), not
from the reference's code, and check what that description requires: a
header that is a JSON object starting with '{', no duplicate keys, a
string-to-string ``__metadata__``, and tensors that tile the data buffer
with no gap, overlap or trailing bytes.  Malformed input raises
``SafetensorsFormatError`` (a ValueError).

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


# ---------------------------------------------------------------------------- format
#
# The file layout, from the safetensors format description (huggingface/safetensors
# README, "Format"):
#   [0, 8)          u64 little-endian: byte length L of the header
#   [8, 8 + L)      UTF-8 JSON object, starting with '{', optionally right-padded with
#                   spaces; keys are tensor names (no duplicates) plus an optional
#                   "__metadata__" str -> str map; each tensor is
#                   {"dtype": code, "shape": [d0, ...], "data_offsets": [begin, end]}
#   [8 + L, EOF)    the data buffer; offsets are relative to its start, row-major,
#                   little-endian, and the tensors must tile it with no holes.

_LEN_PREFIX = struct.Struct("<Q")
_ALIGN = 8  # the writer pads the header so that the data buffer starts 8-byte aligned


class SafetensorsFormatError(ValueError):
    """A buffer that is not a well-formed safetensors file (a ValueError)."""


def _bad(msg: str) -> SafetensorsFormatError:
    return SafetensorsFormatError(f"safetensors: {msg}")


def _is_count(v: Any) -> bool:
    return isinstance(v, int) and not isinstance(v, bool) and v >= 0


def _reject_duplicate_keys(pairs):
    seen: Dict[str, Any] = {}
    for key, value in pairs:
        if key in seen:
            raise _bad(f"key {key!r} appears twice in the header")
        seen[key] = value
    return seen


def parse_header(buf: Any) -> Tuple[Dict[str, Any], int]:
    """Decode the JSON header of a safetensors buffer.

    Returns the header object and the offset at which the data buffer starts.
    Size checks come before any decoding, so a forged length prefix never
    makes the reader allocate or scan more than the buffer holds or than
    MAX_HEADER_BYTES allows."""
    size = len(buf)
    if size < _LEN_PREFIX.size:
        raise _bad(f"{size}-byte input is too small to hold the 8-byte length prefix")
    (hlen,) = _LEN_PREFIX.unpack(bytes(buf[:_LEN_PREFIX.size]))
    if hlen == 0:
        raise _bad("the length prefix says the header is empty")
    if hlen > MAX_HEADER_BYTES:
        raise _bad(f"a {hlen}-byte header is over the {MAX_HEADER_BYTES}-byte ceiling of this reader")
    data_start = _LEN_PREFIX.size + hlen
    if data_start > size:
        raise _bad(f"the length prefix announces {hlen} header bytes but only "
                   f"{size - _LEN_PREFIX.size} follow it (header runs past the end of the input)")
    raw = bytes(buf[_LEN_PREFIX.size:data_start])
    if raw[:1] != b"{":
        raise _bad("the header does not start with '{' (not a JSON object)")
    try:
        header = json.loads(raw.decode("utf-8"), object_pairs_hook=_reject_duplicate_keys)
    except UnicodeDecodeError as e:
        raise _bad(f"the header is not UTF-8 ({e})") from e
    except json.JSONDecodeError as e:
        raise _bad(f"the header is not a JSON object ({e})") from e
    if not isinstance(header, dict):  # e.g. '{' followed by trailing junk that json still rejects
        raise _bad("the header is not a JSON object")
    return header, data_start


def validate_entry(name: str, meta: Any) -> Tuple[str, Tuple[int, ...], int, int]:
    """Check one tensor record of the header.

    Returns (NumPy dtype name, shape, begin, end); begin and end are offsets
    into the data buffer.  BF16 records raise NotImplementedError, as the
    reference loader does (NumPy has no bfloat16)."""
    where = f"tensor {name!r}"
    if not isinstance(meta, dict):
        raise _bad(f"{where}: the record is not a JSON object")
    unknown = set(meta) - {"dtype", "shape", "data_offsets"}
    if unknown:
        raise _bad(f"{where}: unexpected field(s) {sorted(unknown)}")
    code = meta.get("dtype")
    if code == "BF16":
        raise NotImplementedError(
            f"safetensors: {where} holds BF16 data; NumPy has no bfloat16 type, and the reference "
            f"loader leaves BF16 to its mixed-precision milestone PRD-010. Convert the file to F16 or F32.")
    np_name = DTYPE_MAP.get(code) if isinstance(code, str) else None
    if np_name is None:
        raise _bad(f"{where}: dtype code {code!r} is not one this reader knows ({', '.join(sorted(DTYPE_MAP))})")
    shape = meta.get("shape")
    if not isinstance(shape, list) or not all(_is_count(d) for d in shape):
        raise _bad(f"{where}: shape must be a list of non-negative integers, got {shape!r}")
    span = meta.get("data_offsets")
    if not (isinstance(span, list) and len(span) == 2 and all(_is_count(o) for o in span)):
        raise _bad(f"{where}: data_offsets must be two non-negative integers, got {span!r}")
    begin, end = span
    count = 1
    for d in shape:
        count *= d
    nbytes = count * np.dtype(np_name).itemsize
    if end - begin != nbytes:
        raise _bad(f"{where}: data_offsets {span} cover {end - begin} bytes, "
                   f"but {code} x {shape} needs {nbytes}")
    return np_name, tuple(shape), begin, end


def _layout(buf: Any) -> Tuple[list, int]:
    """Every tensor record of a buffer in header order, as
    (name, dtype name, shape, begin, end), and the data buffer's start.

    Beyond the per-record checks this enforces the format's tiling rule:
    sorted by begin, the records must cover the data buffer exactly, with
    no gap, overlap or trailing bytes."""
    header, data_start = parse_header(buf)
    meta = header.get("__metadata__")
    if meta is not None and not (isinstance(meta, dict) and all(isinstance(v, str) for v in meta.values())):
        raise _bad("__metadata__ must map strings to strings")
    records = [(name,) + validate_entry(name, rec) for name, rec in header.items() if name != "__metadata__"]
    data_len = len(buf) - data_start
    cursor = 0
    for name, _, _, begin, end in sorted(records, key=lambda r: (r[3], r[4])):
        if begin != cursor:
            kind = "overlaps the previous tensor" if begin < cursor else f"leaves a gap at byte {cursor}"
            raise _bad(f"tensor {name!r} starts at byte {begin} and {kind}")
        if end > data_len:
            raise _bad(f"tensor {name!r} ends at byte {end}, past the end of the "
                       f"{data_len}-byte data buffer")
        cursor = end
    if cursor != data_len:
        raise _bad(f"the data buffer holds {data_len} bytes but the tensors cover only {cursor}")
    return records, data_start


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
    """(name, read-only array view into buf, end offset, data length) per
    tensor, in header order."""
    records, data_start = _layout(buf)
    data_len = len(buf) - data_start
    for name, np_name, shape, begin, end in records:
        dt = np.dtype(np_name).newbyteorder("<")
        view = np.frombuffer(buf, dtype=dt, count=(end - begin) // dt.itemsize, offset=data_start + begin)
        yield name, view.reshape(shape), end, data_len


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


def _storable(name: str, value: Any) -> Tuple[str, np.ndarray]:
    """(dtype code, C-contiguous little-endian array) of one value to save."""
    if name == "__metadata__":
        raise _bad("'__metadata__' is reserved for the metadata map and cannot name a tensor")
    if isinstance(value, np.ndarray):
        arr = value
    elif hasattr(value, "numpy"):
        arr = value.numpy()
    else:
        raise TypeError(f"safetensors: cannot store {name!r}: a {type(value).__name__} is neither a "
                        f"Tensor nor a NumPy array")
    code = _NAME_OF.get(arr.dtype.name)
    if code is None:
        raise _bad(f"cannot store {name!r}: dtype {arr.dtype.name} has no safetensors code")
    return code, np.ascontiguousarray(arr, dtype=arr.dtype.newbyteorder("<"))


def save_safetensors(tensors: Dict[str, Any], path: Optional[str] = None, *,
                     metadata: Optional[Dict[str, str]] = None) -> bytes:
    """Serialise ``tensors`` (Tensor or ndarray values) to safetensors bytes,
    also written to ``path`` when given.

    Tensors are laid out in the mapping's order with no padding between
    them; the header is right-padded with spaces so that the data buffer
    starts on an 8-byte boundary (as the format library's own writer does),
    which keeps every mapped tensor aligned for zero-copy views."""
    if metadata is not None and not (isinstance(metadata, dict) and all(
            isinstance(k, str) and isinstance(v, str) for k, v in metadata.items())):
        raise _bad("metadata must be a dict mapping str to str")
    staged = [(name,) + _storable(name, value) for name, value in tensors.items()]
    header: Dict[str, Any] = {} if metadata is None else {"__metadata__": dict(metadata)}
    offset = 0
    for name, code, arr in staged:
        header[name] = {"dtype": code, "shape": list(arr.shape), "data_offsets": [offset, offset + arr.nbytes]}
        offset += arr.nbytes
    text = json.dumps(header, separators=(",", ":")).encode("utf-8")
    text += b" " * (-(_LEN_PREFIX.size + len(text)) % _ALIGN)
    out = bytearray(_LEN_PREFIX.pack(len(text)))
    out += text
    for _, _, arr in staged:
        out += arr.tobytes()
    blob = bytes(out)
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
           "gpt2_block_params", "get_default_session", "DTYPE_MAP", "MAX_HEADER_BYTES", "SafetensorsFormatError"]
