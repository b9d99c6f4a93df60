"""Typed non-causal float32 attention forward: contract and HIP execution.

Mirrors the reference's framework-operation contract for ATTENTION_FORWARD,
packages/browsergrad-jit/src/python/_framework_contracts.py:
  * ceilings                              :89-93
  * AttentionForwardContract              :949-961
  * _attention_forward_shape / product    :2755-2789
  * infer_attention_forward_contract      :2792-2878
  * _validate_attention_forward (node)    :7116-7150
  * execute_attention_forward_arrays      :2881-2932 (runtime checks)
with the same field names, ceilings, error type (ShapeError) and messages,
so a caller sees the same acceptance and refusals (C4's 2^36-element
multiply-add work is refused by the contract, as in the reference).

Execution differs in where it runs: ``execute_attention_forward_hip`` keeps
the reference's runtime validation (exact float32 arrays of the contract's
shapes, finite inputs, finite output) and computes on the GPU through the
bridge's float32 attention kernel.  A non-finite scaled score or softmax
state surfaces there as a non-finite output and raises the reference's
output error; the intermediate checks have no separate device counterpart.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Tuple

import numpy as np

from ..errors import ShapeError

ATTENTION_FORWARD_DIMENSION_MAX = 1 << 20
ATTENTION_FORWARD_DEPTH_MAX = 64
ATTENTION_FORWARD_ELEMENT_MAX = 1 << 28
ATTENTION_FORWARD_WORK_ELEMENT_MAX = 1 << 30
ATTENTION_FORWARD_WORKSPACE_BYTE_MAX = 1 << 28
ATTENTION_FORWARD_CONTRACT_ID = "browsergrad.jit.framework.kernels.attention-forward.v1"


@dataclass(frozen=True)
class AttentionForwardContract:
    query_shape: Tuple[int, int, int, int]
    key_shape: Tuple[int, int, int, int]
    value_shape: Tuple[int, int, int, int]
    output_shape: Tuple[int, int, int, int]
    scale: float
    batch: int
    heads: int
    query_length: int
    key_length: int
    depth: int
    work_elements: int
    workspace_bytes: int


def _shape_of(value: Any, role: str) -> Tuple[int, int, int, int]:
    shape = getattr(value, "shape", None)
    dtype = getattr(value, "dtype", None)
    if isinstance(dtype, np.dtype):
        dtype = dtype.name
    if type(shape) is not tuple or len(shape) != 4:
        raise ShapeError(f"attention_forward: {role} must have exact rank-4 (B,H,S,D) shape, got {shape!r}")
    if dtype != "float32":
        raise ShapeError(f"attention_forward: {role} must have dtype 'float32', got {dtype!r}")
    for axis, extent in enumerate(shape):
        if type(extent) is not int or extent <= 0:
            raise ShapeError(f"attention_forward: {role} shape[{axis}] must be a positive built-in integer")
        if extent > ATTENTION_FORWARD_DIMENSION_MAX:
            raise ShapeError(
                f"attention_forward: {role} shape[{axis}] exceeds the {ATTENTION_FORWARD_DIMENSION_MAX}-element ceiling")
    return shape


def _checked_product(extents: Tuple[int, ...], ceiling: int, role: str) -> int:
    product = 1
    for extent in extents:
        if product > ceiling // extent:
            raise ShapeError(f"attention_forward: {role} exceeds the {ceiling}-element ceiling")
        product *= extent
    return product


def infer_attention_forward_contract(query: Any, key: Any, value: Any) -> AttentionForwardContract:
    """Shape / dtype / ceiling checks of _framework_contracts.py:2792-2878."""
    qs = _shape_of(query, "query")
    ks = _shape_of(key, "key")
    vs = _shape_of(value, "value")
    batch, heads, sq, depth = qs
    if (ks[0], ks[1]) != (batch, heads):
        raise ShapeError("attention_forward: query and key batch/head dimensions must match")
    if (vs[0], vs[1]) != (batch, heads):
        raise ShapeError("attention_forward: query and value batch/head dimensions must match")
    if ks[2] != vs[2]:
        raise ShapeError("attention_forward: key and value sequence lengths must match")
    if ks[3] != depth or vs[3] != depth:
        raise ShapeError("attention_forward: v1 requires identical query/key/value head depth")
    if depth > ATTENTION_FORWARD_DEPTH_MAX:
        raise ShapeError(
            f"attention_forward: head depth {depth} exceeds the proved legacy-WebGPU ceiling "
            f"{ATTENTION_FORWARD_DEPTH_MAX}")
    q_el = _checked_product(qs, ATTENTION_FORWARD_ELEMENT_MAX, "query")
    k_el = _checked_product(ks, ATTENTION_FORWARD_ELEMENT_MAX, "key")
    v_el = _checked_product(vs, ATTENTION_FORWARD_ELEMENT_MAX, "value")
    sk = ks[2]
    scores = _checked_product((batch, heads, sq, sk), ATTENTION_FORWARD_WORK_ELEMENT_MAX, "score matrix")
    if scores > ATTENTION_FORWARD_WORK_ELEMENT_MAX // (2 * depth):
        work = ATTENTION_FORWARD_WORK_ELEMENT_MAX + 1
    else:
        work = scores * 2 * depth
    if work > ATTENTION_FORWARD_WORK_ELEMENT_MAX:
        raise ShapeError(
            f"attention_forward: projected multiply-add work exceeds the {ATTENTION_FORWARD_WORK_ELEMENT_MAX}"
            "-element ceiling")
    workspace = (q_el + k_el + v_el + q_el + scores * 2) * 4
    if workspace > ATTENTION_FORWARD_WORKSPACE_BYTE_MAX:
        raise ShapeError(
            f"attention_forward: projected CPU workspace requires {workspace} bytes, exceeding the "
            f"{ATTENTION_FORWARD_WORKSPACE_BYTE_MAX}-byte ceiling")
    scale = float(np.float32(1.0 / math.sqrt(depth)))
    return AttentionForwardContract(qs, ks, vs, qs, scale, batch, heads, sq, sk, depth, work, workspace)


def validate_attention_forward_node(node: Any) -> AttentionForwardContract:
    """Node-level checks of _validate_attention_forward (:7116-7150)."""
    if getattr(node, "op", None) != "ATTENTION_FORWARD":
        raise ShapeError(f"{ATTENTION_FORWARD_CONTRACT_ID} validator received opcode {getattr(node, 'op', None)!r}")
    inputs = getattr(node, "inputs", None)
    if type(inputs) is not tuple or len(inputs) != 3:
        raise ShapeError("ATTENTION_FORWARD inputs must be exactly (query, key, value)")
    arg = getattr(node, "arg", None)
    if type(arg) is not dict or set(arg) != {"scale", "mask"}:
        raise ShapeError("ATTENTION_FORWARD arg fields must be exactly 'scale' and 'mask'")
    if arg["mask"] != "none":
        raise ShapeError("ATTENTION_FORWARD v1 mask must be exactly 'none'")
    contract = infer_attention_forward_contract(*inputs)
    if type(arg["scale"]) is not float or arg["scale"] != contract.scale:
        raise ShapeError(
            "ATTENTION_FORWARD scale must equal the canonical float32 inverse-square-root head-depth value")
    if getattr(node, "shape", None) != contract.output_shape:
        raise ShapeError("ATTENTION_FORWARD output shape must equal the query shape")
    return contract


def check_attention_forward_arrays(contract: AttentionForwardContract, arrays: Any) -> None:
    """Runtime input checks of execute_attention_forward_arrays (:2881-2905)."""
    if type(arrays) is not tuple or len(arrays) != 3:
        raise ShapeError("attention_forward execution requires exactly three arrays")
    for index, (array, expected) in enumerate(zip(arrays, (contract.query_shape, contract.key_shape,
                                                           contract.value_shape))):
        if type(array) is not np.ndarray or tuple(array.shape) != expected or array.dtype.name != "float32":
            raise ShapeError(
                f"attention_forward runtime input {index} must be an exact float32 ndarray with shape {expected}")
        if not bool(np.isfinite(array).all()):
            raise ShapeError(f"attention_forward runtime input {index} must contain only finite float32 values")


def execute_attention_forward_hip(contract: AttentionForwardContract, arrays: Tuple[np.ndarray, ...],
                                  bridge: Any) -> np.ndarray:
    """softmax(Q K^T * scale) V in float32 on the GPU (the bridge's f32
    attention kernel); inputs uploaded, the output materialised and checked."""
    check_attention_forward_arrays(contract, arrays)
    handles = [bridge.upload(np.ascontiguousarray(a), a.shape, "float32") for a in arrays]
    out = None
    try:
        out = bridge.flash_attention(handles[0], handles[1], handles[2], None, contract.batch, contract.heads,
                                     contract.query_length, contract.key_length, contract.depth, contract.scale,
                                     "float32")
        y = np.array(bridge.to_numpy(out), dtype=np.float32, copy=True).reshape(contract.output_shape)
    finally:
        for h in handles + ([out] if out is not None else []):
            bridge.release(h)
    if not bool(np.isfinite(y).all()):
        raise ShapeError("attention_forward output must remain finite float32")
    return y


__all__ = [
    "ATTENTION_FORWARD_CONTRACT_ID", "ATTENTION_FORWARD_DEPTH_MAX", "ATTENTION_FORWARD_DIMENSION_MAX",
    "ATTENTION_FORWARD_ELEMENT_MAX", "ATTENTION_FORWARD_WORKSPACE_BYTE_MAX", "ATTENTION_FORWARD_WORK_ELEMENT_MAX",
    "AttentionForwardContract", "check_attention_forward_arrays", "execute_attention_forward_hip",
    "infer_attention_forward_contract", "validate_attention_forward_node",
]
