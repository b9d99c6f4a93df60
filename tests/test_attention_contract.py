"""Typed ATTENTION_FORWARD contract on the CPU.

Acceptance / refusal cases follow
packages/browsergrad-jit/src/python/_framework_contracts.py:2755-2932 and the
public surface index.ts:212-265; C4's shape is refused by the work ceiling
(_framework_contracts.py:89-93).  The float32 restatement is pinned against the
float64 definition and the Q = 0 -> mean(V) identity.
"""
from __future__ import annotations

import numpy as np
import pytest

from browsergrad_amd.errors import JitNotImplementedError, ShapeError
from browsergrad_amd.jit.attention_forward import (
    ATTENTION_FORWARD_WORK_ELEMENT_MAX, check_attention_forward_arrays, infer_attention_forward_contract,
    validate_attention_forward_node,
)
from browsergrad_amd.jit.ir import UOp
from browsergrad_amd.jit.tensor import Session, attention_forward, flash_attention
from oracle import graph as G
from oracle import ops as O


class _T:
    def __init__(self, shape, dtype="float32"):
        self.shape, self.dtype = shape, dtype


def test_contract_fields():
    c = infer_attention_forward_contract(_T((2, 3, 5, 8)), _T((2, 3, 7, 8)), _T((2, 3, 7, 8)))
    assert c.output_shape == (2, 3, 5, 8) and c.key_length == 7 and c.depth == 8
    assert c.scale == float(np.float32(1 / np.sqrt(8)))
    assert c.work_elements == 2 * 3 * 5 * 7 * 2 * 8
    assert c.workspace_bytes == (2 * 3 * 5 * 8 * 2 + 2 * 3 * 7 * 8 * 2 + 2 * 3 * 5 * 7 * 2) * 4


@pytest.mark.parametrize("q,k,v,msg", [
    ((2, 3, 5), (2, 3, 5, 8), (2, 3, 5, 8), "exact rank-4"),
    ((2, 3, 5, 8), (2, 4, 5, 8), (2, 4, 5, 8), "query and key batch/head"),
    ((2, 3, 5, 8), (2, 3, 5, 8), (1, 3, 5, 8), "query and value batch/head"),
    ((2, 3, 5, 8), (2, 3, 5, 8), (2, 3, 6, 8), "key and value sequence lengths"),
    ((2, 3, 5, 8), (2, 3, 5, 4), (2, 3, 5, 4), "identical query/key/value head depth"),
    ((1, 1, 4, 128), (1, 1, 4, 128), (1, 1, 4, 128), "head depth 128 exceeds"),
    ((1, 1, (1 << 20) + 1, 8), (1, 1, 4, 8), (1, 1, 4, 8), r"shape\[2\] exceeds"),
    ((8, 16, 2048, 64), (8, 16, 2048, 64), (8, 16, 2048, 64), "multiply-add work exceeds"),
])
def test_contract_refusals(q, k, v, msg):
    with pytest.raises(ShapeError, match=msg):
        infer_attention_forward_contract(_T(q), _T(k), _T(v))


def test_contract_dtype_and_extent_types():
    with pytest.raises(ShapeError, match="dtype 'float32'"):
        infer_attention_forward_contract(_T((1, 1, 4, 8), "float16"), _T((1, 1, 4, 8)), _T((1, 1, 4, 8)))
    with pytest.raises(ShapeError, match="positive built-in integer"):
        infer_attention_forward_contract(_T((1, 1, 0, 8)), _T((1, 1, 4, 8)), _T((1, 1, 4, 8)))


def test_c4_work_is_over_the_ceiling():
    # B8 H16 S2048 D64 -> 2^36 multiply-add elements > 2^30 (_framework_contracts.py:89-93).
    assert 8 * 16 * 2048 * 2048 * 2 * 64 == 1 << 36 > ATTENTION_FORWARD_WORK_ELEMENT_MAX


def test_node_validation_and_builders(rng):
    s = Session()
    q = s.from_numpy(rng.standard_normal((1, 2, 4, 8), dtype=np.float32))
    y = attention_forward(q, q, q)
    c = validate_attention_forward_node(y.uop)
    assert y.uop.arg == {"scale": c.scale, "mask": "none"}
    for arg, msg in (({"scale": c.scale}, "exactly 'scale' and 'mask'"),
                     ({"scale": c.scale, "mask": "causal"}, "mask must be exactly 'none'"),
                     ({"scale": 0.5, "mask": "none"}, "canonical float32")):
        with pytest.raises(ShapeError, match=msg):
            validate_attention_forward_node(UOp("ATTENTION_FORWARD", y.uop.inputs, y.uop.shape, "float32", arg))
    with pytest.raises(JitNotImplementedError, match="neither additive masks"):
        flash_attention(q, q, q, scale=0.5)
    with pytest.raises(ShapeError, match="one session"):
        attention_forward(q, Session().from_numpy(np.zeros((1, 2, 4, 8), np.float32)), q)
    with pytest.raises(TypeError):
        attention_forward(q, q, np.zeros((1, 2, 4, 8), np.float32))


def test_runtime_array_checks(rng):
    c = infer_attention_forward_contract(_T((1, 1, 3, 4)), _T((1, 1, 3, 4)), _T((1, 1, 3, 4)))
    a = rng.standard_normal((1, 1, 3, 4)).astype(np.float32)
    check_attention_forward_arrays(c, (a, a, a))
    with pytest.raises(ShapeError, match="exactly three arrays"):
        check_attention_forward_arrays(c, [a, a, a])
    with pytest.raises(ShapeError, match="exact float32 ndarray"):
        check_attention_forward_arrays(c, (a, a, a.astype(np.float64)))
    bad = a.copy()
    bad[0, 0, 1, 2] = np.nan
    with pytest.raises(ShapeError, match="only finite"):
        check_attention_forward_arrays(c, (a, bad, a))


def test_oracle_restatement_pinned(rng):
    q, k, v = (rng.standard_normal((2, 3, 9, 16)).astype(np.float32) for _ in range(3))
    scale = float(np.float32(1 / 4))
    y = O.attention_forward_f32(q, k, v, scale)
    truth = O.attention_f64(q, k, v, scale)
    assert np.max(np.abs(y - truth)) < 2e-6
    # Q = 0: uniform attention, the mean of V over keys.
    y0 = O.attention_forward_f32(np.zeros_like(q), k, v, scale)
    assert np.allclose(y0, v.mean(axis=2, keepdims=True).repeat(9, axis=2), atol=1e-6)


def test_graph_oracle_evaluates_attention_forward(rng):
    s = Session()
    arrs = [rng.standard_normal((1, 2, 5, 8), dtype=np.float32) for _ in range(3)]
    q, k, v = (s.from_numpy(a) for a in arrs)
    y = attention_forward(q, k, v)
    out = G.evaluate(y.uop, s.buffers)
    assert np.array_equal(out, O.attention_forward_f32(*arrs, y.uop.arg["scale"]))
