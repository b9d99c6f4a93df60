"""bg_matmul_ex2 (GPU): the residual epilogue and operands cast in a pre-pass.

Both extras are checked bit-exactly against the entry point they extend:
* residual: bg_matmul_ex2(..., residual=r) must equal bg_matmul_ex's f32
  result plus r in float32 (the epilogue adds r last, one f32 add);
* cast operands: bg_matmul_ex2 on f32 storage must equal bg_matmul_ex on
  operands rounded to the 16-bit type by NumPy's astype (nearest even);
and against the oracle's autocast `x + linear(h)` at the 16-bit tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import ops as O

pytestmark = pytest.mark.gpu

F32 = np.float32


def up(br, a, dtype=None):
    a = np.ascontiguousarray(a)
    return br.upload(a, a.shape, dtype or a.dtype.name)


@pytest.mark.parametrize("m,k,n", [(17, 24, 19), (256, 256, 256), (300, 136, 200), (1024, 768, 512),
                                   (8192 // 8, 768, 768)])
@pytest.mark.parametrize("act", [0, 1, 2])
@pytest.mark.parametrize("out_dtype", ["float32", "float16"])
def test_residual_epilogue_16bit(bridge, rng, m, k, n, act, out_dtype):
    x = rng.uniform(-1, 1, (m, k)).astype(F32)
    w = rng.standard_normal((n, k)).astype(F32) * F32(0.05)
    b = rng.uniform(-0.1, 0.1, (n,)).astype(F32)
    r = rng.standard_normal((m, n)).astype(F32)
    hx, hw, hb, hr = up(bridge, x.astype(np.float16)), up(bridge, w.astype(np.float16)), up(bridge, b), up(bridge, r)
    kw = dict(m=m, n=n, k=k, trans_b=True, in_dtype="float16", out_dtype="float32", bias=hb, round_out=True, act=act)
    base = bridge.to_numpy(bridge.matmul_ex(hx, hw, **kw))
    kw["out_dtype"] = out_dtype
    got = bridge.to_numpy(bridge.matmul_ex(hx, hw, residual=hr, **kw))
    want = (base + r).astype(out_dtype)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), "residual epilogue is not one f32 add"
    # and the reference graph: x + act(linear(h)) under autocast
    ref = O.linear_amp(x, w.T, b)
    if act == 1:
        ref = np.where(ref > 0, ref, F32(0)).astype(F32)
    elif act == 2:
        ref = O.gelu_tanh_f32(ref)
    rep = O.report(got.astype(F32), (ref + r).astype(F32), 2e-2)
    assert rep["pass"], rep


@pytest.mark.parametrize("m,k,n", [(64, 784, 128), (129, 65, 257), (256, 512, 384)])
def test_residual_epilogue_f32(bridge, rng, m, k, n):
    """f32 GEMM, including the split-K path (64 x 784 x 128: partial sums
    plus a finishing pass that applies the epilogue)."""
    x, w = rng.uniform(-1, 1, (m, k)).astype(F32), rng.uniform(-1, 1, (n, k)).astype(F32)
    b, r = rng.uniform(-1, 1, (n,)).astype(F32), rng.standard_normal((m, n)).astype(F32)
    hx, hw, hb, hr = up(bridge, x), up(bridge, w), up(bridge, b), up(bridge, r)
    for act in (0, 1):
        kw = dict(m=m, n=n, k=k, trans_b=True, in_dtype="float32", bias=hb, act=act)
        base = bridge.to_numpy(bridge.matmul_ex(hx, hw, **kw))
        got = bridge.to_numpy(bridge.matmul_ex(hx, hw, residual=hr, **kw))
        assert np.array_equal(got, (base + r).astype(F32))


def test_residual_epilogue_batched(bridge, rng):
    bt, m, k, n = 3, 96, 64, 160
    x = rng.uniform(-1, 1, (bt, m, k)).astype(np.float16)
    w = rng.uniform(-1, 1, (bt, n, k)).astype(np.float16)
    r = rng.standard_normal((bt, m, n)).astype(F32)
    hx, hw, hr = up(bridge, x), up(bridge, w), up(bridge, r)
    kw = dict(m=m, n=n, k=k, batch=bt, trans_b=True, in_dtype="float16", out_dtype="float32")
    base = bridge.to_numpy(bridge.matmul_ex(hx, hw, **kw))
    got = bridge.to_numpy(bridge.matmul_ex(hx, hw, residual=hr, **kw))
    assert np.array_equal(got, (base + r).astype(F32))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("m,k,n,trans_b", [(17, 24, 19, False), (17, 24, 19, True), (256, 256, 256, False),
                                           (300, 136, 200, True), (512, 1024, 384, False), (100, 36, 60, False)])
def test_cast_operands_in_prepass(bridge, rng, dtype, m, k, n, trans_b):
    x = rng.uniform(-1, 1, (m, k)).astype(F32)
    w = rng.uniform(-1, 1, (n, k) if trans_b else (k, n)).astype(F32)
    b = rng.uniform(-0.1, 0.1, (n,)).astype(F32)
    hb = up(bridge, b)
    kw = dict(m=m, n=n, k=k, trans_b=trans_b, in_dtype=dtype, out_dtype="float32", bias=hb, round_out=True)
    hx32, hw32 = up(bridge, x), up(bridge, w)
    got = bridge.to_numpy(bridge.matmul_ex(hx32, hw32, a_dtype="float32", b_dtype="float32", **kw))
    if dtype == "float16":
        hx16, hw16 = up(bridge, x.astype(np.float16)), up(bridge, w.astype(np.float16))
    else:
        hx16 = bridge.upload(O.f32_to_bf16_bits(x), x.shape, "bfloat16")
        hw16 = bridge.upload(O.f32_to_bf16_bits(w), w.shape, "bfloat16")
    base = bridge.to_numpy(bridge.matmul_ex(hx16, hw16, **kw))
    assert np.array_equal(got, base), "pre-pass cast differs from astype rounding"
    # one operand cast, the other already 16-bit
    got_a = bridge.to_numpy(bridge.matmul_ex(hx32, hw16, a_dtype="float32", **kw))
    assert np.array_equal(got_a, base)
    if dtype == "float16":
        ref = O.linear_amp(x, w.T if trans_b else w, b)
        assert O.report(got, ref, 2e-2)["pass"]


def test_cast_operands_batched_and_broadcast_b(bridge, rng):
    bt, m, k, n = 2, 64, 48, 80
    x = rng.uniform(-1, 1, (bt, m, k)).astype(F32)
    w = rng.uniform(-1, 1, (k, n)).astype(F32)
    kw = dict(m=m, n=n, k=k, batch=bt, stride_b=0, trans_b=False, in_dtype="float16", out_dtype="float32")
    got = bridge.to_numpy(bridge.matmul_ex(up(bridge, x), up(bridge, w), a_dtype="float32", b_dtype="float32", **kw))
    base = bridge.to_numpy(bridge.matmul_ex(up(bridge, x.astype(np.float16)), up(bridge, w.astype(np.float16)), **kw))
    assert np.array_equal(got, base)


def test_ex2_refusals(bridge, rng):
    from browsergrad_amd.errors import KernelError as RealizationError
    x = up(bridge, rng.uniform(-1, 1, (32, 64)).astype(F32))
    w = up(bridge, rng.uniform(-1, 1, (48, 64)).astype(np.float16))
    bad_r = up(bridge, np.zeros((31, 48), F32))
    kw = dict(m=32, n=48, k=64, trans_b=True, in_dtype="float16", out_dtype="float32")
    with pytest.raises(RealizationError, match="residual must be float32"):
        bridge.matmul_ex(up(bridge, np.zeros((32, 64), np.float16)), w, residual=bad_r, **kw)
    with pytest.raises(RealizationError, match="stored as"):
        bridge.matmul_ex(x, w, a_dtype="float16", **kw)  # x is f32, claimed f16
    with pytest.raises(RealizationError, match="dense"):
        bridge.matmul_ex(x, w, a_dtype="float32", lda=96, **{**kw, "k": 64})
    with pytest.raises(RealizationError, match="dense output"):
        r = up(bridge, np.zeros((32, 48), F32))
        bridge.matmul_ex(up(bridge, np.zeros((32, 64), np.float16)), w, residual=r, ldc=64, **kw)
