"""The f32 attention kernel on MFMA (k_attn32.hip) against the oracle.

It serves the bridge's f32 flash_attention (with and without the additive
mask, flash_attention.ts:45-211 behind realizer.ts:1122-1151), f32
attention_ex (causal or not, strided views) and so the typed
ATTENTION_FORWARD and the semantic attention.  Bar: 1e-4 (the reference's
f32 contract, flash_attention.ts:25-28), against the float64 brute-force
attention and the legacy online-softmax oracle; the CS336 known answers
(flash_attention_oracle.test.ts:16-52) run through the kernel itself.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import ops as O

pytestmark = pytest.mark.gpu
TOL = 1e-4


def up(br, a, dtype=None):
    a = np.ascontiguousarray(a)
    return br.upload(a, a.shape, dtype or a.dtype.name)


def launched(br, fn):
    br.set_launch_log(True)
    try:
        br.take_launch_log()
        out = fn()
        names = [r["kernel"] for r in br.take_launch_log()]
    finally:
        br.set_launch_log(False)
    return out, names


def fa32_ran(names):
    return any("fa32_fwd_kernel" in t for t in names)


@pytest.mark.parametrize("b,h,sq,sk,d", [(1, 1, 1, 1, 1), (2, 3, 33, 33, 16), (1, 2, 130, 70, 64),
                                         (2, 2, 64, 200, 7), (1, 1, 257, 257, 33), (1, 2, 300, 300, 64),
                                         (3, 1, 96, 128, 24), (1, 1, 1000, 1000, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_f32_mfma_against_f64(bridge, rng, b, h, sq, sk, d, causal):
    print(f"[case] f32 attention b{b} h{h} sq{sq} sk{sk} d{d} causal={causal}", flush=True)
    q = rng.standard_normal((b, h, sq, d)).astype(np.float32)
    k = rng.standard_normal((b, h, sk, d)).astype(np.float32)
    v = rng.standard_normal((b, h, sk, d)).astype(np.float32)
    scale = 1.0 / np.sqrt(d)
    hs = [up(bridge, t) for t in (q, k, v)]
    ho, names = launched(bridge, lambda: bridge.attention_ex(*hs, batch=b, heads=h, sq=sq, sk=sk, d=d, scale=scale,
                                                            causal=causal, in_dtype="float32"))
    assert fa32_ran(names), names
    y = bridge.to_numpy(ho)
    ref = O.attention_f64(q, k, v, scale, causal=causal)
    if causal and sq > sk:
        pass  # queries past Sk see every key (top-left aligned mask), as attention_f64 computes
    assert O.within(y, ref, TOL).all(), O.report(y, ref, TOL)
    if not causal:
        ref2 = O.attention_online_f32(q, k, v, scale)
        assert O.within(y, ref2, TOL).all(), O.report(y, ref2, TOL)
    for t in (*hs, ho):
        bridge.release(t)


@pytest.mark.parametrize("mshape", ["sq_sk", "1_1", "b_1", "1_h", "b_h"])
def test_attention_f32_additive_mask(bridge, rng, mshape):
    """flash_attention with an additive f32 mask broadcast over batch and
    head, including -1e9 entries, -inf entries and a fully -inf row (the
    reference's -1e20 sentinel and l > 0 guard give that row zeros)."""
    b, h, s, d = 2, 3, 70, 64
    q, k, v = (rng.standard_normal((b, h, s, d)).astype(np.float32) for _ in range(3))
    shp = {"sq_sk": (s, s), "1_1": (1, 1, s, s), "b_1": (b, 1, s, s), "1_h": (1, h, s, s),
           "b_h": (b, h, s, s)}[mshape]
    mask = np.where(rng.random(shp) < 0.2, -1e9, 0).astype(np.float32)
    mask = np.where(rng.random(shp) < 0.05, -np.inf, mask).astype(np.float32)
    mask[..., 5, :] = -np.inf
    mask = (mask + rng.uniform(-0.5, 0.5, shp)).astype(np.float32)
    ho, names = launched(bridge, lambda: bridge.flash_attention(up(bridge, q), up(bridge, k), up(bridge, v),
                                                                up(bridge, mask), b, h, s, s, d, 0.125, "float32"))
    assert fa32_ran(names), names
    y = bridge.to_numpy(ho)
    full = np.broadcast_to(mask if mask.ndim == 4 else mask[None, None], (b, h, s, s))
    ref = O.attention_online_f32(q, k, v, 0.125, full)
    assert np.all(y[:, :, 5] == 0.0)
    assert O.within(y, ref, TOL).all(), O.report(y, ref, TOL)


def test_attention_f32_strided_views(bridge, rng):
    """Q, K, V as views into one [B, S, 3, H, D] projection (row stride 3HD)
    and an odd head dim (scalar loads), output [B, S, H, D]."""
    B, S, H, D = 2, 150, 3, 20
    qkv = rng.standard_normal((B, S, 3, H, D)).astype(np.float32)
    hqkv = up(bridge, qkv)
    sb, ss, sh = S * 3 * H * D, 3 * H * D, D
    views = [(i * H * D, sb, sh, ss) for i in range(3)]
    ho, names = launched(bridge, lambda: bridge.attention_ex(
        hqkv, hqkv, hqkv, batch=B, heads=H, sq=S, sk=S, d=D, scale=0.3, causal=True, in_dtype="float32",
        q_view=views[0], k_view=views[1], v_view=views[2], o_strides=(S * H * D, D, H * D)))
    assert fa32_ran(names), names
    y = bridge.to_numpy(ho).reshape(B, S, H, D)
    q, k, v = (np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)) for i in range(3))
    ref = O.attention_f64(q, k, v, 0.3, causal=True).transpose(0, 2, 1, 3)
    assert O.within(y, ref, TOL).all(), O.report(y, ref, TOL)


def test_attention_f32_cs336_known_answers(bridge):
    """flash_attention_oracle.test.ts:16-52 through the kernel: q = k = I2,
    v = [[10, 20], [30, 40]], scale 1."""
    q = np.array([[[[1, 0], [0, 1]]]], np.float32)
    v = np.array([[[[10, 20], [30, 40]]]], np.float32)
    for causal, want in ((False, [15.378828, 25.378828, 24.621172, 34.621172]),
                         (True, [10, 20, 24.621172, 34.621172])):
        ho = bridge.attention_ex(up(bridge, q), up(bridge, q), up(bridge, v), batch=1, heads=1, sq=2, sk=2, d=2,
                                 scale=1.0, causal=causal, in_dtype="float32")
        assert np.allclose(bridge.to_numpy(ho).ravel(), want, atol=1e-4)
    # a very negative valid score still wins over the causally masked key
    ho = bridge.attention_ex(up(bridge, np.ones((1, 1, 1, 1), np.float32)),
                             up(bridge, np.array([[[[-2e6], [0]]]], np.float32)),
                             up(bridge, np.array([[[[7], [99]]]], np.float32)),
                             batch=1, heads=1, sq=1, sk=2, d=1, scale=1.0, causal=True, in_dtype="float32")
    assert bridge.to_numpy(ho).ravel().tolist() == [7.0]


def test_attention_f32_zero_query_is_mean_of_v(bridge):
    # reference.test.ts:203-217
    q = np.zeros((1, 1, 3, 2), np.float32)
    k = np.array([[[[1, 2], [3, 4], [5, 6]]]], np.float32)
    v = np.array([[[[10, 20], [30, 40], [50, 60]]]], np.float32)
    ho = bridge.flash_attention(up(bridge, q), up(bridge, k), up(bridge, v), 0, 1, 1, 3, 3, 2, 1.0, "float32")
    assert np.allclose(bridge.to_numpy(ho), [[[[30, 40]] * 3]], atol=1e-4)
