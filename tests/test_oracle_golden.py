"""Pins the NumPy oracle (oracle/ops.py) on CPU.

Each check is anchored outside the oracle's own formula: known answers and
fixtures copied (as data) from the reference's tests, closed forms,
float64 brute force, or an independent restatement of a rounding rule.
A plausible slip (transposed operand, dropped mask, wrong rounding) fails
one of them -- the last tests plant such slips and check that they do.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import ops as O

F16, F32 = np.float16, np.float32


# ---------------------------------------------------------------- GEMM


def test_matmul_known_answers():
    # packages/browsergrad-kernels/tests/reference.test.ts:42-59
    a = np.array([[1, 2, 3], [4, 5, 6]], F32)
    b = np.array([[7, 8], [9, 10], [11, 12]], F32)
    assert O.matmul(a, b).ravel().tolist() == [58, 64, 139, 154]
    assert O.matmul(np.array([[1, 2, 3, 4]], F32), np.array([[5], [6], [7], [8]], F32)).item() == 70
    # tests-browser/webgpu_real.test.ts:1558-1589 (bridge.matmul)
    c = O.matmul(np.array([[1, 2], [3, 4]], F32), np.array([[5, 6], [7, 8]], F32))
    assert c.ravel().tolist() == [19, 22, 43, 50]


def test_matmul_amp_f32_accumulate_invariant():
    # jit tests-integration/amp.test.ts:47-66: ones(1x4096) @ ones(4096x1) in
    # f16 is exactly 4096 with an f32 accumulator (f16 accumulation stalls at 2048).
    y = O.matmul(np.ones((1, 4096), F16), np.ones((4096, 1), F16))
    assert y.dtype == F16 and float(y[0, 0]) == 4096.0


def test_matmul_amp_vs_f32_max_rel():
    # amp.test.ts:143-175 (RandomState(0), 8x16 @ 16x8, metric |a-r|/(|r|+1e-3) < 5e-2)
    rng = np.random.RandomState(0)
    a = rng.uniform(-1, 1, size=(8, 16)).astype(F32)
    b = rng.uniform(-1, 1, size=(16, 8)).astype(F32)
    ref = a @ b
    amp = O.linear_amp(a, b, None).astype(F32)
    assert float(np.max(np.abs(amp - ref) / (np.abs(ref) + 1e-3))) < 5e-2


def test_matmul_float64_brute_force():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((17, 23)).astype(F32)
    b = rng.standard_normal((23, 19)).astype(F32)
    truth = np.array([[sum(float(a[i, k]) * float(b[k, j]) for k in range(23)) for j in range(19)]
                      for i in range(17)])
    assert np.allclose(O.matmul(a, b), truth, rtol=1e-5, atol=1e-5)


def test_identity_and_scaled_identity():
    # jit tests-integration/webgpu_realizer.test.ts:2399-2426 (I and 2I)
    x = np.arange(16, dtype=F32).reshape(4, 4)
    assert np.array_equal(O.matmul(x, np.eye(4, dtype=F32)), x)
    assert np.array_equal(O.matmul(x, 2 * np.eye(4, dtype=F32)), 2 * x)


# ---------------------------------------------------------------- elementwise


def test_fused_closed_forms():
    a = np.array([0.5, 1.0, -2.0, 3.0], F32)
    b = np.array([1.0, -0.5, 0.25, 2.0], F32)
    # webgpu_real.test.ts:1431-1472: exp(a + b) / a
    y = O.fused_program([a, b], [("ADD", -1, -2), ("EXP", 0, 0), ("DIV", 1, -1)])
    assert np.allclose(y, np.exp(a.astype(np.float64) + b) / a, rtol=1e-6)
    # webgpu_real.test.ts:245-283: log(exp(x) * y) with x=[.1,.2,.3,.4], y=[2,3,4,5]
    x = np.array([0.1, 0.2, 0.3, 0.4], F32)
    yy = np.array([2, 3, 4, 5], F32)
    z = O.fused_program([x, yy], [("EXP", -1, 0), ("MUL", 0, -2), ("LOG", 1, 0)])
    assert np.allclose(z, x + np.log(yy.astype(np.float64)), atol=1e-5)


def test_c2_chain_against_float64():
    rng = np.random.default_rng(5)
    a, b, c = (rng.standard_normal((16, 300)).astype(F32) for _ in range(3))
    a64, b64, c64 = (t.astype(np.float64) for t in (a, b, c))
    truth = (np.maximum(a64 * b64 + c64, 0) * np.exp(-(a64 * a64))).sum(axis=1)
    got = O.c2_chain(a, b, c)
    assert got.dtype == F32 and got.shape == (16,)
    assert O.within(got, truth, 1e-4).all()


def test_relu_is_where_cmp_gt():
    # reference.test.ts relu: [-2,-0.5,0,0.5,2] -> [0,0,0,0.5,2]
    x = np.array([-2, -0.5, 0, 0.5, 2], F32)
    y = O.fused_program([x], [("IMM", 0, 0, 0), ("CMP_GT", -1, 0, 0), ("WHERE", 1, -1, 0)], imms=[0.0])
    assert y.tolist() == [0, 0, 0, 0.5, 2]


# ---------------------------------------------------------------- GELU / LayerNorm / softmax


def test_gelu_known_values():
    # reference.test.ts:122-144
    y = O.gelu_tanh_f32(np.array([-2, -1, 0, 1, 2], F32))
    assert np.all(np.abs(y - np.array([-0.04540231, -0.15880801, 0, 0.8411920, 1.9545977])) < 1e-4)
    assert O.gelu_tanh_f32(np.array([0.0], F32))[0] == 0.0


def test_layer_norm_statistics_and_affine():
    # reference.test.ts:151-197
    x = np.array([[1, 2, 3, 4], [10, 20, 30, 40]], F32)
    y = O.layer_norm(x, np.ones(4, F32), np.zeros(4, F32))
    assert np.all(np.abs(y.mean(axis=1)) < 1e-4)
    assert np.all(np.abs(y.var(axis=1) - 1) < 1e-3)
    y2 = O.layer_norm(x[:1], np.full(4, 2, F32), np.full(4, 10, F32))
    assert abs(y2.mean() - 10) < 1e-3
    # closed form for [1,2,3,4]: mean 2.5, var 1.25
    expect = (np.array([1, 2, 3, 4]) - 2.5) / np.sqrt(1.25 + 1e-5)
    assert np.allclose(y[0], expect, atol=1e-6)


def test_softmax_known_rows():
    # reference.test.ts:78-118 and webgpu_real.test.ts:285-325
    assert np.allclose(O.softmax_lastaxis(np.ones((1, 4), F32)), 0.25)
    x = np.array([[1, 2, 3, 4, 5], [-1, -2, -3, -4, -5], [0.5] * 5], F32)
    assert np.all(np.abs(O.softmax_lastaxis(x).sum(axis=1) - 1) < 1e-5)
    big = O.softmax_lastaxis(np.array([[1000, 1001, 1002]], F32))
    assert np.all(np.isfinite(big)) and abs(big.sum() - 1) < 1e-5
    rows = np.array([[1, 2, 3], [-2, 0.5, 1.5]], F32)
    r64 = rows.astype(np.float64)
    e = np.exp(r64 - r64.max(axis=1, keepdims=True))
    assert np.allclose(O.softmax_lastaxis(rows), e / e.sum(axis=1, keepdims=True), atol=1e-5)


# ---------------------------------------------------------------- attention


CS336_Q = np.array([[[1, 0], [0, 1]]], F32)
CS336_K = np.array([[[1, 0], [0, 1]]], F32)
CS336_V = np.array([[[10, 20], [30, 40]]], F32)


def test_attention_cs336_fixtures():
    # packages/browsergrad-kernels/tests/flash_attention_oracle.test.ts:16-52
    nc = O.attention_f64(CS336_Q, CS336_K, CS336_V, 1.0, causal=False)
    assert np.allclose(nc.ravel(), [15.378828, 25.378828, 24.621172, 34.621172], atol=1e-5)
    c = O.attention_f64(CS336_Q, CS336_K, CS336_V, 1.0, causal=True)
    assert np.allclose(c.ravel(), [10, 20, 24.621172, 34.621172], atol=1e-5)
    # log-sum-exp of the non-causal rows: log(e^1 + e^0) = 1.313262
    s = CS336_Q[0] @ CS336_K[0].T
    assert np.allclose(np.log(np.exp(s).sum(axis=1)), [1.313262, 1.313262], atol=1e-6)
    # hard causal boundary: a very negative valid score still wins over the masked key
    hb = O.attention_f64(np.array([[[1]]], F32), np.array([[[-2e6], [0]]], F32),
                         np.array([[[7], [99]]], F32), 1.0, causal=True)
    assert hb.ravel().tolist() == [7.0]


def test_attention_zero_query_is_mean_of_v():
    # reference.test.ts:203-217
    q = np.zeros((1, 3, 2), F32)
    k = np.array([[[1, 2], [3, 4], [5, 6]]], F32)
    v = np.array([[[10, 20], [30, 40], [50, 60]]], F32)
    for f in (lambda: O.attention_f64(q, k, v, 1.0), lambda: O.attention_online_f32(q, k, v, 1.0)):
        assert np.allclose(f(), [[[30, 40]] * 3], atol=1e-4)


def lcg(n: int, seed: int) -> np.ndarray:
    """The reference test's input generator (webgpu_real.test.ts:1480-1488)."""
    out = np.empty(n, F32)
    s = seed
    for i in range(n):
        s = (s * 1103515245 + 12345) & 0x7FFFFFFF
        out[i] = (s / 0x7FFFFFFF - 0.5) * 2
    return out


def test_attention_online_on_reference_lcg_inputs():
    # webgpu_real.test.ts:1474-1556: B1 H2 S4 D8 against a loop reference, max diff < 1e-4
    B, H, S, D = 1, 2, 4, 8
    q, k, v = (lcg(B * H * S * D, s).reshape(B, H, S, D) for s in (1, 2, 3))
    ref = np.zeros((B, H, S, D))
    for h in range(H):
        for i in range(S):
            sc = np.array([sum(float(q[0, h, i, d]) * float(k[0, h, j, d]) for d in range(D)) for j in range(S)])
            sc = sc / np.sqrt(D)
            p = np.exp(sc - sc.max())
            p /= p.sum()
            ref[0, h, i] = p @ v[0, h].astype(np.float64)
    assert np.max(np.abs(O.attention_online_f32(q, k, v, 1 / np.sqrt(D)) - ref)) < 1e-4


def test_sdpa_amp_close_to_exact_and_causal_row0():
    rng = np.random.default_rng(9)
    q, k, v = (rng.standard_normal((2, 3, 40, 16)).astype(F32) for _ in range(3))
    for causal in (False, True):
        y = O.sdpa_amp(q, k, v, 0.25, causal).astype(F32)
        truth = O.attention_f64(q.astype(F16), k.astype(F16), v.astype(F16), 0.25, causal)
        assert O.within(y, truth, 2e-2).all()
    # causal row 0 attends only to key 0 -> equals v[..., 0, :] rounded to f16
    y = O.sdpa_amp(q, k, v, 0.25, True)
    assert np.array_equal(y[..., 0, :], v.astype(F16)[..., 0, :])


# ---------------------------------------------------------------- casts


def test_f32_to_f16_matches_numpy_rne():
    specials = np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 6.1e-5, 5.96e-8, 2.98e-8, np.inf, -np.inf],
                        F32)
    got = O.f32_to_f16(specials).view(np.uint16)
    assert got.tolist() == specials.astype(F16).view(np.uint16).tolist()
    # ties to even: 1 + 2^-11 is halfway between 1 and 1 + 2^-10 -> rounds to 1
    assert float(O.f32_to_f16(np.array([1 + 2.0 ** -11], F32))[0]) == 1.0
    assert float(O.f32_to_f16(np.array([1 + 3 * 2.0 ** -11], F32))[0]) == 1 + 2 * 2.0 ** -10


def _bf16_nearest_even(x: np.ndarray) -> np.ndarray:
    """Independent restatement: nearest bf16 by float64 distance, ties to the
    even mantissa, computed from the two bracketing bf16 values."""
    out = np.empty(x.shape, np.uint16)
    for i, f in enumerate(x.astype(F32)):
        if np.isnan(f):
            out[i] = 0x7FC0
            continue
        u = int(np.array(f, F32).view(np.uint32))
        lo = u & 0xFFFF0000
        hi = lo + 0x10000
        flo = float(np.array(lo, np.uint32).view(F32))
        # the upper neighbour is |lo| + one bf16 ulp (2^(e-134), subnormals 2^-133),
        # which past the largest finite value is 2^128 and encodes as infinity
        e = (lo >> 23) & 0xFF
        ulp = 2.0 ** ((e if e else 1) - 134)
        fhi = math.copysign(abs(flo) + ulp, flo) if flo != 0 else math.copysign(ulp, float(f))
        dlo, dhi = abs(float(f) - flo), abs(fhi - float(f))
        if dlo < dhi or (dlo == dhi and ((lo >> 16) & 1) == 0):
            out[i] = lo >> 16
        else:
            out[i] = (hi >> 16) & 0xFFFF
    return out


def test_f32_to_bf16_against_independent_rule():
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.standard_normal(4000).astype(F32) * 10 ** rng.uniform(-30, 30, 4000).astype(F32),
                        np.array([1.0, -1.0, 0.0, -0.0, 3.4e38, -3.4e38, 1e-40], F32)])
    # exact ties: lower 16 bits == 0x8000
    ties = (rng.integers(0, 2 ** 31, 500, dtype=np.uint32) & 0x7F7F0000) | 0x8000
    x = np.concatenate([x, ties.view(F32)])
    x = x[np.isfinite(x)]
    assert np.array_equal(O.f32_to_bf16_bits(x), _bf16_nearest_even(x))


def test_bf16_exhaustive_round_trip():
    bits = np.arange(2 ** 16, dtype=np.uint32).astype(np.uint16)
    f = O.bf16_bits_to_f32(bits)
    finite = np.isfinite(f)
    assert np.array_equal(O.f32_to_bf16_bits(f[finite]), bits[finite])
    nan = np.isnan(f)
    assert np.all(np.isnan(O.bf16_bits_to_f32(O.f32_to_bf16_bits(f[nan]))))


# ---------------------------------------------------------------- tolerance rule and planted slips


def test_within_abs_or_rel_rule():
    # semantic-core attention-forward-model.ts:25-29: |y-r| <= tol or |y-r| <= tol*|r|
    assert O.within(np.array([1.00009]), np.array([1.0]), 1e-4).all()
    assert O.within(np.array([1000.09]), np.array([1000.0]), 1e-4).all()
    assert not O.within(np.array([1000.2]), np.array([1000.0]), 1e-4).any()
    assert O.within(np.array([np.inf, np.nan]), np.array([np.inf, np.nan]), 1e-4).all()


def test_planted_slips_are_caught():
    rng = np.random.default_rng(13)
    a = rng.uniform(-1, 1, (12, 12)).astype(F32)
    b = rng.uniform(-1, 1, (12, 12)).astype(F32)
    truth = a.astype(np.float64) @ b.astype(np.float64)
    assert O.within(O.matmul(a, b), truth, 1e-4).all()
    assert not O.within(O.matmul(a, b.T), truth, 1e-4).all()       # transposed operand
    q, k, v = (rng.standard_normal((1, 9, 4)).astype(F32) for _ in range(3))
    c = O.attention_f64(q, k, v, 0.5, causal=True)
    assert not np.allclose(c, O.attention_f64(q, k, v, 0.5, causal=False))  # dropped mask
    x = rng.standard_normal(64).astype(F32)
    assert not np.array_equal(O.f32_to_bf16_bits(x), (x.view(np.uint32) >> 16).astype(np.uint16))  # truncation
    z = rng.standard_normal((3, 50)).astype(F32)
    assert not np.allclose(O.c2_chain(z, z, z), O.c2_chain(z, z, -z))  # sign slip
