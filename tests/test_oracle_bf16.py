"""Pins the bfloat16 functions of the oracle on CPU: ``ops.matmul_bf16``,
``ops.sdpa_bf16`` and the bfloat16 branch of ``graph.evaluate``.

bfloat16 has no reference oracle: the reference IR has no bf16 dtype
(packages/browsergrad-jit/src/python/_ir.py:348-353) and its autocast
policy names float16 only (_amp.py:56-69, 123-128).  This build defines the
bf16 path as the reference's AMP graph with bf16 in place of f16: MATMUL
operands and results are narrow with f32 accumulation (_realize.py:395-412),
the softmax runs in f32 (_functional.py:1505-1533), and P is cast to the
narrow dtype before the PV product.

Nothing here re-evaluates the oracle's own formula.  Each check fixes the
answer from outside it:
  * exact integer arithmetic (sums below 2^24, so every f32 accumulation
    order is exact) rounded by ``rne_bf16``, an exact-rational nearest-even
    rule written from the format (8 significant bits) with Fraction;
  * closed-form softmax values (equal scores give exactly 1/n; a single
    valid key gives exactly 1);
  * float64 truth with the error bound of one bf16 rounding;
  * planted slips (P not rounded, S not rounded, truncating casts, dropped
    mask, bf16 accumulation, transposed operand) that must fail a pin.
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

from browsergrad_amd.jit import configs
from browsergrad_amd.jit.ir import toposort
from browsergrad_amd.jit.tensor import Session, autocast
from oracle import graph as G
from oracle import ops as O

F32 = np.float32


def rne_bf16(x) -> float:
    """Nearest bfloat16 to the exact value x (8 significant bits, ties to the
    even significand), normal range only; computed on exact rationals."""
    if isinstance(x, np.integer):
        x = int(x)
    elif isinstance(x, np.floating):
        x = float(x)
    f = Fraction(x)
    if f == 0:
        return 0.0
    sign = -1 if f < 0 else 1
    a = abs(f)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    assert -126 <= e <= 127, "rne_bf16 covers the normal range only"
    q = a / Fraction(2) ** (e - 7)          # significand scaled to [128, 256)
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * float(n * Fraction(2) ** (e - 7))


def bits(x) -> np.ndarray:
    """bf16 bit patterns of values that are exactly bf16 (asserted)."""
    x = np.asarray(x, dtype=F32)
    b = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(O.bf16_bits_to_f32(b), x), "value is not bf16-representable"
    return b


def val(b) -> np.ndarray:
    return O.bf16_bits_to_f32(b).astype(np.float64)


def test_rne_bf16_rule_itself():
    # 8 significant bits: 256..512 has spacing 2; ties go to the even significand.
    assert rne_bf16(257) == 256.0 and rne_bf16(259) == 260.0 and rne_bf16(258) == 258.0
    assert rne_bf16(Fraction(1, 3)) == 0.333984375      # 171 / 512
    assert rne_bf16(-1.00390625) == -1.0                # tie below 1 + 2^-7 -> even (1.0)
    assert rne_bf16(1.01171875) == 1.015625             # tie between 1+2^-7 and 1+2^-6 -> even


# ---------------------------------------------------------------- matmul_bf16


def test_matmul_bf16_known_answers_and_f32_accumulation():
    # reference.test.ts:42-59 values are exact in bf16
    a, b = bits([[1, 2, 3], [4, 5, 6]]), bits([[7, 8], [9, 10], [11, 12]])
    assert val(O.matmul_bf16(a, b)).ravel().tolist() == [58, 64, 139, 154]
    # amp.test.ts:47-66 analogue: ones(1x4096) @ ones(4096x1) is exactly 4096
    # with an f32 accumulator (a bf16 accumulator stalls at 256).
    ones = bits(np.ones((1, 4096)))
    assert val(O.matmul_bf16(ones, ones.reshape(4096, 1).copy())).item() == 4096.0


def _int_case(seed, m=9, k=64, n=7, lo=-120, hi=121):
    rng = np.random.default_rng(seed)
    a = rng.integers(lo, hi, (m, k))
    b = rng.integers(lo, hi, (k, n))
    return a, b, a @ b                                    # exact int64; |sum| < 2^24


def test_matmul_bf16_exact_integer_sums_round_nearest_even():
    for seed in range(4):
        a, b, exact = _int_case(seed)
        got = val(O.matmul_bf16(bits(a), bits(b)))
        want = np.vectorize(rne_bf16)(exact)
        assert np.array_equal(got, want)
        assert (exact != want).mean() > 0.5               # the cases do exercise rounding


def test_matmul_bf16_against_float64_truth():
    rng = np.random.default_rng(21)
    a = O.f32_to_bf16_bits(rng.standard_normal((33, 200)).astype(F32))
    b = O.f32_to_bf16_bits(rng.standard_normal((200, 17)).astype(F32))
    truth = val(a) @ val(b)
    mag = np.abs(val(a)) @ np.abs(val(b))
    got = val(O.matmul_bf16(a, b))
    # one bf16 rounding (unit roundoff 2^-8 for 8 significant bits) of an f32
    # sum (at most K * 2^-24 of sum |a||b|)
    bound = 2.0 ** -8 * np.abs(truth) + (200 * 2.0 ** -24) * mag * (1 + 2.0 ** -8)
    assert np.all(np.abs(got - truth) <= bound)


def test_matmul_bf16_planted_slips_fail():
    a, b, exact = _int_case(5)
    want = np.vectorize(rne_bf16)(exact)
    ab, bb = bits(a), bits(b)

    def truncating(x, y):                                  # cast by dropping the low half
        p = O.bf16_bits_to_f32(x) @ O.bf16_bits_to_f32(y)
        return (p.view(np.uint32) >> 16).astype(np.uint16)

    def bf16_accumulate(x, y):                             # accumulator rounded every step
        xa, ya = O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(y)
        acc = np.zeros((xa.shape[0], ya.shape[1]), F32)
        for kk in range(xa.shape[1]):
            acc = O.round_bf16(acc + np.outer(xa[:, kk], ya[kk]))
        return O.f32_to_bf16_bits(acc)

    assert np.array_equal(val(O.matmul_bf16(ab, bb)), want)
    assert not np.array_equal(val(truncating(ab, bb)), want)
    assert not np.array_equal(val(bf16_accumulate(ab, bb)), want)
    sq_a, sq_b, sq_exact = _int_case(6, m=8, k=8, n=8)
    assert not np.array_equal(val(O.matmul_bf16(bits(sq_a), bits(sq_b.T.copy()))),
                              np.vectorize(rne_bf16)(sq_exact))           # transposed operand
    ones = bits(np.ones((1, 4096)))
    assert val(bf16_accumulate(ones, ones.reshape(4096, 1).copy())).item() != 4096.0


# ---------------------------------------------------------------- sdpa_bf16


def _uniform_case(n_keys, d, seed):
    """Q = 0: every score is 0, so softmax gives exactly 1/n over the valid keys."""
    rng = np.random.default_rng(seed)
    q = bits(np.zeros((1, 1, n_keys, d)))
    k = O.f32_to_bf16_bits(rng.standard_normal((1, 1, n_keys, d)).astype(F32))
    v = bits(rng.integers(-60, 61, (1, 1, n_keys, d)))
    return q, k, v


def _uniform_expected(v, causal):
    """out[i, c] = rne(sum_{j valid} rne(1/n_i) * v[j, c]); the products and
    their sum are exact in f32 (8 + 6 significant bits, n <= 64 terms)."""
    vv = val(v)[0, 0]
    n_keys, d = vv.shape
    out = np.empty((n_keys, d))
    for i in range(n_keys):
        valid = i + 1 if causal else n_keys
        p = Fraction(rne_bf16(Fraction(1, valid)))
        for c in range(d):
            out[i, c] = rne_bf16(sum(p * Fraction(float(vv[j, c])) for j in range(valid)))
    return out


def _s_rounding_case(pairs):
    """Two keys per query row, D = 2, Q = [1, 1]: the scores are the integer
    dot products k0[0]+k0[1] and k1[0]+k1[1].  V = [[1], [-1]]."""
    k = np.array([[[[a0, a1], [b0, b1]]] for (a0, a1), (b0, b1) in pairs], F32)
    nb = len(pairs)
    q = bits(np.ones((nb, 1, 1, 2)))
    v = bits(np.tile(np.array([[1.0], [-1.0]], F32), (nb, 1, 1, 1)))
    return q, bits(k), v


def _sdpa_slipped(q_bits, k_bits, v_bits, scale, causal, *, round_s=True, round_p=True,
                  truncate=False, mask=True):
    """The bf16 SDPA definition with one step planted wrong (test use only)."""
    def rnd(x):
        if truncate:
            return ((np.asarray(x, F32).view(np.uint32) >> 16) << 16).view(F32)
        return O.round_bf16(x)
    q, k, v = (O.bf16_bits_to_f32(t) for t in (q_bits, k_bits, v_bits))
    out = np.empty(q.shape[:-1] + (v.shape[-1],), F32)
    sq, sk = q.shape[-2], k.shape[-2]
    m = np.triu(np.ones((sq, sk), bool), k=1)
    for idx in np.ndindex(*q.shape[:-2]):
        s = q[idx] @ k[idx].T
        s = (rnd(s) if round_s else s) * F32(scale)
        if causal and mask:
            s = np.where(m, F32(-np.inf), s).astype(F32)
        p = O.softmax_lastaxis(s)
        out[idx] = rnd((rnd(p) if round_p else p) @ v[idx])
    return out.astype(np.float64)


def test_sdpa_bf16_causal_row0_is_v0():
    rng = np.random.default_rng(31)
    q, k, v = (O.f32_to_bf16_bits(rng.standard_normal((2, 3, 20, 16)).astype(F32)) for _ in range(3))
    y = O.sdpa_bf16(q, k, v, 0.25, True)
    assert np.array_equal(y[..., 0, :], v[..., 0, :])
    assert not np.array_equal(bits(_sdpa_slipped(q, k, v, 0.25, True, mask=False)[..., 0, :]), v[..., 0, :])


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_bf16_uniform_scores_closed_form(causal):
    for n_keys, seed in ((3, 1), (7, 2), (48, 3)):
        q, k, v = _uniform_case(n_keys, 8, seed)
        want = _uniform_expected(v, causal)
        assert np.array_equal(val(O.sdpa_bf16(q, k, v, 0.5, causal))[0, 0], want)
    # the same pin rejects a softmax whose P is not rounded before P @ V
    q, k, v = _uniform_case(48, 8, 3)
    assert not np.array_equal(_sdpa_slipped(q, k, v, 0.5, causal, round_p=False)[0, 0],
                              _uniform_expected(v, causal))


def test_sdpa_bf16_scores_rounded_before_scaling():
    # q.k = 256 and 257: 257 rounds to 256 (tie to even), so both keys get
    # P = 1/2 exactly and the output is 1/2 - 1/2 = 0.  Same for 260 / 259
    # (259 rounds up to 260).
    q, k, v = _s_rounding_case([((128, 128), (129, 128)), ((130, 130), (130, 129))])
    y = val(O.sdpa_bf16(q, k, v, 0.5, False))
    assert y.ravel().tolist() == [0.0, 0.0]
    # 258 vs 259 -> 258 vs 260: the scaled scores differ by exactly 1, so
    # P = (1/(1+e), e/(1+e)) and the output is rne(rne(P0) - rne(P1)).
    q2, k2, v2 = _s_rounding_case([((129, 129), (130, 129))])
    p0, p1 = 1 / (1 + math.e), math.e / (1 + math.e)
    want = rne_bf16(Fraction(rne_bf16(p0)) - Fraction(rne_bf16(p1)))
    assert val(O.sdpa_bf16(q2, k2, v2, 0.5, False)).item() == want == -0.4609375
    # slips: scores not rounded, or rounded by truncation (259 -> 258)
    assert _sdpa_slipped(q, k, v, 0.5, False, round_s=False).ravel().tolist() != [0.0, 0.0]
    assert _sdpa_slipped(q, k, v, 0.5, False, truncate=True).ravel().tolist() != [0.0, 0.0]


def test_sdpa_bf16_against_float64_attention():
    rng = np.random.default_rng(9)
    q, k, v = (O.f32_to_bf16_bits(rng.standard_normal((2, 3, 40, 16)).astype(F32)) for _ in range(3))
    for causal in (False, True):
        y = val(O.sdpa_bf16(q, k, v, 0.25, causal))
        truth = O.attention_f64(val(q), val(k), val(v), 0.25, causal)
        assert O.within(y, truth, 2e-2).all()
    causal_truth = O.attention_f64(val(q), val(k), val(v), 0.25, True)
    assert not O.within(_sdpa_slipped(q, k, v, 0.25, True, mask=False), causal_truth, 2e-2).all()
    k_rev = np.ascontiguousarray(k[..., ::-1, :])             # keys paired with the wrong values
    assert not O.within(val(O.sdpa_bf16(q, k_rev, v, 0.25, True)), causal_truth, 2e-2).all()


def test_sdpa_bf16_correct_definition_passes_every_pin():
    """The planted-slip helper with no slip equals the oracle bit for bit, so
    the slips above differ from the oracle only in the step they plant."""
    rng = np.random.default_rng(17)
    q, k, v = (O.f32_to_bf16_bits(rng.standard_normal((1, 2, 24, 8)).astype(F32)) for _ in range(3))
    for causal in (False, True):
        assert np.array_equal(_sdpa_slipped(q, k, v, 0.3, causal), val(O.sdpa_bf16(q, k, v, 0.3, causal)))


# ---------------------------------------------------------------- graph.evaluate, bfloat16 branch


def test_graph_bf16_matmul_exact_integers():
    a, b, exact = _int_case(11, m=5, k=40, n=6)
    s = Session()
    ta, tb = s.from_numpy(a.astype(F32)), s.from_numpy(b.astype(F32))
    with autocast("bfloat16"):
        r = ta @ tb
    out = G.evaluate(r.uop, s.buffers)
    assert np.array_equal(out.astype(np.float64), np.vectorize(rne_bf16)(exact))
    ones, col = s.from_numpy(np.ones((1, 4096), F32)), s.from_numpy(np.ones((4096, 1), F32))
    with autocast("bfloat16"):
        r2 = ones @ col
    assert G.evaluate(r2.uop, s.buffers).item() == 4096.0


def test_graph_bf16_c3_matches_pinned_ops():
    s, y = configs.c3(scale=1 / 64)
    x, w, b = (s.buffers.get(n.inputs[0].arg) for n in toposort(y.uop) if n.op == "LOAD")
    s2 = Session()
    tx, tw, tb = s2.from_numpy(x), s2.from_numpy(w), s2.from_numpy(b)
    with autocast("bfloat16"):
        yb = tx @ tw + tb
    got = G.evaluate(yb.uop, s2.buffers)
    want = O.bf16_bits_to_f32(O.matmul_bf16(O.f32_to_bf16_bits(x), O.f32_to_bf16_bits(w))) + b
    assert got.dtype == F32 and np.array_equal(got, want)


def test_graph_bf16_c4_matches_pinned_sdpa():
    s, y = configs.c4(scale=1 / 32, dtype="bfloat16")
    got = G.evaluate(y.uop, s.buffers)
    q, k, v = (s.buffers.get(n.inputs[0].arg) for n in toposort(y.uop)
               if n.op == "LOAD" and n.dtype == "float16")
    qb, kb, vb = (O.f32_to_bf16_bits(t.astype(F32)) for t in (q, k, v))
    assert np.array_equal(got, val(O.sdpa_bf16(qb, kb, vb, 0.125, True)).astype(F32))


def test_graph_bf16_rounding_slip_is_caught(monkeypatch):
    """Dropping the per-op bf16 rounding in the graph oracle breaks the pins."""
    a, b, exact = _int_case(12, m=4, k=40, n=4)
    s = Session()
    ta, tb = s.from_numpy(a.astype(F32)), s.from_numpy(b.astype(F32))
    with autocast("bfloat16"):
        r = ta @ tb
    monkeypatch.setattr(G, "_fix", lambda x, dtype: np.asarray(x))
    out = G.evaluate(r.uop, s.buffers)
    assert not np.array_equal(out.astype(np.float64), np.vectorize(rne_bf16)(exact))
