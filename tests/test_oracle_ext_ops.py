"""Pins the extension opcodes of ``oracle.ops.fused_program`` on CPU.

The reference's fused-elementwise program has six opcodes
(fused_elementwise.ts:83-110: ADD MUL DIV NEG EXP LOG); this build's fused
kernel adds MAX MIN SUB TANH SQRT RECIP ABS COPY ROUND_F16 ROUND_BF16 (and
the comparisons and WHERE) for the plan-level fuser.  The oracle evaluates
them with NumPy in float32.  Each check below fixes the answer from outside
that formula:
  * IEEE facts that hold for a correctly rounded operation: f32 sqrt and
    reciprocal equal the float64 result rounded once to f32 (53 >= 2*24 + 2
    bits, so the double rounding is exact), MAX / MIN of exact values, SUB
    equal to ADD of the negation, ABS clearing the sign bit only, COPY the
    identity on every bit pattern;
  * Python's ``math.tanh`` in float64 (an independent libm) within two f32
    ulps (NumPy's float32 tanh is not correctly rounded: it lands up to
    1.25 ulp away near |x| = 0.5), tanh odd and saturating to exactly 1;
  * ROUND_F16 against Python's ``struct`` half-float packing, which rounds
    to nearest even by its own algorithm (ties, overflow to infinity,
    subnormals);
  * planted slips (min for max, truncation for round-to-nearest, a
    reciprocal through f16) that must fail a pin.
"""
from __future__ import annotations

import math
import struct

import numpy as np
import pytest

from oracle import ops as O

F32 = np.float32


def run1(code, x, y=None):
    ins = [np.asarray(x, F32)] + ([np.asarray(y, F32)] if y is not None else [])
    ops = [(code, -1, -2 if y is not None else 0, 0)]
    return np.asarray(O.fused_program(ins, ops), F32)


def sample(n=4096, seed=0):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    x = bits.view(F32)
    return x[np.isfinite(x)]


def test_max_min_on_exact_values_and_nan():
    a = np.array([1, -3, 0.5, -0.0, 7, np.nan, 2], F32)
    b = np.array([2, 4, -0.5, 3, 7, 1, np.nan], F32)
    mx, mn = run1("MAX", a, b), run1("MIN", a, b)
    assert mx[:5].tolist() == [2, 4, 0.5, 3, 7] and mn[:5].tolist() == [1, -3, -0.5, -0.0, 7]
    assert np.isnan(mx[5:]).all() and np.isnan(mn[5:]).all()  # NaN propagates, as np.maximum does
    assert not np.array_equal(run1("MIN", a[:5], b[:5]), mx[:5])  # planted slip: min for max


def test_sub_is_add_of_negation():
    a, b = sample(seed=1), sample(seed=2)
    n = min(len(a), len(b))
    a, b = a[:n], b[:n]
    got = run1("SUB", a, b)
    via = np.asarray(O.fused_program([a, b], [("NEG", -2, 0, 0), ("ADD", -1, 0, 0)]), F32)
    same = (got.view(np.uint32) == via.view(np.uint32)) | (np.isnan(got) & np.isnan(via))
    assert same.all()
    assert run1("SUB", [5.0], [7.0]).tolist() == [-2.0]


def test_sqrt_and_recip_are_correctly_rounded():
    x = np.abs(sample(seed=3))
    x = x[x > 0]
    s = run1("SQRT", x)
    r = run1("RECIP", x)
    want_s = np.array([F32(math.sqrt(float(v))) for v in x], F32)
    with np.errstate(over="ignore"):
        want_r = np.array([F32(1.0 / float(v)) for v in x], F32)
    assert np.array_equal(s.view(np.uint32), want_s.view(np.uint32))
    assert np.array_equal(r.view(np.uint32), want_r.view(np.uint32))
    assert run1("SQRT", [4.0, 0.0]).tolist() == [2.0, 0.0] and np.isnan(run1("SQRT", [-1.0])).all()
    inf = run1("RECIP", [0.0, -0.0])
    assert inf[0] == np.inf and inf[1] == -np.inf
    # planted slip: a reciprocal taken through f16 misses the pin
    with np.errstate(over="ignore", divide="ignore"):
        slip = (F32(1.0) / x.astype(np.float16).astype(F32)).astype(F32)
    assert not np.array_equal(slip.view(np.uint32), want_r.view(np.uint32))


def test_tanh_against_libm():
    x = np.concatenate([np.linspace(-12, 12, 4001, dtype=F32), np.array([1e-30, -1e-30, 20, -20, 88], F32)])
    got = run1("TANH", x)
    want = np.array([math.tanh(float(v)) for v in x])
    ulp = np.spacing(np.abs(want).astype(F32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2 * ulp)
    # planted slip: tanh taken in f16 misses the pin
    slip = np.tanh(x.astype(np.float16)).astype(F32)
    assert not np.all(np.abs(slip - want) <= 2 * ulp)
    assert np.array_equal(run1("TANH", -x), -got)  # odd
    assert run1("TANH", [20.0, -20.0, 0.0]).tolist() == [1.0, -1.0, 0.0]


def test_abs_clears_only_the_sign_and_copy_keeps_every_bit():
    bits = np.array([0x80000000, 0x00000000, 0xBF800000, 0x7F800000, 0xFF800000, 0xFFC00001, 0x00000001,
                     0x807FFFFF], np.uint32)
    x = bits.view(F32)
    a = run1("ABS", x).view(np.uint32)
    assert np.array_equal(a, bits & 0x7FFFFFFF)
    c = run1("COPY", x).view(np.uint32)
    assert np.array_equal(c, bits)


def _half_bits(v: float) -> int:
    try:
        return struct.unpack("<H", struct.pack("<e", v))[0]
    except OverflowError:  # struct refuses values that round past the largest half
        return 0x7C00 if v > 0 else 0xFC00


def test_round_f16_against_struct_half_packing():
    rng = np.random.default_rng(4)
    x = np.concatenate([
        rng.standard_normal(2000).astype(F32) * F32(1000),
        rng.standard_normal(500).astype(F32) * F32(1e-5),   # half subnormals
        np.array([65504, 65519.996, 65520, 70000, -65520, 2049, 2051, 1 + 2 ** -11, 1 + 3 * 2 ** -11, 2 ** -25,
                  3 * 2 ** -25, 0.0, -0.0], F32),            # largest finite, overflow edge, ties
    ])
    got = run1("ROUND_F16", x)
    want = np.array([_half_bits(float(v)) for v in x], np.uint16).view(np.float16).astype(F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert run1("ROUND_F16", [2049.0, 2051.0]).tolist() == [2048.0, 2052.0]  # ties to even
    # planted slip: truncation instead of round-to-nearest fails
    trunc = (x.view(np.uint32) & np.uint32(0xFFFFE000)).view(F32)
    small = np.abs(x) < 60000
    assert not np.array_equal(trunc[small], got[small])


def test_round_bf16_matches_the_pinned_rule():
    """ROUND_BF16 is ``ops.round_bf16``, pinned by the exact-rational rule
    in test_oracle_bf16.py; here the program path must call it unchanged."""
    x = sample(seed=5)
    assert np.array_equal(run1("ROUND_BF16", x).view(np.uint32), O.round_bf16(x).view(np.uint32))
    assert run1("ROUND_BF16", [1 + 2 ** -8, 1 + 3 * 2 ** -8]).tolist() == [1.0, 1 + 2 ** -6]


@pytest.mark.parametrize("code,fn", [("CMP_EQ", lambda a, b: a == b), ("CMP_NE", lambda a, b: a != b),
                                     ("CMP_LT", lambda a, b: a < b), ("CMP_LE", lambda a, b: a <= b),
                                     ("CMP_GT", lambda a, b: a > b), ("CMP_GE", lambda a, b: a >= b)])
def test_comparisons_give_zero_or_one(code, fn):
    a = [1.0, 2.0, 3.0, np.nan, -0.0]
    b = [2.0, 2.0, 1.0, 1.0, 0.0]
    want = [1.0 if fn(x, y) else 0.0 for x, y in zip(a, b)]
    assert run1(code, a, b).tolist() == want
