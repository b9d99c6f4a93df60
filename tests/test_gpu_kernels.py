"""Kernel-level parity of the HIP path against the NumPy oracle (GPU).

Every test calls libbghip through the bridge (C ABI) on seeded inputs and
compares with oracle/ops.py at sizes the oracle finishes in seconds:
bit-exact for casts / masks / copies, abs-or-rel 1e-4 for f32 and 2e-2 for
f16/bf16 MFMA paths (the tolerances BASELINE.json's north star states).
"""
from __future__ import annotations

import re

import numpy as np
import pytest

from oracle import ops as O

pytestmark = pytest.mark.gpu

TOL32 = 1e-4
TOL16 = 2e-2


@pytest.fixture(params=["auto", "256"])
def fa7_block(request, monkeypatch):
    """The attention kernel picks 256-query workgroups for grids of at least
    768 such blocks and 128-query ones below; the small test shapes land on
    the second, so each attention test also runs with the first forced."""
    if request.param != "auto":
        monkeypatch.setenv("BG_FA7_BLOCK", request.param)
    return request.param


def up(br, a, dtype=None):
    a = np.ascontiguousarray(a)
    return br.upload(a, a.shape, dtype or a.dtype.name)


def test_upload_materialize_roundtrip(bridge, rng):
    for dt in (np.float32, np.float16, np.uint8):
        a = (rng.standard_normal((7, 33)) * 10).astype(dt)
        h = up(bridge, a)
        back = bridge.to_numpy(h)
        assert back.dtype == a.dtype and np.array_equal(back.view(np.uint8), a.view(np.uint8))
        bridge.release(h)
        bridge.release(h)  # idempotent (realizer.ts:1036-1041)


def test_bridge_matmul_known_answer(bridge):
    # webgpu_real.test.ts:1558-1589
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    ha, hb = up(bridge, a), up(bridge, b)
    hc = bridge.matmul(ha, hb, 2, 2, 2, "float32")
    assert bridge.to_numpy(hc).ravel().tolist() == [19, 22, 43, 50]
    # reference.test.ts:42-50
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    b = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    hd = bridge.matmul(up(bridge, a), up(bridge, b), 2, 3, 2, "float32")
    assert bridge.to_numpy(hd).ravel().tolist() == [58, 64, 139, 154]


@pytest.mark.parametrize("m,k,n", [(17, 23, 19), (64, 784, 128), (64, 128, 10), (129, 65, 257), (256, 512, 384)])
@pytest.mark.parametrize("trans_b", [False, True])
def test_gemm_f32(bridge, rng, m, k, n, trans_b):
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k) if trans_b else (k, n)).astype(np.float32)
    h = bridge.matmul_ex(up(bridge, a), up(bridge, b), m=m, n=n, k=k, trans_b=trans_b, in_dtype="float32")
    y = bridge.to_numpy(h)
    ref = a @ (b.T if trans_b else b)
    truth = a.astype(np.float64) @ (b.T if trans_b else b).astype(np.float64)
    err_gpu = np.abs(y - truth)
    err_ref = np.abs(ref - truth)
    ok = O.within(y, ref, TOL32) | (err_gpu <= np.maximum(err_ref, TOL32))
    assert ok.all(), O.report(y, ref, TOL32)


@pytest.mark.parametrize("m,k,n", [(64, 784, 128), (64, 128, 10), (1, 129, 1), (100, 1001, 37), (512, 300, 512),
                                   (33, 4096, 65)])
@pytest.mark.parametrize("trans_b", [False, True])
@pytest.mark.parametrize("epi", ["plain", "bias_relu_residual", "f16_out"])
def test_gemm_f32_wide_k(bridge, rng, m, k, n, trans_b, epi):
    """Few output tiles and a long K take the one-launch wide-K kernel (32 x
    32 blocks, K split over 16 wavefronts, partials summed through LDS in
    wavefront order), with the full epilogue; against float64 truth within
    the rounding bound of a K-term f32 sum, and the same bits on a second
    run (fixed summation order)."""
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k) if trans_b else (k, n)).astype(np.float32)
    bias = rng.uniform(-1, 1, (n,)).astype(np.float32)
    res = rng.uniform(-1, 1, (m, n)).astype(np.float32)
    kw = dict(m=m, n=n, k=k, trans_b=trans_b, in_dtype="float32")
    if epi == "bias_relu_residual":
        kw.update(bias=up(bridge, bias), act=1, residual=up(bridge, res))
    if epi == "f16_out":
        kw.update(out_dtype="float16")
    ha, hb = up(bridge, a), up(bridge, b)
    bridge.set_launch_log(True)
    try:
        bridge.take_launch_log()
        h = bridge.matmul_ex(ha, hb, **kw)
        names = [r["kernel"] for r in bridge.take_launch_log()]
    finally:
        bridge.set_launch_log(False)
    assert [t for t in names if "gemm32_wide_k_kernel" in t] and len(names) == 1, names
    y = bridge.to_numpy(h).astype(np.float32)
    y2 = bridge.to_numpy(bridge.matmul_ex(ha, hb, **kw)).astype(np.float32)
    assert np.array_equal(y, y2)
    bm = (b.T if trans_b else b).astype(np.float64)
    truth = a.astype(np.float64) @ bm
    mass = np.abs(a.astype(np.float64)) @ np.abs(bm)
    if epi == "bias_relu_residual":
        truth = np.maximum(truth + bias, 0) + res
        mass = mass + np.abs(bias) + np.abs(res)
    bound = 2.0 * np.sqrt(k) * 2.0 ** -24 * mass + 1e-7
    if epi == "f16_out":
        bound = bound + np.abs(truth) * 2.0 ** -11  # one rounding to f16
    err = np.abs(y - truth)
    assert np.all(err <= bound), float(np.max(err / bound))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("m,k,n,trans_b", [(17, 24, 19, False), (128, 64, 128, True), (256, 256, 256, False),
                                           (300, 136, 200, True), (512, 1024, 768, True)])
def test_gemm_16bit_round_bias(bridge, rng, dtype, m, k, n, trans_b):
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k) if trans_b else (k, n)).astype(np.float32)
    bias = rng.uniform(-0.1, 0.1, (n,)).astype(np.float32)
    if dtype == "float16":
        a16, b16 = a.astype(np.float16), b.astype(np.float16)
        ha, hb = up(bridge, a16), up(bridge, b16)
        bm = b16.T if trans_b else b16
        ref = O.matmul(a16, np.ascontiguousarray(bm)).astype(np.float32) + bias
    else:
        a16, b16 = O.f32_to_bf16_bits(a), O.f32_to_bf16_bits(b)
        ha, hb = up(bridge, a16, "bfloat16"), up(bridge, b16, "bfloat16")
        bm = b16.T if trans_b else b16
        ref = O.bf16_bits_to_f32(O.matmul_bf16(a16, np.ascontiguousarray(bm))) + bias
    hbias = up(bridge, bias)
    h = bridge.matmul_ex(ha, hb, m=m, n=n, k=k, trans_b=trans_b, in_dtype=dtype, out_dtype="float32",
                         bias=hbias, round_out=True)
    y = bridge.to_numpy(h)
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


def test_gemm_batched_f16(bridge, rng):
    B, m, k, n = 6, 96, 64, 80
    a = rng.standard_normal((B, m, k)).astype(np.float16)
    b = rng.standard_normal((B, n, k)).astype(np.float16)
    h = bridge.matmul_ex(up(bridge, a), up(bridge, b), batch=B, m=m, n=n, k=k, trans_b=True,
                         in_dtype="float16", out_dtype="float16", round_out=True)
    y = bridge.to_numpy(h).astype(np.float32)
    ref = np.stack([O.matmul(a[i], np.ascontiguousarray(b[i].T)) for i in range(B)]).astype(np.float32)
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


@pytest.mark.parametrize("shape", [(4, 4096), (33, 100), (128, 4096), (3, 5, 64)])
def test_fused_c2_rowsum(bridge, rng, shape):
    a, b, c = (rng.standard_normal(shape).astype(np.float32) for _ in range(3))
    ops = [("MUL", -1, -2, 0), ("ADD", 0, -3, 0), ("IMM", 0, 0, 0), ("CMP_GT", 1, 2, 0),
           ("WHERE", 3, 1, 2), ("NEG", -1, 0, 0), ("MUL", 5, -1, 0), ("EXP", 6, 0, 0), ("MUL", 4, 7, 0)]
    hs = [up(bridge, t) for t in (a, b, c)]
    h = bridge.fused_ex(hs, ops, shape, "float32", imms=[0.0], reduce=1)
    y = bridge.to_numpy(h)
    ref = O.c2_chain(a.reshape(-1, shape[-1]), b.reshape(-1, shape[-1]), c.reshape(-1, shape[-1]))
    ref = ref.reshape(shape[:-1])
    assert O.within(y, ref, TOL32).all(), O.report(y, ref, TOL32)
    # Elementwise part alone (no reduction): within 1e-4 (exp is not bit-exact).
    h2 = bridge.fused_ex(hs, ops, shape, "float32", imms=[0.0])
    y2 = bridge.to_numpy(h2)
    ref2 = O.fused_program([a, b, c], ops, [0.0])
    assert O.within(y2, ref2, TOL32).all(), O.report(y2, ref2, TOL32)


# reduce_last across row widths: narrow rows take as few lanes per row as
# cover the row (1 ... 64), rows of 2048+ columns a whole workgroup, and
# fewer than 512 such rows are cut into column chunks whose partials a
# second kernel combines (16384+ columns, both vector widths, ragged last
# chunks).  The data carry a positive offset, so a dropped or repeated
# chunk moves a sum far outside the tolerance.
@pytest.mark.parametrize("rows,cols", [(4099, 1), (5000, 2), (5000, 3), (3001, 5), (4096, 16), (1000, 17),
                                       (777, 63), (1024, 64), (999, 65), (513, 100), (300, 255), (300, 256),
                                       (100, 1000), (64, 2047), (1, 2048), (1, 16384), (1, 1 << 20),
                                       (3, 100003), (7, 65536), (511, 8192), (512, 8192), (2, (1 << 21) + 4)])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_reduce_last_widths(bridge, rng, rows, cols, dtype):
    if dtype == "float16" and cols > 100003:
        pytest.skip("row sums beyond float16's range")
    x = (rng.uniform(-1, 1, (rows, cols)) + 0.25).astype(np.float32)
    if dtype == "float32":
        hx = up(bridge, x)
    else:
        x16 = _to16(x, dtype)
        hx = up(bridge, x16, dtype)
        x = _from16(x16, dtype)
    x64 = x.astype(np.float64)
    refs = {1: x64.sum(axis=1), 2: x64.max(axis=1), 3: x64.mean(axis=1), 4: x64.min(axis=1)}
    bound = 1e-5 * np.abs(x64).sum(axis=1) + 1e-6
    for op, ref in refs.items():
        h = bridge.reduce_last(hx, rows, cols, op)
        y = bridge.to_numpy(h)
        bridge.release(h)
        assert y.shape == (rows,)
        if dtype != "float32":
            y32, r32 = _from16(y, dtype), _from16(_to16(ref.astype(np.float32), dtype), dtype)
            assert O.within(y32, r32, TOL16).all(), (op, O.report(y32, r32, TOL16))
        elif op in (2, 4):
            assert np.array_equal(y, ref.astype(np.float32)), op
        else:
            err = np.abs(y.astype(np.float64) - ref)
            b = bound / cols if op == 3 else bound
            assert (err <= b).all(), (op, float(err.max()), float(b.min()))
    bridge.release(hx)


def _reduce_plan(shape, axis, op, dtype):
    ax = axis if isinstance(axis, list) else [axis]
    oshape = [d for i, d in enumerate(shape) if i not in ax]

    def st(i, code, ins, shp, arg=None):
        return {"step": i, "value_id": i, "op": code, "input_ids": ins, "shape": list(shp), "dtype": dtype,
                "arg": arg}
    return {"steps": [st(0, "BUFFER", [], shape),
                      st(1, "REDUCE", [0], oshape, {"op": op, "axis": axis, "keepdims": False})],
            "buffers": [], "root_id": 1, "materialization_boundary": "root", "peak_live_bytes": 0,
            "has_custom_ops": False}, tuple(ax)


# Plan REDUCE over a contiguous block of axes that is not trailing (a
# leading prefix: a bias gradient's sum over the batch) reads the input in
# place: 4, 16 or 64 column lanes per wavefront by width, vector and scalar
# columns, one row chunk (final result written directly) and many (partials
# combined by a second kernel), batches of such blocks (middle axes).  A
# leading prefix plus a trailing suffix is a row reduction into f32, then
# the prefix; other axis sets transpose first.
@pytest.mark.parametrize("shape,axis", [((4099, 768), 0), ((3, 5, 64), [0, 1]), ((1000, 3), 0), ((16, 17), 0),
                                        ((100000, 16), 0), ((7, 2050), 0), ((2, 3, 4, 40), [0, 1, 2]),
                                        ((20000, 64), 0), ((1, 4096), 0), ((300, 50), 0),
                                        ((4, 6, 40), 1), ((8, 300, 64), 1), ((5, 2000, 3), 1),
                                        ((64, 32, 100), [0, 2]), ((2, 3, 4, 40), [0, 3]),
                                        ((16, 8, 5, 7), [0, 1, 3]), ((6, 5, 4, 3), [0, 2]), ((3, 4, 5), [1, 2])])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_plan_reduce_leading_axes(bridge, rng, shape, axis, dtype):
    x = (rng.uniform(-1, 1, shape) + 0.25).astype(np.float32)
    if dtype == "float32":
        hx = up(bridge, x)
    else:
        x16 = _to16(x, dtype)
        hx = up(bridge, x16, dtype)
        x = _from16(x16, dtype)
    x64 = x.astype(np.float64)
    for op in ("sum", "mean", "max", "min"):
        plan, ax = _reduce_plan(shape, axis, op, dtype)
        h = bridge.run_tensor_plan_resident(plan, [{"value_id": 0, "handle": hx}], dtype)
        y = bridge.to_numpy(h)
        bridge.release(h)
        ref = getattr(x64, op)(axis=ax)
        n = int(np.prod([shape[a] for a in ax]))
        if dtype != "float32":
            y32, r32 = _from16(y, dtype).reshape(ref.shape), _from16(_to16(ref.astype(np.float32), dtype), dtype)
            assert O.within(y32, r32, TOL16).all(), (op, O.report(y32, r32, TOL16))
        elif op in ("max", "min"):
            assert np.array_equal(y.reshape(ref.shape), ref.astype(np.float32)), op
        else:
            bound = 1e-5 * np.abs(x64).sum(axis=ax) + 1e-6
            err = np.abs(y.reshape(ref.shape).astype(np.float64) - ref)
            b = bound / n if op == "mean" else bound
            assert (err <= b).all(), (op, float(err.max()), float(b.min()))
    bridge.release(hx)


# Broadcast operands index their leading dims by multiply-high division:
# odd and large leading dims (up to 2^22 rows), 1-3 leading dims, scalar and
# vector columns, column broadcasts, both with and without a reduction.
@pytest.mark.parametrize("shape,bshape", [((7, 13, 2999, 5), (7, 1, 2999, 1)), ((5000, 3, 17), (1, 3, 1)),
                                          ((4194305, 4), (4194305, 1)), ((3, 65537, 8), (3, 1, 8)),
                                          ((6, 7, 11, 12), (1, 7, 1, 12)), ((1000, 1001), (1, 1001))])
def test_fused_broadcast_index_math(bridge, rng, shape, bshape):
    x = rng.standard_normal(shape).astype(np.float32)
    b = rng.standard_normal(bshape).astype(np.float32)
    hx, hb = up(bridge, x), up(bridge, b)
    bst = [0 if d == 1 else int(np.prod(bshape[i + 1:])) for i, d in enumerate(bshape)]
    xst = [int(np.prod(shape[i + 1:])) for i in range(len(shape))]
    ops = [("ADD", -1, -2, 0)]
    y = bridge.to_numpy(bridge.fused_ex([hx, hb], ops, shape, "float32", in_strides=[xst, bst]))
    assert np.array_equal(y, x + b)
    r = bridge.to_numpy(bridge.fused_ex([hx, hb], ops, shape, "float32", in_strides=[xst, bst], reduce=2))
    assert np.array_equal(r, (x + b).max(axis=-1))


# An operand read transposed (innermost stride neither 0 nor 1) of 2^20+
# elements is first copied to row-major order; smaller ones are gathered in
# place.  Both must give NumPy's bits, with and without a row reduction.
@pytest.mark.parametrize("rows,cols,batch", [(1100, 1000, 0), (3, 7, 0), (700, 600, 3)])
def test_fused_transposed_operand(bridge, rng, rows, cols, batch):
    x = rng.standard_normal(((batch,) if batch else ()) + (rows, cols)).astype(np.float32)
    t = rng.standard_normal((cols, rows)).astype(np.float32)  # read as t.T
    hx, ht = up(bridge, x), up(bridge, t)
    shape = x.shape
    xst = [int(np.prod(shape[i + 1:])) for i in range(len(shape))]
    tst = ([0] if batch else []) + [1, rows]
    ops = [("MUL", -1, -2, 0), ("ADD", 0, -1, 0)]
    ref = x * t.T + x
    y = bridge.to_numpy(bridge.fused_ex([hx, ht], ops, shape, "float32", in_strides=[xst, tst]))
    assert np.array_equal(y, ref)
    r = bridge.to_numpy(bridge.fused_ex([hx, ht], ops, shape, "float32", in_strides=[xst, tst], reduce=2))
    assert np.array_equal(r, ref.max(axis=-1))


def test_fused_reference_opcodes_bit_exact(bridge, rng):
    # ADD/MUL/DIV/NEG are IEEE single ops: bit-exact against NumPy.
    a = rng.standard_normal((257, 31)).astype(np.float32)
    b = rng.standard_normal((257, 31)).astype(np.float32) + 3
    ops = [("ADD", -1, -2), ("MUL", 0, -1), ("DIV", 1, -2), ("NEG", 2, 0)]
    h = bridge.fused_elementwise([up(bridge, a), up(bridge, b)], ops, a.shape, "float32")
    y = bridge.to_numpy(h)
    ref = O.fused_program([a, b], ops)
    assert np.array_equal(y, ref)
    # closed form exp(a+b)/a (webgpu_real.test.ts:1431-1472), tolerance 1e-3 there.
    ops2 = [("ADD", -1, -2), ("EXP", 0, 0), ("DIV", 1, -1)]
    h2 = bridge.fused_elementwise([up(bridge, a), up(bridge, b)], ops2, a.shape, "float32")
    y2 = bridge.to_numpy(h2)
    assert O.within(y2, np.exp(a + b) / a, TOL32).all()


def test_fused_broadcast_where_cmp_bool(bridge, rng):
    x = rng.standard_normal((6, 40)).astype(np.float32)
    bias = rng.standard_normal((40,)).astype(np.float32)
    col = rng.standard_normal((6, 1)).astype(np.float32)
    hx, hb, hc = up(bridge, x), up(bridge, bias), up(bridge, col)
    ops = [("ADD", -1, -2, 0), ("CMP_LT", 0, -3, 0)]
    strides = [[40, 1], [0, 1], [1, 0]]
    h = bridge.fused_ex([hx, hb, hc], ops, (6, 40), "bool", in_strides=strides)
    y = bridge.to_numpy(h)
    assert y.dtype == np.bool_ and np.array_equal(y, (x + bias) < col)


@pytest.mark.parametrize("n", [1, 3, 4, 1000, 4099])
def test_cast_bit_exact(bridge, rng, n):
    x = (rng.standard_normal(n) * 300).astype(np.float32)
    x[: min(n, 3)] = [np.inf, -0.0, 65520.0][: min(n, 3)]
    h = up(bridge, x)
    h16 = bridge.cast(h, "float32", "float16", (n,))
    assert np.array_equal(bridge.to_numpy(h16).view(np.uint16), x.astype(np.float16).view(np.uint16))
    hb = bridge.cast(h, "float32", "bfloat16", (n,))
    assert np.array_equal(bridge.to_numpy(hb), O.f32_to_bf16_bits(x))
    hback = bridge.cast(h16, "float16", "float32", (n,))
    assert np.array_equal(bridge.to_numpy(hback), x.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("rows,cols", [(8, 768), (5, 100), (3, 3000), (64, 2048)])
def test_layer_norm(bridge, rng, rows, cols):
    x = rng.standard_normal((rows, cols)).astype(np.float32) * 3 + 1
    w = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    h = bridge.layer_norm(up(bridge, x), up(bridge, w), up(bridge, b), rows, cols, 1e-5)
    y = bridge.to_numpy(h)
    ref = O.layer_norm(x, w, b, 1e-5)
    assert O.within(y, ref, TOL32).all(), O.report(y, ref, TOL32)


def _to16(x, dtype):
    return x.astype(np.float16) if dtype == "float16" else O.f32_to_bf16_bits(x)


def _from16(y, dtype):
    return y.astype(np.float32) if dtype == "float16" else O.bf16_bits_to_f32(y)


# softmax_last: wavefront-per-row kernels below 512 columns (and unaligned
# up to 2048), the workgroup-per-row kernel for aligned rows of 512-32768
# (256 threads with 1, 2, 4 or 8 groups each, 1024 threads with 4 or 8), a
# 1024-thread register kernel for other rows up to 65536 (a GPT-2
# vocabulary row), the three-pass workgroup-per-row kernel past that.
@pytest.mark.parametrize("cols", [3, 64, 512, 768, 1000, 2048, 2052, 4096, 5000, 8192, 16384, 32768, 32772,
                                  50257, 2051, 16385, 65537])
@pytest.mark.parametrize("in_dtype,out_dtype", [("float32", "float32"), ("float16", "float16"),
                                                ("bfloat16", "float32"), ("float32", "float16")])
def test_softmax_last_widths(bridge, rng, cols, in_dtype, out_dtype):
    rows = 5
    x = (rng.standard_normal((rows, cols)) * 4).astype(np.float32)
    x[1] += 30.0  # a row far from zero: the max is subtracted before the exponential
    if in_dtype == "float32":
        hx = up(bridge, x)
    else:
        x16 = _to16(x, in_dtype)
        hx = up(bridge, x16, in_dtype)
        x = _from16(x16, in_dtype)
    y = bridge.to_numpy(bridge.softmax_last(hx, rows, cols, out_dtype=out_dtype))
    ref = O.softmax_lastaxis(x)
    if out_dtype == "float32":
        assert O.within(y, ref, TOL32).all(), O.report(y, ref, TOL32)
        assert np.allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=1e-4)
    else:
        y32, r32 = _from16(y, out_dtype), _from16(_to16(ref, out_dtype), out_dtype)
        assert O.within(y32, r32, TOL16).all(), O.report(y32, r32, TOL16)


# Widths for every register-group count of the vector path (1, 2, 3, 4, 8
# groups of 4 columns per lane), its widest row (2048), the workgroup-per-row
# kernel (4, 8, 16, 32 groups per thread, partial last groups), and widths
# that take the scalar kernels (not a multiple of 4, wider than 32768).
@pytest.mark.parametrize("cols", [4, 200, 512, 768, 1024, 1028, 2048, 2052, 766, 4096, 5000, 8192, 16380,
                                  32768, 2050, 32772])
@pytest.mark.parametrize("in_dtype,out_dtype", [("float32", "float32"), ("float16", "float16"),
                                                ("bfloat16", "bfloat16"), ("float32", "float16"),
                                                ("float16", "float32"), ("bfloat16", "float32")])
def test_layer_norm_dtypes(bridge, rng, cols, in_dtype, out_dtype):
    rows = 37
    x = (rng.standard_normal((rows, cols)) * 3 + 1).astype(np.float32)
    w = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32)
    if in_dtype == "float32":
        hx = up(bridge, x)
    else:
        x16 = _to16(x, in_dtype)
        hx = up(bridge, x16, in_dtype)
        x = _from16(x16, in_dtype)
    h = bridge.layer_norm(hx, up(bridge, w), up(bridge, b), rows, cols, 1e-5, out_dtype=out_dtype)
    ref = O.layer_norm(x, w, b, 1e-5)
    y = bridge.to_numpy(h)
    if out_dtype == "float32":
        assert O.within(y, ref, TOL32).all(), O.report(y, ref, TOL32)
    else:
        # One rounding of the f32 result to the output dtype (nearest even).
        r16 = _to16(ref, out_dtype)
        y32, r32 = _from16(y, out_dtype), _from16(r16, out_dtype)
        assert O.within(y32, r32, TOL16).all(), O.report(y32, r32, TOL16)
        # Away from zero (where the f32 result's absolute error of ~1e-6 is
        # many 16-bit ulps) most elements round identically, and none lands
        # more than one code away.
        big = np.abs(r32) >= 0.25
        ulp = np.abs(y.view(np.uint16).astype(np.int32) - r16.view(np.uint16).astype(np.int32))[big]
        assert (ulp <= 1).all() and (ulp == 0).mean() > 0.99


def test_copy_strided_permute(bridge, rng):
    x = rng.standard_normal((2, 5, 3, 4)).astype(np.float32)
    h = up(bridge, x)
    perm = (0, 2, 1, 3)
    shape = tuple(x.shape[p] for p in perm)
    st = np.array(x.strides) // 4
    strides = tuple(int(st[p]) for p in perm)
    y = bridge.to_numpy(bridge.copy_strided(h, 0, shape, strides))
    assert np.array_equal(y, np.transpose(x, perm))


# Strided copies by path: rows contiguous in the source copied in 16-byte
# pieces (head split/merge permutes, slices of rows), tiled transposes (the
# source's contiguous dim moved outward, with 0-2 batch dims, ragged tiles,
# 1/2/4/8-byte elements, a broadcast innermost dim), and the generic
# element kernel (negative strides, odd row bytes, 5+ collapsed dims).
# Each copy is checked bit-exactly against NumPy's view of the same bytes.
COPY_CASES = [
    ((2, 128, 12, 64), (0, 2, 1, 3), None),   # [B,S,H,D] -> [B,H,S,D]
    ((2, 12, 128, 64), (0, 2, 1, 3), None),   # and back
    ((4096, 768), (1, 0), None),               # 2-D transpose
    ((3, 100, 70), (0, 2, 1), None),           # batched, ragged tiles
    ((5, 7, 9, 11), (3, 1, 0, 2), None),       # rank 4, two batch dims
    ((8, 64, 56, 56), (0, 2, 3, 1), None),     # NCHW -> NHWC
    ((8, 56, 56, 64), (0, 3, 1, 2), None),     # NHWC -> NCHW
    ((2, 3, 4, 5, 6, 7), (5, 0, 4, 1, 3, 2), None),  # rank 6: generic kernel
    ((64, 48), None, "slice_rows"),            # rows of a slice
    ((33, 47), None, "reverse"),               # negative stride
    ((40, 30), None, "broadcast_inner"),       # innermost stride 0
    ((17, 13), None, "every_other"),           # innermost stride 2, no stride-1 dim
]


def _copy_case(x, perm, kind):
    es = x.itemsize
    st = [v // es for v in x.strides]
    if perm is not None:
        return 0, [x.shape[p] for p in perm], [st[p] for p in perm], np.transpose(x, perm)
    if kind == "slice_rows":  # rows 5..36 of every 4th column block of 16
        return 5 * st[0] + 16, [32, 16], [st[0], 1], x[5:37, 16:32]
    if kind == "reverse":
        return (x.shape[0] - 1) * st[0], [x.shape[0], x.shape[1]], [-st[0], 1], x[::-1]
    if kind == "broadcast_inner":
        return 0, [x.shape[0], x.shape[1], 9], [st[0], 1, 0], np.broadcast_to(x[:, :, None], x.shape + (9,))
    return 0, [x.shape[0], (x.shape[1] + 1) // 2], [st[0], 2], x[:, ::2]


@pytest.mark.parametrize("shape,perm,kind", COPY_CASES)
@pytest.mark.parametrize("dtype", ["float32", "float16", "uint8", "int64"])
def test_copy_strided_paths(bridge, rng, shape, perm, kind, dtype):
    if dtype == "int64":
        x = rng.integers(-2**62, 2**62, size=shape, dtype=np.int64)
    else:
        x = (rng.standard_normal(shape) * 100).astype(dtype)
    h = up(bridge, x)
    off, shp, strides, ref = _copy_case(x, perm, kind)
    y = bridge.to_numpy(bridge.copy_strided(h, off, shp, strides))
    assert y.shape == ref.shape and np.array_equal(y.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8))


@pytest.mark.parametrize("b,h,s,causal", [(1, 2, 4, False), (2, 3, 128, True), (1, 2, 200, True),
                                          (2, 2, 256, False), (1, 1, 1000, True)])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("round_scores", [False, True])
def test_attention_mfma(bridge, rng, fa7_block, b, h, s, causal, dtype, round_scores):
    d = 64
    q, k, v = (rng.standard_normal((b, h, s, d)).astype(np.float32) for _ in range(3))
    scale = 1.0 / np.sqrt(d)
    if dtype == "float16":
        q16, k16, v16 = (t.astype(np.float16) for t in (q, k, v))
        hq, hk, hv = up(bridge, q16), up(bridge, k16), up(bridge, v16)
        ref = O.sdpa_amp(q16, k16, v16, scale, causal).astype(np.float32)
    else:
        q16, k16, v16 = (O.f32_to_bf16_bits(t) for t in (q, k, v))
        hq, hk, hv = (up(bridge, t, "bfloat16") for t in (q16, k16, v16))
        ref = O.bf16_bits_to_f32(O.sdpa_bf16(q16, k16, v16, scale, causal))
    ho = bridge.attention_ex(hq, hk, hv, batch=b, heads=h, sq=s, sk=s, d=d, scale=scale, causal=causal,
                             in_dtype=dtype, round_scores=round_scores)
    y = bridge.to_numpy(ho)
    y = y.astype(np.float32) if dtype == "float16" else O.bf16_bits_to_f32(y)
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


@pytest.mark.parametrize("d", [8, 16, 32, 48])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("round_scores", [False, True])
def test_attention_mfma_small_head_dims(bridge, rng, fa7_block, d, causal, dtype, round_scores):
    """Head dims below 64 (multiples of 8, the reference admits 1..64) run
    the fast MFMA kernel with the missing 16-byte chunks of Q, K and V read
    as zeros and only the first d output columns stored."""
    b, h, sq, sk = 2, 3, 200, 200
    print(f"[case] small head dim d={d} causal={causal} {dtype} round_scores={round_scores}", flush=True)
    q, k, v = (rng.standard_normal((b, h, s_, d)).astype(np.float32) for s_ in (sq, sk, sk))
    scale = 1.0 / np.sqrt(d)
    if dtype == "float16":
        ts = [t.astype(np.float16) for t in (q, k, v)]
        hs = [up(bridge, t) for t in ts]
        ref = O.sdpa_amp(*ts, scale, causal).astype(np.float32)
    else:
        ts = [O.f32_to_bf16_bits(t) for t in (q, k, v)]
        hs = [up(bridge, t, "bfloat16") for t in ts]
        ref = O.bf16_bits_to_f32(O.sdpa_bf16(*ts, scale, causal))
    bridge.set_launch_log(True)
    try:
        bridge.take_launch_log()
        ho = bridge.attention_ex(*hs, batch=b, heads=h, sq=sq, sk=sk, d=d, scale=scale, causal=causal,
                                 in_dtype=dtype, round_scores=round_scores)
        names = [r["kernel"] for r in bridge.take_launch_log()]
    finally:
        bridge.set_launch_log(False)
    assert any("fa7_fwd_kernel" in t or "fa8_fwd_kernel" in t for t in names), names
    y = bridge.to_numpy(ho)
    y = y.astype(np.float32) if dtype == "float16" else O.bf16_bits_to_f32(y)
    assert y.shape == (b, h, sq, d)
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


def test_attention_small_head_dim_dominant_key(bridge, rng):
    """d = 32 with a key that beats the first 32 by far more than 2^16: the
    exact recompute pass also reads and writes only the first d columns."""
    b, h, s, d = 1, 1, 300, 32
    q = rng.standard_normal((b, h, s, d)).astype(np.float32)
    k = (0.25 * rng.standard_normal((b, h, s, d))).astype(np.float32)
    v = rng.standard_normal((b, h, s, d)).astype(np.float32)
    u = np.ones(d, np.float32) / np.sqrt(d / 16.0)
    q[0, 0] += 4.0 * u
    k[0, 0, 100] = 4.0 * u
    ts = [t.astype(np.float16) for t in (q, k, v)]
    ho = bridge.attention_ex(*[up(bridge, t) for t in ts], batch=b, heads=h, sq=s, sk=s, d=d, scale=0.125,
                             causal=True, in_dtype="float16")
    y = bridge.to_numpy(ho).astype(np.float32)
    ref = O.sdpa_amp(*ts, 0.125, True).astype(np.float32)
    assert np.isfinite(y).all()
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


def test_attention_generic_f32_legacy(bridge, rng):
    b, h, s, d = 1, 2, 33, 16
    q, k, v = (rng.standard_normal((b, h, s, d)).astype(np.float32) for _ in range(3))
    mask = np.where(rng.random((s, s)) < 0.2, -1e9, 0).astype(np.float32)
    ho = bridge.flash_attention(up(bridge, q), up(bridge, k), up(bridge, v), up(bridge, mask),
                                b, h, s, s, d, 0.25, "float32")
    y = bridge.to_numpy(ho)
    ref = O.attention_online_f32(q, k, v, 0.25, mask)
    assert O.within(y, ref, TOL32).all(), O.report(y, ref, TOL32)


def test_alive_handles_and_snapshot(bridge, rng):
    before = bridge.aliveHandleCount()
    h = up(bridge, rng.standard_normal(10).astype(np.float32))
    assert bridge.aliveHandleCount() == before + 1
    snap = bridge.resourceSnapshot()
    assert snap["currentOwnedGpuBytes"] >= 40
    bridge.release(h)
    assert bridge.aliveHandleCount() == before


@pytest.mark.parametrize("m,k,n", [(300, 136, 200), (256, 256, 256), (129, 72, 77), (70, 100, 33), (1024, 768, 512)])
@pytest.mark.parametrize("act", ["relu", "gelu"])
@pytest.mark.parametrize("out_dtype", ["float32", "float16"])
def test_gemm_amp_epilogue_act(bridge, rng, m, k, n, act, out_dtype):
    """AMP linear + activation: f16(x) @ f16(W).T -> f16 round -> + b (f32) ->
    relu / tanh-GELU in f32 -> out dtype.  K = 136 exercises the K-tail loads,
    K = 100 the element-load fallback, 129 x 77 the edge tiles."""
    x = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    w = rng.uniform(-1, 1, (n, k)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, (n,)).astype(np.float32)
    x16, w16 = x.astype(np.float16), w.astype(np.float16)
    h = bridge.matmul_ex(up(bridge, x16), up(bridge, w16), m=m, n=n, k=k, trans_b=True, in_dtype="float16",
                         out_dtype=out_dtype, bias=up(bridge, b), round_out=True,
                         act={"relu": 1, "gelu": 2}[act])
    y = bridge.to_numpy(h).astype(np.float32)
    z = O.matmul(x16, np.ascontiguousarray(w16.T)).astype(np.float32) + b
    ref = np.where(z > 0, z, np.float32(0)) if act == "relu" else O.gelu_tanh_f32(z)
    if out_dtype == "float16":
        ref = ref.astype(np.float16).astype(np.float32)
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


def _gelu_edge_values():
    """Every f32 on both sides of the reference GELU's overflow edge
    (|u| = 88.72283935546875 at |x| ~ 12.99825) and the special values."""
    lo = np.float32(12.99822)
    edge = [lo]
    for _ in range(60):
        edge.append(np.nextafter(edge[-1], np.float32(np.inf), dtype=np.float32))
    edge = np.array(edge, np.float32)
    special = np.array([0.0, -0.0, 1.0, -1.0, 3.0, -3.0, 1e-4, -1e-4, 5.5, -5.5, 40.0, -40.0, 60.0, -60.0,
                        1e20, -1e20, np.inf, -np.inf, np.nan], np.float32)
    return np.concatenate([edge, -edge, special])


@pytest.mark.parametrize("in_dtype", ["float16", "float32"])
def test_gemm_gelu_overflow_edge(bridge, in_dtype):
    """tanh-GELU's NaN set is the reference's: NaN exactly where one of its
    f32 exponentials overflows, finite on the last f32 before.  z = 0 @ 0 + b
    puts the bias values through the epilogue unchanged (f16: GELU in the
    GEMM epilogue; f32: the separate GELU pass)."""
    b = _gelu_edge_values()
    n, m, k = b.size, 3, 8
    ref = O.gelu_tanh_f32(b)
    assert np.isnan(ref).any() and np.isfinite(ref).any()
    dt = np.float16 if in_dtype == "float16" else np.float32
    z = np.zeros((m, k), dt)
    w = np.zeros((n, k), dt)
    h = bridge.matmul_ex(up(bridge, z), up(bridge, w), m=m, n=n, k=k, trans_b=True, in_dtype=in_dtype,
                         out_dtype="float32", bias=up(bridge, b), round_out=in_dtype == "float16", act=2)
    y = bridge.to_numpy(h)
    for row in y:
        assert np.array_equal(np.isnan(row), np.isnan(ref)), (b[np.isnan(row) != np.isnan(ref)])
        assert O.within(row, ref, TOL32).all(), O.report(row, ref, TOL32)


@pytest.mark.parametrize("m,k,n", [(64, 784, 128), (64, 128, 10), (33, 17, 65)])
def test_gemm_f32_bias_relu_gelu(bridge, rng, m, k, n):
    """f32 linear layer epilogues (C1's Linear + ReLU), rel 1e-4."""
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = rng.uniform(-1 / np.sqrt(k), 1 / np.sqrt(k), (n, k)).astype(np.float32)
    b = rng.uniform(-1 / np.sqrt(k), 1 / np.sqrt(k), (n,)).astype(np.float32)
    hx, hw, hb = up(bridge, x), up(bridge, w), up(bridge, b)
    z = x.astype(np.float64) @ w.T.astype(np.float64) + b
    for act, f in ((1, lambda t: np.maximum(t, 0)), (2, lambda t: O.gelu_tanh_f32(t.astype(np.float32)))):
        y = bridge.to_numpy(bridge.matmul_ex(hx, hw, m=m, n=n, k=k, trans_b=True, bias=hb, act=act))
        ref = f(z)
        assert O.within(y, ref, TOL32).all(), O.report(y, ref, TOL32)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("round_scores", [False, True])
def test_attention_long_sequence(bridge, rng, fa7_block, dtype, causal, round_scores):
    """Two full S=2048 heads (the C4 shape per head) and a ragged 1100."""
    for (b, h, s) in ((1, 2, 2048), (1, 1, 1100)):
        d = 64
        q, k, v = (rng.standard_normal((b, h, s, d)).astype(np.float32) for _ in range(3))
        scale = 0.125
        if dtype == "float16":
            q16, k16, v16 = (t.astype(np.float16) for t in (q, k, v))
            hq, hk, hv = up(bridge, q16), up(bridge, k16), up(bridge, v16)
            ref = O.sdpa_amp(q16, k16, v16, scale, causal).astype(np.float32)
        else:
            q16, k16, v16 = (O.f32_to_bf16_bits(t) for t in (q, k, v))
            hq, hk, hv = (up(bridge, t, "bfloat16") for t in (q16, k16, v16))
            ref = O.bf16_bits_to_f32(O.sdpa_bf16(q16, k16, v16, scale, causal))
        ho = bridge.attention_ex(hq, hk, hv, batch=b, heads=h, sq=s, sk=s, d=d, scale=scale, causal=causal,
                                 in_dtype=dtype, round_scores=round_scores)
        y = bridge.to_numpy(ho)
        y = y.astype(np.float32) if dtype == "float16" else O.bf16_bits_to_f32(y)
        assert O.within(y, ref, TOL16).all(), (b, h, s, O.report(y, ref, TOL16))


def test_attention_rectangular_noncausal(bridge, rng, fa7_block):
    b, h, sq, sk, d = 2, 3, 100, 300, 64
    q = rng.standard_normal((b, h, sq, d)).astype(np.float16)
    k = rng.standard_normal((b, h, sk, d)).astype(np.float16)
    v = rng.standard_normal((b, h, sk, d)).astype(np.float16)
    ho = bridge.attention_ex(up(bridge, q), up(bridge, k), up(bridge, v), batch=b, heads=h, sq=sq, sk=sk, d=d,
                             scale=0.125, causal=False, in_dtype="float16", round_scores=True)
    y = bridge.to_numpy(ho).astype(np.float32)
    ref = O.sdpa_amp(q, k, v, 0.125, False).astype(np.float32)
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


@pytest.mark.parametrize("sq,sk", [(300, 100), (100, 300), (600, 130), (257, 257), (64, 2048)])
@pytest.mark.parametrize("round_scores", [False, True])
def test_attention_rectangular_causal(bridge, rng, fa7_block, sq, sk, round_scores):
    """Causal with Sq != Sk: the reference mask triu(ones(Sq, Sk), k=1) is
    top-left aligned (key j visible to query i iff j <= i), so queries past Sk
    see every key.  (600, 130) puts whole query blocks past the last key."""
    b, h, d = 1, 2, 64
    q = rng.standard_normal((b, h, sq, d)).astype(np.float16)
    k = rng.standard_normal((b, h, sk, d)).astype(np.float16)
    v = rng.standard_normal((b, h, sk, d)).astype(np.float16)
    ho = bridge.attention_ex(up(bridge, q), up(bridge, k), up(bridge, v), batch=b, heads=h, sq=sq, sk=sk, d=d,
                             scale=0.125, causal=True, in_dtype="float16", round_scores=round_scores)
    y = bridge.to_numpy(ho).astype(np.float32)
    ref = O.sdpa_amp(q, k, v, 0.125, True).astype(np.float32)
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("round_scores", [False, True])
def test_attention_late_dominant_key(bridge, rng, fa7_block, causal, dtype, round_scores):
    """Head 0 holds a key (index 100) whose score beats every key of the first
    32 by far more than 16 (log2 units): a reference max taken from the first
    keys must move, or P overflows the 16-bit range.  Head 1 is ordinary
    random data in the same launch, so blocks that need no recompute must be
    left as they are."""
    b, h, s, d = 1, 2, 300, 64
    q = rng.standard_normal((b, h, s, d)).astype(np.float32)
    k = (0.25 * rng.standard_normal((b, h, s, d))).astype(np.float32)
    v = rng.standard_normal((b, h, s, d)).astype(np.float32)
    u = np.ones(d, np.float32) / 2.0
    q[0, 0] += 4.0 * u   # every query of head 0 leans towards u
    k[0, 0, 100] = 4.0 * u  # q.k ~ 256 for key 100: 46 log2 units above the rest
    scale = 0.125
    if dtype == "float16":
        q16, k16, v16 = (t.astype(np.float16) for t in (q, k, v))
        hq, hk, hv = up(bridge, q16), up(bridge, k16), up(bridge, v16)
        ref = O.sdpa_amp(q16, k16, v16, scale, causal).astype(np.float32)
    else:
        q16, k16, v16 = (O.f32_to_bf16_bits(t) for t in (q, k, v))
        hq, hk, hv = (up(bridge, t, "bfloat16") for t in (q16, k16, v16))
        ref = O.bf16_bits_to_f32(O.sdpa_bf16(q16, k16, v16, scale, causal))
    ho = bridge.attention_ex(hq, hk, hv, batch=b, heads=h, sq=s, sk=s, d=d, scale=scale, causal=causal,
                             in_dtype=dtype, round_scores=round_scores)
    y = bridge.to_numpy(ho)
    y = y.astype(np.float32) if dtype == "float16" else O.bf16_bits_to_f32(y)
    assert np.isfinite(y).all()
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_attention_dominant_key_long_sequence(bridge, rng, fa7_block, dtype):
    """C4-length heads where keys 1500 and 40 dominate every earlier key by
    far more than 2^16: the fast kernel's reference max (from each query's
    first 32 keys) overflows P for the queries that see them, and those
    wavefronts must be recomputed exactly; head 1 is plain random data."""
    b, h, s, d = 1, 2, 2048, 64
    q = rng.standard_normal((b, h, s, d)).astype(np.float32)
    k = (0.25 * rng.standard_normal((b, h, s, d))).astype(np.float32)
    v = rng.standard_normal((b, h, s, d)).astype(np.float32)
    u = np.ones(d, np.float32) / 2.0
    q[0, 0] += 4.0 * u
    k[0, 0, 1500] = 4.0 * u
    k[0, 0, 40] = 3.0 * u
    if dtype == "float16":
        ts = [t.astype(np.float16) for t in (q, k, v)]
        hs = [up(bridge, t) for t in ts]
        ref = O.sdpa_amp(*ts, 0.125, True).astype(np.float32)
    else:
        ts = [O.f32_to_bf16_bits(t) for t in (q, k, v)]
        hs = [up(bridge, t, "bfloat16") for t in ts]
        ref = O.bf16_bits_to_f32(O.sdpa_bf16(*ts, 0.125, True))
    ho = bridge.attention_ex(*hs, batch=b, heads=h, sq=s, sk=s, d=d, scale=0.125, causal=True,
                             in_dtype=dtype, round_scores=False)
    y = bridge.to_numpy(ho)
    y = y.astype(np.float32) if dtype == "float16" else O.bf16_bits_to_f32(y)
    assert np.isfinite(y).all()
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


def test_attention_reordered_grid_every_head(bridge, rng):
    """128-query workgroups of a grid that fills the resident slots take
    their (head, query block) from a heavy-first order whose rounds of 32 per
    XCD alternate direction.  4 x 16 heads x 8 blocks = 512 workgroups walk a
    reversed round; every head and query block must come out once and right."""
    b, h, s, d = 4, 16, 1024, 64
    q, k, v = (rng.standard_normal((b, h, s, d)).astype(np.float16) for _ in range(3))
    ho = bridge.attention_ex(up(bridge, q), up(bridge, k), up(bridge, v), batch=b, heads=h, sq=s, sk=s, d=d,
                             scale=0.125, causal=True, in_dtype="float16", round_scores=False)
    y = bridge.to_numpy(ho).astype(np.float32)
    ref = O.sdpa_amp(q, k, v, 0.125, True).astype(np.float32)
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


@pytest.mark.parametrize("round_scores", [False, True])
def test_attention_strided_fused_qkv_views(bridge, rng, round_scores):
    """Q/K/V as views into one fused QKV projection [B, S, 3, H, D] (the GPT-2
    block layout): head-split without a copy, output [B, S, H, D]."""
    B, S, H, D = 2, 192, 3, 64
    qkv = rng.standard_normal((B, S, 3, H, D)).astype(np.float16)
    h = up(bridge, qkv)
    sb, ss, sh = S * 3 * H * D, 3 * H * D, D
    views = [(i * H * D, sb, sh, ss) for i in range(3)]
    ho = bridge.attention_ex(h, h, h, batch=B, heads=H, sq=S, sk=S, d=D, scale=0.125, causal=True,
                             in_dtype="float16", round_scores=round_scores, q_view=views[0], k_view=views[1],
                             v_view=views[2], o_strides=(S * H * D, D, H * D))
    y = bridge.to_numpy(ho).reshape(B, S, H, D).astype(np.float32)
    q, k, v = (np.ascontiguousarray(qkv[:, :, i].transpose(0, 2, 1, 3)) for i in range(3))
    ref = O.sdpa_amp(q, k, v, 0.125, True).astype(np.float32).transpose(0, 2, 1, 3)
    assert O.within(y, ref, TOL16).all(), O.report(y, ref, TOL16)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_attention_round_scores_is_honoured(bridge, dtype):
    """q.k = 2049 and 2048 (f16; 257 and 256 for bf16) round to the same
    16-bit score, so with round_scores the two keys get P = 1/2 each and the
    output is v0/2 + v1/2 = 0 exactly, as the reference graph (and the
    oracle) computes; without the rounding the second key wins slightly and
    the output is not 0."""
    d, sk = 64, 2
    big = 1024.0 if dtype == "float16" else 128.0
    q = np.zeros((1, 1, 1, d), np.float32)
    q[..., :2] = 1.0
    k = np.zeros((1, 1, sk, d), np.float32)
    k[0, 0, 0, :2] = (big, big)
    k[0, 0, 1, :2] = (big + 1, big)
    v = np.zeros((1, 1, sk, d), np.float32)
    v[0, 0, 0], v[0, 0, 1] = 1.0, -1.0
    scale = 1.0 / (2 * big)
    if dtype == "float16":
        ts = [t.astype(np.float16) for t in (q, k, v)]
        ref = O.sdpa_amp(*ts, scale, False).astype(np.float32)
        hs = [up(bridge, t) for t in ts]
    else:
        ts = [O.f32_to_bf16_bits(t) for t in (q, k, v)]
        ref = O.bf16_bits_to_f32(O.sdpa_bf16(*ts, scale, False))
        hs = [up(bridge, t, "bfloat16") for t in ts]
    assert np.all(ref == 0.0)
    out, names = {}, {}
    bridge.set_launch_log(True)
    try:
        bridge.take_launch_log()
        for rs in (True, False):
            ho = bridge.attention_ex(*hs, batch=1, heads=1, sq=1, sk=sk, d=d, scale=scale, causal=False,
                                     in_dtype=dtype, out_dtype="float32", round_scores=rs)
            out[rs] = bridge.to_numpy(ho)
            names[rs] = [r["kernel"] for r in bridge.take_launch_log()]
    finally:
        bridge.set_launch_log(False)
    # Both forms run the fast kernel; its fifth template argument is ROUND_S
    # (<BF16, CAUSAL, NW, RING, ROUND_S[, queries per wavefront / 16]>).
    def fa7(ts, rs):
        want = "1" if rs else "0"
        for t in ts:
            m = (re.search(r"fa[78]_fwd_kernelILb[01]ELb[01]ELi\d+ELi\d+ELb([01])E", t)  # mangled
                 or re.search(r"fa[78]_fwd_kernel<(?:true|false), (?:true|false), \d+, \d+, (true|false)[,>]", t))
            if m and {"true": "1", "false": "0"}.get(m.group(1), m.group(1)) == want:
                return True
        return False
    assert fa7(names[True], True), names[True]
    assert fa7(names[False], False), names[False]
    assert np.all(out[True] == 0.0), out[True][..., :4]
    assert np.all(out[False] < 0.0), out[False][..., :4]
    assert O.within(out[False], ref, TOL16).all()


def test_attention_large_scale_routes_around_prescaled_q(bridge, rng):
    """scale * log2(e) > 1 would let Q' = Q * scale * log2(e) overflow f16 in
    the pre-scaling kernel; such calls must still match the oracle."""
    b, h, s, d = 1, 2, 96, 64
    q = (rng.standard_normal((b, h, s, d)) * 2000).astype(np.float16)
    k = (rng.standard_normal((b, h, s, d)) * 1e-3).astype(np.float16)
    v = rng.standard_normal((b, h, s, d)).astype(np.float16)
    hq, hk, hv = up(bridge, q), up(bridge, k), up(bridge, v)
    # S rounded as the reference graph does -> the oracle; S kept in f32 ->
    # float64 attention over the same f16 inputs (at this scale the f16
    # rounding of S moves the softmax by more than the tolerance).
    refs = {True: O.sdpa_amp(q, k, v, 40.0, True).astype(np.float32),
            False: O.attention_f64(q, k, v, 40.0, causal=True)}
    for rs, ref in refs.items():
        ho = bridge.attention_ex(hq, hk, hv, batch=b, heads=h, sq=s, sk=s, d=d, scale=40.0, causal=True,
                                 in_dtype="float16", round_scores=rs)
        y = bridge.to_numpy(ho).astype(np.float32)
        assert np.isfinite(y).all()
        assert O.within(y, ref, TOL16).all(), (rs, O.report(y, ref, TOL16))


@pytest.mark.parametrize("m,k,n,act,residual", [(8000, 768, 768, 0, True), (4100, 768, 2304, 0, False),
                                                (8192, 136, 3072, 2, False), (2000, 3072, 768, 1, True)])
def test_gemm_128x192_tiles_ragged(bridge, rng, monkeypatch, m, k, n, act, residual):
    """Widths that are multiples of 192 take 128x192 tiles (an 8-wavefront
    4 x 2 grid); ragged M and a K tail must give the same bits as another
    tile shape's kernel (both accumulate each 16-wide k chunk in order) and
    match the oracle's autocast linear."""
    x = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, (n,)).astype(np.float32)
    x16, w16 = x.astype(np.float16), w.astype(np.float16)
    hx, hw, hb = up(bridge, x16), up(bridge, w16), up(bridge, b)
    r = rng.standard_normal((m, n)).astype(np.float32) if residual else None
    kw = dict(m=m, n=n, k=k, trans_b=True, in_dtype="float16", out_dtype="float32", bias=hb, round_out=True,
              act=act, residual=up(bridge, r) if residual else None)
    y = bridge.to_numpy(bridge.matmul_ex(hx, hw, **kw))
    monkeypatch.setenv("BG_GEMM_TILE", "128x128x64s2")
    y2 = bridge.to_numpy(bridge.matmul_ex(hx, hw, **kw))
    assert np.array_equal(y.view(np.uint8), y2.view(np.uint8))
    z = O.matmul(x16, np.ascontiguousarray(w16.T)).astype(np.float32) + b
    if act == 1:
        z = np.maximum(z, np.float32(0))
    elif act == 2:
        z = O.gelu_tanh_f32(z)
    if residual:
        z = z + r
    assert O.within(y, z, TOL16).all(), O.report(y, z, TOL16)


@pytest.mark.parametrize("m,k,n,act,residual,trans_b", [
    (1, 4096, 4096, 0, False, True), (17, 1024, 300, 1, True, True), (32, 4096, 4096, 0, False, False),
    (33, 768, 2304, 2, False, True), (64, 3072, 768, 0, True, True), (64, 512, 50, 1, False, True),
    (5, 4104, 130, 2, True, False), (48, 520, 4000, 0, False, True), (100, 1024, 2304, 1, True, True),
    (128, 4096, 4096, 0, False, False), (65, 768, 3000, 2, True, True), (256, 1024, 4000, 1, True, True),
    (200, 2048, 2500, 0, False, False), (450, 2200, 1024, 2, True, True)])
@pytest.mark.parametrize("dtype,out_dtype", [("float16", "float32"), ("float16", "float16"),
                                             ("bfloat16", "bfloat16"), ("float32", "float32")])
def test_gemm_skinny_split_k(bridge, rng, monkeypatch, m, k, n, act, residual, trans_b, dtype, out_dtype):
    """At most 64 rows (f32: 512, in 64-row blocks) with K >= 512 and fewer
    128-column tiles than CUs (f32 also with B stored [K][N]): K split over
    workgroups (f32 partials summed in split order by a second
    kernel, or one split), M of one or two 32-row MFMA blocks, ragged N,
    a K that is a multiple of 8 but not 16, every epilogue stage.  Checked
    against the oracle's autocast linear and against the tiled kernel."""
    x = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, (n,)).astype(np.float32)
    if dtype == "float32":
        hx = up(bridge, x)
        hw = up(bridge, w if trans_b else np.ascontiguousarray(w.T))
        z = (x.astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32)
    elif dtype == "float16":
        x16, w16 = x.astype(np.float16), w.astype(np.float16)
        hx = up(bridge, x16)
        wm = w16 if trans_b else np.ascontiguousarray(w16.T)
        hw = up(bridge, wm)
        z = O.matmul(x16, np.ascontiguousarray(w16.T)).astype(np.float32)
    else:
        x16, w16 = O.f32_to_bf16_bits(x), O.f32_to_bf16_bits(w)
        hx = up(bridge, x16, "bfloat16")
        wm = w16 if trans_b else np.ascontiguousarray(w16.T)
        hw = up(bridge, wm, "bfloat16")
        z = O.bf16_bits_to_f32(O.matmul_bf16(x16, np.ascontiguousarray(w16.T)))
    z = z + b
    if act == 1:
        z = np.maximum(z, np.float32(0))
    elif act == 2:
        z = O.gelu_tanh_f32(z)
    r = rng.standard_normal((m, n)).astype(np.float32) if residual else None
    if residual:
        z = z + r
    kw = dict(m=m, n=n, k=k, trans_b=trans_b, in_dtype=dtype, out_dtype=out_dtype, bias=up(bridge, b),
              round_out=dtype != "float32", act=act, residual=up(bridge, r) if residual else None)
    y = bridge.to_numpy(bridge.matmul_ex(hx, hw, **kw))
    monkeypatch.setenv("BG_GEMM_SKINNY", "0")
    y2 = bridge.to_numpy(bridge.matmul_ex(hx, hw, **kw))
    if out_dtype == "float32":
        y, y2 = y.astype(np.float32), y2.astype(np.float32)
    elif out_dtype == "float16":
        y, y2, z = y.astype(np.float32), y2.astype(np.float32), z.astype(np.float16).astype(np.float32)
    else:
        y, y2, z = (O.bf16_bits_to_f32(y), O.bf16_bits_to_f32(y2),
                    O.bf16_bits_to_f32(O.f32_to_bf16_bits(z.astype(np.float32))))
    tol = TOL32 if dtype == "float32" else TOL16
    assert O.within(y, z, tol).all(), O.report(y, z, tol)
    assert O.within(y, y2, tol).all(), O.report(y, y2, tol)


@pytest.mark.parametrize("shared_w", [True, False])
def test_gemm_128x192_tiles_batched(bridge, rng, monkeypatch, shared_w):
    """Batched 128x192 tiles (batch 8, ragged M = 1100, K tail 200): each
    batch reads its own A, residual and C slices and either one shared B
    (stride 0) or its own; bit-identical to the 128x128 kernel and within
    the bar of the oracle's per-batch autocast linear."""
    bt, m, k, n = 8, 1100, 200, 768
    x = rng.uniform(-1, 1, (bt, m, k)).astype(np.float32)
    nw = 1 if shared_w else bt
    w = (rng.standard_normal((nw, n, k)) * 0.05).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, (n,)).astype(np.float32)
    r = rng.standard_normal((bt, m, n)).astype(np.float32)
    x16, w16 = x.astype(np.float16), w.astype(np.float16)
    hx, hw, hb, hr = up(bridge, x16), up(bridge, w16), up(bridge, b), up(bridge, r)
    kw = dict(m=m, n=n, k=k, batch=bt, trans_b=True, stride_b=0 if shared_w else n * k, in_dtype="float16",
              out_dtype="float32", bias=hb, round_out=True, residual=hr)
    y = bridge.to_numpy(bridge.matmul_ex(hx, hw, **kw)).reshape(bt, m, n)
    monkeypatch.setenv("BG_GEMM_TILE", "128x128x64s2")
    y2 = bridge.to_numpy(bridge.matmul_ex(hx, hw, **kw)).reshape(bt, m, n)
    assert np.array_equal(y.view(np.uint8), y2.view(np.uint8))
    for i in range(bt):
        wi = w16[0 if shared_w else i]
        z = O.matmul(x16[i], np.ascontiguousarray(wi.T)).astype(np.float32) + b + r[i]
        assert O.within(y[i], z, TOL16).all(), (i, O.report(y[i], z, TOL16))
