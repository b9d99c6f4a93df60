"""Convolutions on the HIP path (implicit-GEMM f32 MFMA kernels) against the
oracle and float64 torch (GPU).

* Small cases: the reference's known answers (webgpu_real.test.ts:943-1400,
  integer-valued, compared exactly as the reference does with toEqual), its
  bridge-test configurations (:1591-1900) and grouped / strided / dilated
  1-D, 2-D, 3-D and transposed cases against oracle/ops.py with the f32
  abs-or-rel 1e-4 rule.
* Larger cases (ResNet-sized 3x3 layers, split-K weight gradients over 4096
  to 32768 terms): against float64 torch with the bound
  |y - truth| <= 8 sqrt(K) 2^-24 * mass + 1e-6, mass being the same
  operation on absolute values and K its reduction length.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from browsergrad_amd.errors import KernelError
from oracle import ops as O

pytestmark = pytest.mark.gpu

F32 = np.float32
TOL = 1e-4


def up(br, a):
    a = np.ascontiguousarray(a, dtype=F32)
    return br.upload(a, a.shape, "float32")


def fetch(br, h):
    y = br.to_numpy(h)
    br.release(h)
    return y


def conv_ex(br, op, a, b=None, bias=None, **kw):
    hs = [up(br, t) if t is not None else 0 for t in (a, b, bias)]
    try:
        return fetch(br, br.conv_ex(op, hs[0], hs[1], hs[2], **kw))
    finally:
        for h in hs:
            if h:
                br.release(h)


# ---------------------------------------------------------------- reference bridge methods


def _sin_fill(n, f, scale=1.0):
    return (np.sin(np.arange(n) * f) * scale).astype(F32)


def test_bridge_conv1d_reference_config(bridge):
    # webgpu_real.test.ts:1591-1700: N1 C4 L9 COut6 K3 stride2 pad2 dil2 groups2 LOut5
    N, C, L, CO, K, s, p, d, g, LO = 1, 4, 9, 6, 3, 2, 2, 2, 2, 5
    x = _sin_fill(N * C * L, 0.11).reshape(N, C, L)
    w = np.cos(np.arange(CO * (C // g) * K) * 0.09).astype(F32).reshape(CO, C // g, K)
    b = (np.arange(CO) * 0.03 - 0.1).astype(F32)
    dy = _sin_fill(N * CO * LO, 0.17, 0.5).reshape(N, CO, LO)
    hx, hw, hb, hdy = (up(bridge, t) for t in (x, w, b, dy))
    y = fetch(bridge, bridge.conv1d(hx, hw, hb, N, C, L, CO, K, s, p, d, g, LO, "float32"))
    gx = fetch(bridge, bridge.conv1d_backward_input(hdy, hw, N, C, L, CO, K, s, p, d, g, LO, "float32"))
    gw = fetch(bridge, bridge.conv1d_backward_weight(hdy, hx, N, C, L, CO, K, s, p, d, g, LO, "float32"))
    gb = fetch(bridge, bridge.conv1d_backward_bias(hdy, N, CO, LO, "float32"))
    for h in (hx, hw, hb, hdy):
        bridge.release(h)
    assert y.shape == (N, CO, LO) and gx.shape == (N, C, L) and gw.shape == (CO, C // g, K) and gb.shape == (CO,)
    for got, ref in ((y, O.conv_forward(x, w, b, (s,), (p,), (d,), g, (LO,))),
                     (gx, O.conv_backward_input(dy, w, (s,), (p,), (d,), g, (L,))),
                     (gw, O.conv_backward_weight(dy, x, (K,), (s,), (p,), (d,), g)),
                     (gb, O.conv_backward_bias(dy))):
        assert O.within(got, ref, TOL).all(), O.report(got, ref, TOL)


def test_bridge_conv2d_reference_config(bridge):
    # webgpu_real.test.ts:1702-1900: N1 C4 H5 W4 COut6 K2x2 pad (2,0) dil (2,1) groups 2, out 7x3
    N, C, H, W, CO, KH, KW, g, OH, OW = 1, 4, 5, 4, 6, 2, 2, 2, 7, 3
    s, p, d = (1, 1), (2, 0), (2, 1)
    x = _sin_fill(N * C * H * W, 0.13).reshape(N, C, H, W)
    w = np.cos(np.arange(CO * (C // g) * KH * KW) * 0.07).astype(F32).reshape(CO, C // g, KH, KW)
    b = (np.arange(CO) * 0.05 - 0.1).astype(F32)
    dy = _sin_fill(N * CO * OH * OW, 0.17, 0.5).reshape(N, CO, OH, OW)
    hx, hw, hb, hdy = (up(bridge, t) for t in (x, w, b, dy))
    args = (N, C, H, W, CO, KH, KW, s[0], s[1], p[0], p[1], d[0], d[1], g, OH, OW, "float32")
    y = fetch(bridge, bridge.conv2d(hx, hw, hb, *args))
    y_nb = fetch(bridge, bridge.conv2d(hx, hw, None, *args))
    gx = fetch(bridge, bridge.conv2d_backward_input(hdy, hw, *args))
    gw = fetch(bridge, bridge.conv2d_backward_weight(hdy, hx, *args))
    gb = fetch(bridge, bridge.conv2d_backward_bias(hdy, N, CO, OH, OW, "float32"))
    for h in (hx, hw, hb, hdy):
        bridge.release(h)
    for got, ref in ((y, O.conv_forward(x, w, b, s, p, d, g, (OH, OW))),
                     (y_nb, O.conv_forward(x, w, None, s, p, d, g, (OH, OW))),
                     (gx, O.conv_backward_input(dy, w, s, p, d, g, (H, W))),
                     (gw, O.conv_backward_weight(dy, x, (KH, KW), s, p, d, g)),
                     (gb, O.conv_backward_bias(dy))):
        assert O.within(got, ref, TOL).all(), O.report(got, ref, TOL)


@pytest.mark.parametrize("n,o,oh,ow", [(32, 128, 28, 28), (5, 7, 8, 8), (3, 2, 400, 250), (4, 3, 5, 7), (1, 1, 1, 4)])
def test_conv2d_backward_bias_paths(bridge, n, o, oh, ow):
    """The bias gradient sums dy over (n, p) per channel: one workgroup per
    channel in one launch when rows are 4-aligned and a channel holds at most
    2^16 float4 groups (the ResNet layer, a small grid, a 1x4 image), else
    per-row sums then an in-order sum over n (3 x 100000 positions, 5x7
    images).  Checked against float64 sums with a bound of 1e-5 times the
    channel's L1 mass, and repeated bit for bit."""
    rng = np.random.default_rng(n * 1000 + o)
    dy = rng.standard_normal((n, o, oh, ow)).astype(F32)
    h = up(bridge, dy)
    gb = bridge.to_numpy(bridge.conv2d_backward_bias(h, n, o, oh, ow, "float32"))
    gb2 = bridge.to_numpy(bridge.conv2d_backward_bias(h, n, o, oh, ow, "float32"))
    bridge.release(h)
    d64 = dy.astype(np.float64)
    ref = d64.sum(axis=(0, 2, 3))
    bound = 1e-5 * np.abs(d64).sum(axis=(0, 2, 3)) + 1e-6
    assert np.all(np.abs(gb - ref) <= bound), float(np.max(np.abs(gb - ref) / bound))
    assert np.array_equal(gb, gb2)


def test_bridge_conv_errors(bridge):
    x = up(bridge, np.ones((1, 4, 9), F32))
    w = up(bridge, np.ones((6, 2, 3), F32))
    with pytest.raises(KernelError, match="float32"):
        bridge.conv1d(x, w, None, 1, 4, 9, 6, 3, 1, 0, 1, 2, 7, "float16")
    with pytest.raises(KernelError, match="groups"):
        bridge.conv1d(x, w, None, 1, 4, 9, 6, 3, 1, 0, 1, 4, 7, "float32")
    with pytest.raises(KernelError, match="stride must be a positive integer"):
        bridge.conv1d(x, w, None, 1, 4, 9, 6, 3, 0, 0, 1, 2, 7, "float32")
    with pytest.raises(KernelError, match="padding"):
        bridge.conv1d(x, w, None, 1, 4, 9, 6, 3, 1, -1, 1, 2, 7, "float32")
    with pytest.raises(KernelError, match="expected"):
        bridge.conv1d(x, w, None, 1, 4, 8, 6, 3, 1, 0, 1, 2, 6, "float32")  # x holds 36, not 32
    for h in (x, w):
        bridge.release(h)


def test_output_size_beyond_formula_reads_zeros(bridge):
    x = up(bridge, np.array([[[1, 2, 3, 4]]], F32))
    w = up(bridge, np.array([[[2, -1]]], F32))
    y = fetch(bridge, bridge.conv1d(x, w, None, 1, 1, 4, 1, 2, 1, 0, 1, 1, 5, "float32"))
    assert y.ravel().tolist() == [0, 1, 2, 8, 0]
    for h in (x, w):
        bridge.release(h)


# ---------------------------------------------------------------- the reference's plans


def _plan(ops_steps, shapes, root_shape, op, arg):
    steps = [{"step": i, "value_id": i, "op": "BUFFER", "input_ids": [], "shape": list(sh), "dtype": "float32"}
             for i, sh in enumerate(shapes)]
    k = len(shapes)
    steps += [{"step": k + i, "value_id": k + i, "op": "LOAD", "input_ids": [i], "shape": list(sh),
               "dtype": "float32"} for i, sh in enumerate(shapes)]
    root = 2 * k
    steps.append({"step": root, "value_id": root, "op": op, "input_ids": [k + i for i in range(ops_steps)],
                  "shape": list(root_shape), "dtype": "float32", "arg": arg})
    buffers = [{"value_id": st["value_id"], "op": st["op"], "shape": st["shape"], "dtype": "float32",
                "bytes": 4 * int(np.prod(st["shape"])), "first_step": st["step"], "last_step": root,
                "materialize": st["value_id"] == root} for st in steps]
    return {"steps": steps, "buffers": buffers, "root_id": root, "materialization_boundary": "root",
            "peak_live_bytes": 0, "has_custom_ops": False}


def run_plan(bridge, op, arg, inputs, root_shape):
    plan = _plan(len(inputs), [t.shape for t in inputs], root_shape, op, arg)
    data = [{"value_id": i, "data": np.ascontiguousarray(t, F32).tobytes()} for i, t in enumerate(inputs)]
    return np.frombuffer(bridge.run_tensor_plan(plan, data, "float32"), F32).tolist()


A1 = dict(n=1, c_in=1, l_in=4, c_out=1, k=2, stride=1, padding=0, dilation=1, groups=1, l_out=3)
A2 = dict(n=1, c_in=1, h=3, w=3, c_out=1, kh=2, kw=2, stride_h=1, stride_w=1, pad_h=0, pad_w=0,
          dilation_h=1, dilation_w=1, groups=1, out_h=2, out_w=2)
AT = dict(n=1, c_in=1, h=2, w=2, c_out=1, c_out_per_group=1, kh=2, kw=2, stride_h=1, stride_w=1, pad_h=0,
          pad_w=0, output_pad_h=0, output_pad_w=0, dilation_h=1, dilation_w=1, groups=1, out_h=3, out_w=3)
A3 = dict(n=1, c_in=1, d=3, h=3, w=3, c_out=1, kd=2, kh=2, kw=2, stride_d=1, stride_h=1, stride_w=1,
          pad_d=0, pad_h=0, pad_w=0, dilation_d=1, dilation_h=1, dilation_w=1, groups=1, out_d=2, out_h=2, out_w=2)


def t(*v, shape):
    return np.array(v, F32).reshape(shape)


def test_plan_conv1d_conv2d_forward(bridge):
    # webgpu_real.test.ts:943-1033
    y = run_plan(bridge, "CONV1D", {**A1, "has_bias": True},
                 [t(1, 2, 3, 4, shape=(1, 1, 4)), t(2, -1, shape=(1, 1, 2)), t(0.5, shape=(1,))], (1, 1, 3))
    assert y == [0.5, 1.5, 2.5]
    y = run_plan(bridge, "CONV2D", {**A2, "has_bias": True},
                 [np.arange(1, 10, dtype=F32).reshape(1, 1, 3, 3), t(1, 0, 0, -1, shape=(1, 1, 2, 2)),
                  t(0.5, shape=(1,))], (1, 1, 2, 2))
    assert y == [-3.5] * 4


def test_plan_conv1d_conv2d_backward(bridge):
    # webgpu_real.test.ts:1035-1203
    dy1, w1, x1 = t(10, 20, 30, shape=(1, 1, 3)), t(2, -1, shape=(1, 1, 2)), t(1, 2, 3, 4, shape=(1, 1, 4))
    assert run_plan(bridge, "CONV1D_BACKWARD_INPUT", A1, [dy1, w1], (1, 1, 4)) == [20, 30, 40, -30]
    assert run_plan(bridge, "CONV1D_BACKWARD_WEIGHT", A1, [dy1, x1], (1, 1, 2)) == [140, 200]
    assert run_plan(bridge, "CONV1D_BACKWARD_BIAS", A1, [dy1], (1,)) == [60]
    dy2, w2 = t(10, 20, 30, 40, shape=(1, 1, 2, 2)), t(1, 0, 0, -1, shape=(1, 1, 2, 2))
    x2 = np.arange(1, 10, dtype=F32).reshape(1, 1, 3, 3)
    assert run_plan(bridge, "CONV2D_BACKWARD_INPUT", A2, [dy2, w2], (1, 1, 3, 3)) == \
        [10, 20, 0, 30, 30, -20, 0, -30, -40]
    assert run_plan(bridge, "CONV2D_BACKWARD_WEIGHT", A2, [dy2, x2], (1, 1, 2, 2)) == [370, 470, 670, 770]
    assert run_plan(bridge, "CONV2D_BACKWARD_BIAS", A2, [dy2], (1,)) == [100]


def test_plan_conv_transpose2d(bridge):
    # webgpu_real.test.ts:1205-1281
    x, w = t(1, 2, 3, 4, shape=(1, 1, 2, 2)), t(1, 0, 0, -1, shape=(1, 1, 2, 2))
    dy = np.arange(1, 10, dtype=F32).reshape(1, 1, 3, 3)
    assert run_plan(bridge, "CONV_TRANSPOSE2D", AT, [x, w, t(0.5, shape=(1,))], (1, 1, 3, 3)) == \
        [1.5, 2.5, 0.5, 3.5, 3.5, -1.5, 0.5, -2.5, -3.5]
    assert run_plan(bridge, "CONV_TRANSPOSE2D_BACKWARD_INPUT", AT, [dy, w], (1, 1, 2, 2)) == [-4] * 4
    assert run_plan(bridge, "CONV_TRANSPOSE2D_BACKWARD_WEIGHT", AT, [dy, x], (1, 1, 2, 2)) == [37, 47, 67, 77]
    assert run_plan(bridge, "CONV_TRANSPOSE2D_BACKWARD_BIAS", AT, [dy], (1,)) == [45]


def test_plan_conv3d(bridge):
    # webgpu_real.test.ts:1283-1400 (expectations from that test's loop references)
    x = np.arange(1, 28, dtype=F32).reshape(1, 1, 3, 3, 3)
    w = t(1, 0, 0, 0, 0, 0, 0, -1, shape=(1, 1, 2, 2, 2))
    dy = np.arange(1, 9, dtype=F32).reshape(1, 1, 2, 2, 2)
    one, zero = (1, 1, 1), (0, 0, 0)
    assert run_plan(bridge, "CONV3D", A3, [x, w, t(0.5, shape=(1,))], (1, 1, 2, 2, 2)) == \
        O.conv_forward(x, w, t(0.5, shape=(1,)), one, zero, one, 1, (2, 2, 2)).ravel().tolist()
    assert run_plan(bridge, "CONV3D_BACKWARD_INPUT", A3, [dy, w], (1, 1, 3, 3, 3)) == \
        O.conv_backward_input(dy, w, one, zero, one, 1, (3, 3, 3)).ravel().tolist()
    assert run_plan(bridge, "CONV3D_BACKWARD_WEIGHT", A3, [dy, x], (1, 1, 2, 2, 2)) == \
        O.conv_backward_weight(dy, x, (2, 2, 2), one, zero, one, 1).ravel().tolist()
    assert run_plan(bridge, "CONV3D_BACKWARD_BIAS", A3, [dy], (1,)) == [36]


def test_plan_conv_argument_rules(bridge):
    x, w = t(1, 2, 3, 4, shape=(1, 1, 4)), t(2, -1, shape=(1, 1, 2))
    bad = dict(A1)
    del bad["l_out"]
    with pytest.raises(KernelError, match="CONV1D.l_out must be an integer"):
        run_plan(bridge, "CONV1D", bad, [x, w], (1, 1, 3))
    with pytest.raises(KernelError, match="tensor plan CONV1D.stride must be a positive integer"):
        run_plan(bridge, "CONV1D", {**A1, "stride": 0}, [x, w], (1, 1, 3))
    with pytest.raises(KernelError, match="tensor plan CONV1D.padding must be a non-negative integer"):
        run_plan(bridge, "CONV1D", {**A1, "padding": -1}, [x, w], (1, 1, 3))
    with pytest.raises(KernelError, match="CONV1D.output shape mismatch at dim 2"):
        run_plan(bridge, "CONV1D", A1, [x, w], (1, 1, 4))
    with pytest.raises(KernelError, match="CONV1D.weight"):
        run_plan(bridge, "CONV1D", A1, [x, t(2, -1, 0, shape=(1, 1, 3))], (1, 1, 3))
    with pytest.raises(KernelError, match="CONV2D padding must be non-negative integers"):
        run_plan(bridge, "CONV2D", {**A2, "pad_w": -1}, [np.ones((1, 1, 3, 3), F32), np.ones((1, 1, 2, 2), F32)],
                 (1, 1, 2, 2))
    with pytest.raises(KernelError, match="channels must be divisible by groups"):
        run_plan(bridge, "CONV2D", {**A2, "groups": 2}, [np.ones((1, 1, 3, 3), F32), np.ones((1, 1, 2, 2), F32)],
                 (1, 1, 2, 2))
    xt_, wt_ = t(1, 2, 3, 4, shape=(1, 1, 2, 2)), t(1, 0, 0, -1, shape=(1, 1, 2, 2))
    with pytest.raises(KernelError, match="output_padding must be smaller than stride"):
        run_plan(bridge, "CONV_TRANSPOSE2D", {**AT, "output_pad_h": 1}, [xt_, wt_], (1, 1, 3, 3))
    with pytest.raises(KernelError, match="channels must match groups"):
        run_plan(bridge, "CONV_TRANSPOSE2D", {**AT, "c_out_per_group": 2}, [xt_, wt_], (1, 1, 3, 3))
    with pytest.raises(KernelError, match="tensor plan CONV3D.kd must be a positive integer"):
        run_plan(bridge, "CONV3D", {**A3, "kd": 0}, [np.ones((1, 1, 3, 3, 3), F32), np.ones((1, 1, 2, 2, 2), F32)],
                 (1, 1, 2, 2, 2))


# ---------------------------------------------------------------- descriptor route vs the oracle

CASES = [
    (1, 1, 4, (9,), 6, (3,), (2,), (2,), (2,), 2),
    (2, 1, 4, (5, 4), 6, (2, 2), (1, 1), (2, 0), (2, 1), 2),
    (2, 3, 6, (11, 9), 4, (3, 3), (2, 1), (1, 2), (1, 2), 2),
    (2, 2, 8, (13, 7), 8, (1, 1), (1, 1), (0, 0), (1, 1), 8),     # depthwise 1x1
    (3, 2, 4, (5, 6, 4), 6, (3, 2, 2), (1, 2, 1), (1, 0, 1), (1, 1, 2), 2),
    (1, 2, 3, (17,), 5, (4,), (3,), (0,), (1,), 1),
    (2, 3, 5, (31, 29), 70, (3, 3), (2, 2), (1, 1), (1, 1), 1),   # column tiles past 64
]


def _out_size(in_, k, s, p, d):
    return tuple((in_[i] + 2 * p[i] - d[i] * (k[i] - 1) - 1) // s[i] + 1 for i in range(len(k)))


@pytest.mark.parametrize("case", CASES)
def test_conv_ex_matches_oracle(bridge, case):
    r, n, ci, ins, co, k, s, p, d, g = case
    rng = np.random.default_rng(sum(ins) + 13 * co)
    x = rng.standard_normal((n, ci) + ins).astype(F32)
    w = rng.standard_normal((co, ci // g) + k).astype(F32)
    b = rng.standard_normal(co).astype(F32)
    out = _out_size(ins, k, s, p, d)
    dy = rng.standard_normal((n, co) + out).astype(F32)
    kw = dict(n=n, c_in=ci, c_out=co, in_size=ins, out_size=out, k=k, stride=s, pad=p, dilation=d, groups=g)
    checks = [
        (conv_ex(bridge, "forward", x, w, b, **kw), O.conv_forward(x, w, b, s, p, d, g, out)),
        (conv_ex(bridge, "backward_input", dy, w, **kw), O.conv_backward_input(dy, w, s, p, d, g, ins)),
        (conv_ex(bridge, "backward_weight", dy, x, **kw), O.conv_backward_weight(dy, x, k, s, p, d, g)),
        (conv_ex(bridge, "backward_bias", dy, **kw), O.conv_backward_bias(dy)),
    ]
    for got, ref in checks:
        assert got.shape == ref.shape
        assert O.within(got, ref, TOL).all(), O.report(got, ref, TOL)


@pytest.mark.parametrize("case", [CASES[i] for i in (0, 2, 3, 5, 6)])
def test_conv_forward_ring_matches_register_kernel(bridge, case, monkeypatch):
    """The forward (and the stride-1 input gradient, which runs as a forward
    convolution) copies its operands into an LDS ring; BG_CONV_RING=0 selects
    the register-staged kernel. Both feed the MFMAs the same k sequence, so
    the outputs are bit-identical, and both match the oracle.  (A strided
    input gradient runs as phase convolutions on the ring kernel, a
    different sum order from the DGRAD kernel: switched off here.)"""
    monkeypatch.setenv("BG_CONV_DGRAD_PHASES", "0")
    r, n, ci, ins, co, k, s, p, d, g = case
    rng = np.random.default_rng(sum(ins) + 29 * co)
    x = rng.standard_normal((n, ci) + ins).astype(F32)
    w = rng.standard_normal((co, ci // g) + k).astype(F32)
    b = rng.standard_normal(co).astype(F32)
    out = _out_size(ins, k, s, p, d)
    dy = rng.standard_normal((n, co) + out).astype(F32)
    kw = dict(n=n, c_in=ci, c_out=co, in_size=ins, out_size=out, k=k, stride=s, pad=p, dilation=d, groups=g)
    runs = {}
    for env in ("1", "0"):
        monkeypatch.setenv("BG_CONV_RING", env)
        runs[env] = (conv_ex(bridge, "forward", x, w, b, **kw), conv_ex(bridge, "backward_input", dy, w, **kw))
    for got, ref in zip(runs["1"], (O.conv_forward(x, w, b, s, p, d, g, out),
                                    O.conv_backward_input(dy, w, s, p, d, g, ins))):
        assert O.within(got, ref, TOL).all(), O.report(got, ref, TOL)
    for a, c in zip(runs["1"], runs["0"]):
        assert np.array_equal(a, c)


TCASES = [
    (2, 4, (3, 4), 6, (3, 2), (2, 2), (1, 0), (1, 1), (1, 1), 2),
    (1, 3, (5, 5), 2, (2, 3), (1, 2), (0, 1), (0, 1), (2, 1), 1),
]


@pytest.mark.parametrize("case", TCASES)
def test_conv_transpose_ex_matches_oracle(bridge, case):
    n, ci, ins, co, k, s, p, op, d, g = case
    rng = np.random.default_rng(ci * 7 + co)
    x = rng.standard_normal((n, ci) + ins).astype(F32)
    w = rng.standard_normal((ci, co // g) + k).astype(F32)
    b = rng.standard_normal(co).astype(F32)
    out = tuple((ins[i] - 1) * s[i] - 2 * p[i] + d[i] * (k[i] - 1) + op[i] + 1 for i in range(2))
    dy = rng.standard_normal((n, co) + out).astype(F32)
    kw = dict(n=n, c_in=ci, c_out=co, in_size=ins, out_size=out, k=k, stride=s, pad=p, dilation=d, groups=g,
              transposed=True, output_pad=op)
    checks = [
        (conv_ex(bridge, "forward", x, w, b, **kw), O.conv_transpose_forward(x, w, b, s, p, d, g, out)),
        (conv_ex(bridge, "backward_input", dy, w, **kw), O.conv_transpose_backward_input(dy, w, s, p, d, g, ins)),
        (conv_ex(bridge, "backward_weight", dy, x, **kw), O.conv_transpose_backward_weight(dy, x, k, s, p, d, g)),
        (conv_ex(bridge, "backward_bias", dy, **kw), O.conv_backward_bias(dy)),
    ]
    for got, ref in checks:
        assert got.shape == ref.shape
        assert O.within(got, ref, TOL).all(), O.report(got, ref, TOL)


# ---------------------------------------------------------------- larger layers vs float64


BIG = [
    # (n, c_in, hw, c_out, k, stride, pad)
    (4, 64, (32, 32), 64, (3, 3), (1, 1), (1, 1)),
    (8, 32, (16, 16), 96, (3, 3), (2, 2), (1, 1)),
    (2, 3, (64, 64), 16, (7, 7), (2, 2), (3, 3)),
    # 512 output tiles of 128 x 128 for the forward and of 128 x 64 for the
    # stride-1 input gradient (run as a forward convolution with C and O
    # exchanged): the ring kernel's 128-wide shapes.
    (16, 4, (64, 64), 128, (3, 3), (1, 1), (1, 1)),
]


def _bound(truth, mass, K):
    return 8 * math.sqrt(K) * 2.0 ** -24 * mass + 1e-6


@pytest.mark.parametrize("case", BIG)
def test_conv2d_large_against_float64(bridge, case):
    n, ci, hw, co, k, s, p = case
    rng = np.random.default_rng(ci + co)
    x = rng.standard_normal((n, ci) + hw).astype(F32)
    w = (rng.standard_normal((co, ci) + k) / math.sqrt(ci * k[0] * k[1])).astype(F32)
    out = _out_size(hw, k, s, p, (1, 1))
    dy = rng.standard_normal((n, co) + out).astype(F32)
    kw = dict(n=n, c_in=ci, c_out=co, in_size=hw, out_size=out, k=k, stride=s, pad=p, dilation=(1, 1))

    def torch_grads(xa, wa, dya):
        xt = torch.tensor(xa, dtype=torch.float64, requires_grad=True)
        wt = torch.tensor(wa, dtype=torch.float64, requires_grad=True)
        y = F.conv2d(xt, wt, stride=s, padding=p)
        y.backward(torch.tensor(dya, dtype=torch.float64))
        return y.detach().numpy(), xt.grad.numpy(), wt.grad.numpy()

    y64, gx64, gw64 = torch_grads(x, w, dy)
    my, mgx, mgw = torch_grads(np.abs(x), np.abs(w), np.abs(dy))
    y = conv_ex(bridge, "forward", x, w, **kw)
    gx = conv_ex(bridge, "backward_input", dy, w, **kw)
    gw = conv_ex(bridge, "backward_weight", dy, x, **kw)
    for got, truth, mass, K in ((y, y64, my, ci * k[0] * k[1]), (gx, gx64, mgx, co * k[0] * k[1]),
                                (gw, gw64, mgw, n * out[0] * out[1])):
        err = np.abs(got - truth)
        bound = _bound(truth, mass, K)
        assert np.all(err <= bound), float(np.max(err / bound))


def test_conv_ring_wide_tiles_launched(bridge, monkeypatch):
    """BIG's last case runs the ring kernel's 128 x 128 shape (forward) and
    128 x 64 shape (stride-1 input gradient), as the launch log shows (with
    the 3x3 input-patch kernel switched off: it takes this shape by default)."""
    monkeypatch.setenv("BG_CONV_HALO", "0")
    n, ci, hw, co, k, s, p = BIG[-1]
    rng = np.random.default_rng(5)
    x = rng.standard_normal((n, ci) + hw).astype(F32)
    w = rng.standard_normal((co, ci) + k).astype(F32)
    out = _out_size(hw, k, s, p, (1, 1))
    dy = rng.standard_normal((n, co) + out).astype(F32)
    kw = dict(n=n, c_in=ci, c_out=co, in_size=hw, out_size=out, k=k, stride=s, pad=p, dilation=(1, 1))
    bridge.set_launch_log(True)
    try:
        bridge.take_launch_log()
        conv_ex(bridge, "forward", x, w, **kw)
        fwd = [r["kernel"] for r in bridge.take_launch_log()]
        conv_ex(bridge, "backward_input", dy, w, **kw)
        bwd = [r["kernel"] for r in bridge.take_launch_log()]
    finally:
        bridge.set_launch_log(False)
    wide = lambda names, bn: any("conv_fwd_ring_kernel" in t and (f"ILi128ELi{bn}ELi4E" in t or f"<128, {bn}, 4>" in t)
                                 for t in names)
    assert wide(fwd, 128), fwd
    assert wide(bwd, 64), bwd


def test_conv_ring_64x128_tiles(bridge, monkeypatch):
    """Fewer than 128 output positions (M = 64) against 256 output channels
    per group and 256 groups make 512 tiles of 64 x 128: the ring kernel's
    64 x 128 shape.  It is bit-identical to the register-staged kernel and
    within the float64 bound."""
    n, hw, cpg, opg, g, k = 1, (8, 8), 2, 256, 256, (3, 3)
    ci, co = cpg * g, opg * g
    rng = np.random.default_rng(64128)
    x = rng.standard_normal((n, ci) + hw).astype(F32)
    w = (rng.standard_normal((co, cpg) + k) / math.sqrt(cpg * 9)).astype(F32)
    b = rng.standard_normal(co).astype(F32)
    kw = dict(n=n, c_in=ci, c_out=co, in_size=hw, out_size=hw, k=k, stride=(1, 1), pad=(1, 1), dilation=(1, 1),
              groups=g)
    monkeypatch.setenv("BG_CONV_RING", "1")
    monkeypatch.setenv("BG_CONV_HALO", "0")
    bridge.set_launch_log(True)
    try:
        bridge.take_launch_log()
        y = conv_ex(bridge, "forward", x, w, b, **kw)
        names = [r["kernel"] for r in bridge.take_launch_log()]
    finally:
        bridge.set_launch_log(False)
    assert any("conv_fwd_ring_kernel" in t and ("ILi64ELi128ELi4E" in t or "<64, 128, 4>" in t) for t in names), names
    monkeypatch.setenv("BG_CONV_RING", "0")
    y0 = conv_ex(bridge, "forward", x, w, b, **kw)
    assert np.array_equal(y, y0)
    xt = torch.tensor(x, dtype=torch.float64)
    wt = torch.tensor(w, dtype=torch.float64)
    bt = torch.tensor(b, dtype=torch.float64)
    y64 = F.conv2d(xt, wt, bt, padding=1, groups=g).numpy()
    mass = F.conv2d(xt.abs(), wt.abs(), bt.abs(), padding=1, groups=g).numpy()
    err = np.abs(y - y64)
    assert np.all(err <= _bound(y64, mass, cpg * 9)), float(np.max(err / _bound(y64, mass, cpg * 9)))


HALO = [
    # n, c_in, (H, W), c_out, pad, groups
    (2, 5, (28, 28), 12, (1, 1), 1),    # two output rows per tile, odd channel count
    (3, 4, (18, 18), 8, (1, 1), 1),     # 54-row tiles: every other one starts off a multiple of 4
    (2, 6, (7, 9), 16, (1, 1), 2),      # groups; 63 of the 64 tile rows used
    (1, 3, (64, 64), 68, (1, 1), 1),    # one output row per 64-row tile; a second column tile
    (2, 4, (40, 40), 8, (1, 1), 1),     # three output rows per 128-row tile (120 of 128 used)
    (2, 4, (10, 12), 4, (0, 0), 1),     # no padding; the last tile of each image is partial
    (1, 2, (5, 3), 8, (2, 2), 1),       # padding 2: whole patch rows and columns outside the image
    (1, 9, (1, 1), 4, (1, 1), 1),       # a 1 x 1 image
    (32, 128, (28, 28), 128, (1, 1), 1),  # the benchmark layer (register kernel only, no oracle)
    (32, 8, (7, 7), 512, (1, 1), 1),    # 7 x 7 images: 64-row tiles (49 of 64 rows) though 128 would fill the CUs
    (1, 3, (100, 112), 8, (1, 1), 1),   # 112-wide rows: 128-row tiles with two patch copies per wavefront
]


def _halo_fits(bm, ow):
    tr = bm // ow
    return tr > 0 and 2 * (tr + 2) * (ow + 2) <= (1024 if bm == 128 else 512)


def _halo_tile(names):
    """Tile height of the input-patch kernel in a launch log (0 if absent)."""
    for t in names:
        if "conv_fwd_halo_kernel" in t:
            return 128 if any(f"ILi4ELi2ELi4ELi2ELi{pc}E" in t or f"<4, 2, 4, 2, {pc}>" in t for pc in (1, 2)) else 64
    return 0


@pytest.mark.parametrize("case", HALO)
def test_conv3x3_input_patch_kernel(bridge, case, monkeypatch):
    """3x3 stride-1 2-D convolutions run on the input-patch kernel, in
    128 x 64 or 64 x 64 tiles (BG_CONV_HALO=128 / =64 ask for one where
    the two channels' patches fit; the launch log shows which ran; the
    stride-1 input gradient takes it too when c_in per group is a multiple
    of 4).  Both take the ring kernel's k order and MFMA pairs, so they are
    bit-identical to the register-staged kernel (BG_CONV_RING=0), and they
    match the oracle."""
    n, ci, hw, co, p, g = case
    k, s, d = (3, 3), (1, 1), (1, 1)
    rng = np.random.default_rng(n * 1000 + ci * 10 + co)
    x = rng.standard_normal((n, ci) + hw).astype(F32)
    w = rng.standard_normal((co, ci // g) + k).astype(F32)
    b = rng.standard_normal(co).astype(F32)
    out = _out_size(hw, k, s, p, d)
    dy = rng.standard_normal((n, co) + out).astype(F32)
    kw = dict(n=n, c_in=ci, c_out=co, in_size=hw, out_size=out, k=k, stride=s, pad=p, dilation=d, groups=g)
    runs = {}
    for ask in ("", "64", "128"):
        if ask and not _halo_fits(int(ask), out[1]):
            continue
        if ask:
            monkeypatch.setenv("BG_CONV_HALO", ask)
        bridge.set_launch_log(True)
        try:
            bridge.take_launch_log()
            y = conv_ex(bridge, "forward", x, w, b, **kw)
            fwd = [r["kernel"] for r in bridge.take_launch_log()]
            gx = conv_ex(bridge, "backward_input", dy, w, **kw)
            bwd = [r["kernel"] for r in bridge.take_launch_log()]
        finally:
            bridge.set_launch_log(False)
        if ask:
            assert _halo_tile(fwd) == int(ask), fwd
        else:  # 128-row tiles where they fit, give a workgroup per CU and leave no more rows empty
            tr = 128 // out[1]
            tiles = n * -(-out[0] // tr) * -(-(co // g) // 64) * g if tr else 0
            tr64 = 64 // out[1]
            big = _halo_fits(128, out[1]) and (not _halo_fits(64, out[1]) or (
                tiles >= 256 and -(-out[0] // tr64) * 64 >= -(-out[0] // tr) * 128))
            assert _halo_tile(fwd) == (128 if big else 64), fwd
        if (ci // g) % 4 == 0 and _halo_fits(64, hw[1]):
            assert _halo_tile(bwd), bwd
        runs[ask] = (y, gx)
    assert "128" in runs or "64" in runs
    monkeypatch.setenv("BG_CONV_RING", "0")
    monkeypatch.delenv("BG_CONV_HALO", raising=False)
    y0 = conv_ex(bridge, "forward", x, w, b, **kw)
    gx0 = conv_ex(bridge, "backward_input", dy, w, **kw)
    for y, gx in runs.values():
        assert np.array_equal(y, y0)
        assert np.array_equal(gx, gx0)
    if n * ci * hw[0] * hw[1] <= 1 << 16 and co * 9 <= 600:
        for got, ref in ((y0, O.conv_forward(x, w, b, s, p, d, g, out)),
                         (gx0, O.conv_backward_input(dy, w, s, p, d, g, hw))):
            assert O.within(got, ref, TOL).all(), O.report(got, ref, TOL)
    elif n * ci * hw[0] * hw[1] <= 1 << 16:
        # Long input-gradient sums (co * 9 terms): float64 with the sqrt(K) bound.
        xt, wt, dyt = (torch.tensor(t, dtype=torch.float64) for t in (x, w, dy))
        y64 = F.conv2d(xt, wt, torch.tensor(b, dtype=torch.float64), padding=p, groups=g).numpy()
        ym = F.conv2d(xt.abs(), wt.abs(), torch.tensor(np.abs(b), dtype=torch.float64), padding=p, groups=g).numpy()
        gx64 = torch.nn.grad.conv2d_input(xt.shape, wt, dyt, padding=p, groups=g).numpy()
        gxm = torch.nn.grad.conv2d_input(xt.shape, wt.abs(), dyt.abs(), padding=p, groups=g).numpy()
        for got, truth, mass, kk in ((y0, y64, ym, (ci // g) * 9), (gx0, gx64, gxm, (co // g) * 9)):
            assert np.all(np.abs(got - truth) <= _bound(truth, mass, kk))


def test_conv3x3_input_patch_output_beyond_formula(bridge, monkeypatch):
    """A caller-given output larger than the formula's (8 x 7 from a 6 x 6
    input with padding 1) reads zeros past the input, as the reference's
    bounds-checked loop does; the input-patch kernel runs it (launch log),
    bit-identical to the register-staged kernel and equal to the oracle."""
    rng = np.random.default_rng(87)
    x = rng.standard_normal((2, 4, 6, 6)).astype(F32)
    w = rng.standard_normal((8, 4, 3, 3)).astype(F32)
    b = rng.standard_normal(8).astype(F32)
    kw = dict(n=2, c_in=4, c_out=8, in_size=(6, 6), out_size=(8, 7), k=(3, 3), stride=(1, 1), pad=(1, 1),
              dilation=(1, 1), groups=1)
    bridge.set_launch_log(True)
    try:
        bridge.take_launch_log()
        y = conv_ex(bridge, "forward", x, w, b, **kw)
        names = [r["kernel"] for r in bridge.take_launch_log()]
    finally:
        bridge.set_launch_log(False)
    assert _halo_tile(names), names
    ref = O.conv_forward(x, w, b, (1, 1), (1, 1), (1, 1), 1, (8, 7))
    assert y.shape == ref.shape == (2, 8, 8, 7)
    assert O.within(y, ref, TOL).all(), O.report(y, ref, TOL)
    monkeypatch.setenv("BG_CONV_RING", "0")
    assert np.array_equal(y, conv_ex(bridge, "forward", x, w, b, **kw))


STRIDED = [
    # n, c_in, (H, W), c_out, k, stride, pad, groups, phases used
    (2, 6, (11, 9), 8, (3, 3), (2, 2), (1, 1), 1, True),
    (1, 4, (12, 12), 6, (3, 3), (2, 2), (0, 0), 2, True),
    (2, 4, (9, 10), 4, (1, 1), (2, 2), (0, 0), 1, True),    # 1x1 stride 2: three phases no tap reaches
    (1, 2, (10, 11), 3, (3, 3), (3, 2), (0, 1), 1, True),   # stride 3 x 2
    (1, 3, (8, 8), 5, (2, 2), (2, 2), (0, 0), 1, True),     # one tap per phase
    (2, 3, (9, 13), 4, (5, 3), (2, 2), (2, 1), 1, True),    # a 5-tall kernel: up to 3 taps per phase
    (2, 3, (7, 13), 4, (5, 3), (2, 3), (2, 1), 1, True),    # a phase whose first tap reads past dy's first column
    (1, 2, (10, 11), 3, (3, 3), (3, 3), (1, 1), 1, True),   # stride 3, padding 1: negative leading padding
    (2, 2, (6, 6), 3, (3, 3), (2, 2), (1, 1), 1, True),     # tiny images
    (32, 64, (56, 56), 128, (3, 3), (2, 2), (1, 1), 1, True),  # ResNet's downsampling layer (float64 bound)
]


@pytest.mark.parametrize("case", STRIDED)
def test_conv_strided_input_gradient_phases(bridge, case, monkeypatch):
    """A strided 2-D input gradient runs as stride_h x stride_w phase
    convolutions (dense stride-1 forward convolutions of dy by each phase's
    taps, written to that phase's positions of dx; the launch log shows the
    phase weights), against the oracle (or float64 with the sqrt(K) bound at
    the large shape) and against the DGRAD kernel (BG_CONV_DGRAD_PHASES=0)."""
    n, ci, hw, co, k, s, p, g, phases = case
    d = (1, 1)
    rng = np.random.default_rng(n * 31 + ci * 7 + co)
    w = rng.standard_normal((co, ci // g) + k).astype(F32)
    out = _out_size(hw, k, s, p, d)
    dy = rng.standard_normal((n, co) + out).astype(F32)
    kw = dict(n=n, c_in=ci, c_out=co, in_size=hw, out_size=out, k=k, stride=s, pad=p, dilation=d, groups=g)
    bridge.set_launch_log(True)
    try:
        bridge.take_launch_log()
        gx = conv_ex(bridge, "backward_input", dy, w, **kw)
        names = [r["kernel"] for r in bridge.take_launch_log()]
    finally:
        bridge.set_launch_log(False)
    assert any("conv_phase_weight_kernel" in t for t in names) == phases, names
    monkeypatch.setenv("BG_CONV_DGRAD_PHASES", "0")
    gx0 = conv_ex(bridge, "backward_input", dy, w, **kw)
    if n * ci * hw[0] * hw[1] <= 1 << 16:
        ref = O.conv_backward_input(dy, w, s, p, d, g, hw)
        for got in (gx, gx0):
            assert got.shape == ref.shape
            assert O.within(got, ref, TOL).all(), O.report(got, ref, TOL)
    else:
        wt, dyt = torch.tensor(w, dtype=torch.float64), torch.tensor(dy, dtype=torch.float64)
        shape = (n, ci) + hw
        truth = torch.nn.grad.conv2d_input(shape, wt, dyt, stride=s, padding=p, groups=g).numpy()
        mass = torch.nn.grad.conv2d_input(shape, wt.abs(), dyt.abs(), stride=s, padding=p, groups=g).numpy()
        bound = _bound(truth, mass, (co // g) * k[0] * k[1])
        for got in (gx, gx0):
            assert np.all(np.abs(got - truth) <= bound), float(np.max(np.abs(got - truth) / bound))


@pytest.mark.parametrize("shape", [(4, 16, 28, 28), (3, 5, 7, 7), (2, 3, 4, 300)])
def test_bias_gradient_float4_and_scalar_rows(bridge, shape):
    """Spatial sizes that are multiples of 4 (784, 1200) take the float4 row
    sum, 49 the scalar one; both against the oracle's sum over (n, spatial)."""
    n, co, oh, ow = shape
    dy = np.random.default_rng(oh * ow + co).standard_normal(shape).astype(F32)
    kw = dict(n=n, c_in=co, c_out=co, in_size=(oh, ow), out_size=(oh, ow), k=(1, 1), stride=(1, 1),
              pad=(0, 0), dilation=(1, 1), groups=1)
    got = conv_ex(bridge, "backward_bias", dy, **kw)
    ref = O.conv_backward_bias(dy)
    assert got.shape == ref.shape
    assert O.within(got, ref, TOL).all(), O.report(got, ref, TOL)
