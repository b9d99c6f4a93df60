"""Pins the oracle's convolution restatements (oracle/ops.py conv_*) on CPU.

Anchors outside the oracle's own code:
  * the reference's known answers for CONV1D / CONV2D / CONV3D /
    CONV_TRANSPOSE2D forward and backward (packages/browsergrad-kernels/
    tests-browser/webgpu_real.test.ts:943-1400; the conv3d expectations are
    that test's own loop references, restated here as float64 loops);
  * torch.nn.functional.conv1d / conv2d / conv3d / conv_transpose2d and
    their autograd gradients in float64, at the reference bridge tests'
    configurations (webgpu_real.test.ts:1591-1900: groups 2, stride 2,
    padding 2, dilation 2) and at strided / padded / grouped 3-D and
    transposed cases;
  * planted slips (flipped kernel, dilation dropped, padding on one side,
    a transposed convolution taken as a plain one without flipping the
    kernel) that must fail.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops as O

F32 = np.float32


def a(*v):
    return np.array(v, F32)


# ---------------------------------------------------------------- reference known answers


def test_conv1d_conv2d_forward_known_answers():
    # webgpu_real.test.ts:943-1033
    y = O.conv_forward(a(1, 2, 3, 4).reshape(1, 1, 4), a(2, -1).reshape(1, 1, 2), a(0.5), (1,), (0,), (1,), 1, (3,))
    assert y.ravel().tolist() == [0.5, 1.5, 2.5]
    y = O.conv_forward(np.arange(1, 10, dtype=F32).reshape(1, 1, 3, 3), a(1, 0, 0, -1).reshape(1, 1, 2, 2), a(0.5),
                       (1, 1), (0, 0), (1, 1), 1, (2, 2))
    assert y.ravel().tolist() == [-3.5, -3.5, -3.5, -3.5]


def test_conv1d_backward_known_answers():
    # webgpu_real.test.ts:1035-1117
    dy = a(10, 20, 30).reshape(1, 1, 3)
    w = a(2, -1).reshape(1, 1, 2)
    x = a(1, 2, 3, 4).reshape(1, 1, 4)
    assert O.conv_backward_input(dy, w, (1,), (0,), (1,), 1, (4,)).ravel().tolist() == [20, 30, 40, -30]
    assert O.conv_backward_weight(dy, x, (2,), (1,), (0,), (1,), 1).ravel().tolist() == [140, 200]
    assert O.conv_backward_bias(dy).tolist() == [60]


def test_conv2d_backward_known_answers():
    # webgpu_real.test.ts:1119-1203
    dy = a(10, 20, 30, 40).reshape(1, 1, 2, 2)
    w = a(1, 0, 0, -1).reshape(1, 1, 2, 2)
    x = np.arange(1, 10, dtype=F32).reshape(1, 1, 3, 3)
    dx = O.conv_backward_input(dy, w, (1, 1), (0, 0), (1, 1), 1, (3, 3))
    assert dx.ravel().tolist() == [10, 20, 0, 30, 30, -20, 0, -30, -40]
    assert O.conv_backward_weight(dy, x, (2, 2), (1, 1), (0, 0), (1, 1), 1).ravel().tolist() == [370, 470, 670, 770]
    assert O.conv_backward_bias(dy).tolist() == [100]


def test_conv_transpose2d_known_answers():
    # webgpu_real.test.ts:1205-1281
    x = a(1, 2, 3, 4).reshape(1, 1, 2, 2)
    w = a(1, 0, 0, -1).reshape(1, 1, 2, 2)
    dy = np.arange(1, 10, dtype=F32).reshape(1, 1, 3, 3)
    y = O.conv_transpose_forward(x, w, a(0.5), (1, 1), (0, 0), (1, 1), 1, (3, 3))
    assert y.ravel().tolist() == [1.5, 2.5, 0.5, 3.5, 3.5, -1.5, 0.5, -2.5, -3.5]
    assert O.conv_transpose_backward_input(dy, w, (1, 1), (0, 0), (1, 1), 1, (2, 2)).ravel().tolist() == [-4] * 4
    assert O.conv_transpose_backward_weight(dy, x, (2, 2), (1, 1), (0, 0), (1, 1), 1).ravel().tolist() == \
        [37, 47, 67, 77]
    assert O.conv_backward_bias(dy).tolist() == [45]


def _conv3d_test_refs():
    """The loop references of webgpu_real.test.ts:1283-1400 (conv3dRef,
    conv3dDxRef, conv3dDwRef), float64."""
    x = np.arange(1, 28, dtype=np.float64).reshape(3, 3, 3)
    w = np.array([1, 0, 0, 0, 0, 0, 0, -1], np.float64).reshape(2, 2, 2)
    dy = np.arange(1, 9, dtype=np.float64).reshape(2, 2, 2)
    y = np.zeros((2, 2, 2))
    dx = np.zeros((3, 3, 3))
    dw = np.zeros((2, 2, 2))
    for od, oh, ow in np.ndindex(2, 2, 2):
        acc = 0.5
        for rd, rh, rw in np.ndindex(2, 2, 2):
            acc += x[od + rd, oh + rh, ow + rw] * w[rd, rh, rw]
            dx[od + rd, oh + rh, ow + rw] += dy[od, oh, ow] * w[rd, rh, rw]
            dw[rd, rh, rw] += dy[od, oh, ow] * x[od + rd, oh + rh, ow + rw]
        y[od, oh, ow] = acc
    return x, w, dy, y, dx, dw


def test_conv3d_known_answers():
    x, w, dy, y, dx, dw = _conv3d_test_refs()
    x5, w5, dy5 = (t.astype(F32).reshape((1, 1) + t.shape) for t in (x, w, dy))
    one, zero = (1, 1, 1), (0, 0, 0)
    assert np.array_equal(O.conv_forward(x5, w5, a(0.5), one, zero, one, 1, (2, 2, 2)).ravel(), y.ravel())
    assert np.array_equal(O.conv_backward_input(dy5, w5, one, zero, one, 1, (3, 3, 3)).ravel(), dx.ravel())
    assert np.array_equal(O.conv_backward_weight(dy5, x5, (2, 2, 2), one, zero, one, 1).ravel(), dw.ravel())
    assert O.conv_backward_bias(dy5).tolist() == [36]


# ---------------------------------------------------------------- torch float64 cross-checks

CASES = [
    # (rank, n, c_in, in, c_out, k, stride, pad, dil, groups)
    (1, 1, 4, (9,), 6, (3,), (2,), (2,), (2,), 2),                       # webgpu_real.test.ts:1591-1700
    (2, 1, 4, (5, 4), 6, (2, 2), (1, 1), (2, 0), (2, 1), 2),             # webgpu_real.test.ts:1702-1900
    (2, 3, 6, (11, 9), 4, (3, 3), (2, 1), (1, 2), (1, 2), 2),
    (3, 2, 4, (5, 6, 4), 6, (3, 2, 2), (1, 2, 1), (1, 0, 1), (1, 1, 2), 2),
    (1, 2, 3, (17,), 5, (4,), (3,), (0,), (1,), 1),
]

_TORCH_CONV = {1: F.conv1d, 2: F.conv2d, 3: F.conv3d}


def _rand(rng, shape):
    return rng.standard_normal(shape).astype(F32)


def _out_size(in_, k, s, p, d):
    return tuple((in_[i] + 2 * p[i] - d[i] * (k[i] - 1) - 1) // s[i] + 1 for i in range(len(k)))


@pytest.mark.parametrize("case", CASES)
def test_conv_matches_torch_forward_and_grads(case):
    r, n, ci, ins, co, k, s, p, d, g = case
    rng = np.random.default_rng(sum(ins) * 31 + co)
    x = _rand(rng, (n, ci) + ins)
    w = _rand(rng, (co, ci // g) + k)
    b = _rand(rng, (co,))
    out = _out_size(ins, k, s, p, d)
    dy = _rand(rng, (n, co) + out)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    yt = _TORCH_CONV[r](xt, wt, bt, stride=s, padding=p, dilation=d, groups=g)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    tol = 1e-4
    assert O.within(O.conv_forward(x, w, b, s, p, d, g, out), yt.detach().numpy(), tol).all()
    assert O.within(O.conv_backward_input(dy, w, s, p, d, g, ins), xt.grad.numpy(), tol).all()
    assert O.within(O.conv_backward_weight(dy, x, k, s, p, d, g), wt.grad.numpy(), tol).all()
    assert O.within(O.conv_backward_bias(dy), bt.grad.numpy(), tol).all()


TCASES = [
    # (n, c_in, in, c_out, k, stride, pad, out_pad, dil, groups)
    (2, 4, (3, 4), 6, (3, 2), (2, 2), (1, 0), (1, 1), (1, 1), 2),
    (1, 3, (5, 5), 2, (2, 3), (1, 2), (0, 1), (0, 1), (2, 1), 1),
]


@pytest.mark.parametrize("case", TCASES)
def test_conv_transpose2d_matches_torch(case):
    n, ci, ins, co, k, s, p, op, d, g = case
    rng = np.random.default_rng(ci * 7 + co)
    x = _rand(rng, (n, ci) + ins)
    w = _rand(rng, (ci, co // g) + k)
    b = _rand(rng, (co,))
    out = tuple((ins[i] - 1) * s[i] - 2 * p[i] + d[i] * (k[i] - 1) + op[i] + 1 for i in range(2))
    dy = _rand(rng, (n, co) + out)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    yt = F.conv_transpose2d(xt, wt, bt, stride=s, padding=p, output_padding=op, groups=g, dilation=d)
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    tol = 1e-4
    assert O.within(O.conv_transpose_forward(x, w, b, s, p, d, g, out), yt.detach().numpy(), tol).all()
    assert O.within(O.conv_transpose_backward_input(dy, w, s, p, d, g, ins), xt.grad.numpy(), tol).all()
    assert O.within(O.conv_transpose_backward_weight(dy, x, k, s, p, d, g), wt.grad.numpy(), tol).all()
    assert O.within(O.conv_backward_bias(dy), bt.grad.numpy(), tol).all()


def test_output_sizes_beyond_the_formula_read_zeros():
    # The reference takes l_out as given; windows past the padded input read 0.
    x = a(1, 2, 3, 4).reshape(1, 1, 4)
    w = a(2, -1).reshape(1, 1, 2)
    y = O.conv_forward(x, w, None, (1,), (0,), (1,), 1, (5,))
    assert y.ravel().tolist() == [2 * 1 - 2, 2 * 2 - 3, 2 * 3 - 4, 2 * 4 - 0, 0]


# ---------------------------------------------------------------- planted slips


def test_planted_conv_slips_are_caught():
    r, n, ci, ins, co, k, s, p, d, g = CASES[1]
    rng = np.random.default_rng(9)
    x = _rand(rng, (n, ci) + ins)
    w = _rand(rng, (co, ci // g) + k)
    out = _out_size(ins, k, s, p, d)
    ref = F.conv2d(torch.tensor(x, dtype=torch.float64), torch.tensor(w, dtype=torch.float64), stride=s,
                   padding=p, dilation=d, groups=g).numpy()
    assert O.within(O.conv_forward(x, w, None, s, p, d, g, out), ref, 1e-4).all()
    flipped = np.ascontiguousarray(w[:, :, ::-1, ::-1])
    assert not O.within(O.conv_forward(x, flipped, None, s, p, d, g, out), ref, 1e-4).all()
    assert not O.within(O.conv_forward(x, w, None, s, p, (1, 1), g, out), ref, 1e-4).all()
    one_side = np.pad(x, ((0, 0), (0, 0), (2 * p[0], 0), (0, 0)))
    assert not O.within(O.conv_forward(one_side, w, None, s, (0, 0), d, g, out), ref, 1e-4).all()
    xt = _rand(rng, (1, 4, 3, 3))
    wt = _rand(rng, (4, 3, 2, 2))  # transposed layout [c_in, c_out/groups, kh, kw]
    reft = F.conv_transpose2d(torch.tensor(xt, dtype=torch.float64), torch.tensor(wt, dtype=torch.float64)).numpy()
    assert O.within(O.conv_transpose_forward(xt, wt, None, (1, 1), (0, 0), (1, 1), 1, (4, 4)), reft, 1e-4).all()
    # conv_transpose(x, w) == conv(x padded by k - 1, w flipped with its channel axes swapped);
    # without the flip it must fail.
    xp = np.pad(xt, ((0, 0), (0, 0), (1, 1), (1, 1)))
    swapped = np.ascontiguousarray(wt.transpose(1, 0, 2, 3))
    flip = np.ascontiguousarray(swapped[:, :, ::-1, ::-1])
    assert O.within(O.conv_forward(xp, flip, None, (1, 1), (0, 0), (1, 1), 1, (4, 4)), reft, 1e-4).all()
    assert not O.within(O.conv_forward(xp, swapped, None, (1, 1), (0, 0), (1, 1), 1, (4, 4)), reft, 1e-4).all()
