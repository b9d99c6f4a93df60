"""Convolution nodes in this package's front end (browsergrad_amd/jit):
graph building (tensor.conv1d/2d/3d), the graph oracle's CONV handlers, the
plan builder (CONV steps with the reference plan's arg fields), and on the
GPU the walker and the plan route against the graph oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from browsergrad_amd.jit.buffers import GpuBufferTable
from browsergrad_amd.jit.gpu_plan import build_gpu_execution_submission
from browsergrad_amd.jit.realize import realize_hip, realize_tensor_plan_hip
from browsergrad_amd.jit.tensor import Session, conv1d, conv2d, conv3d, relu
from oracle import graph as G
from oracle import ops as O

F32 = np.float32


def _cnn(rng):
    s = Session()
    x = rng.standard_normal((2, 4, 13, 11)).astype(F32)
    w1 = rng.standard_normal((8, 2, 3, 3)).astype(F32)
    b1 = rng.standard_normal(8).astype(F32)
    w2 = rng.standard_normal((6, 8, 2, 2)).astype(F32)
    y = conv2d(relu(conv2d(s.from_numpy(x), s.from_numpy(w1), s.from_numpy(b1), stride=2, padding=1, groups=2)),
               s.from_numpy(w2), dilation=(1, 2))
    return s, y, (x, w1, b1, w2)


def test_conv_graph_oracle_matches_torch():
    rng = np.random.default_rng(0)
    s, y, (x, w1, b1, w2) = _cnn(rng)
    t = lambda a: torch.tensor(a, dtype=torch.float64)  # noqa: E731
    ref = F.conv2d(torch.relu(F.conv2d(t(x), t(w1), t(b1), stride=2, padding=1, groups=2)), t(w2), dilation=(1, 2))
    got = G.evaluate(y.uop, s.buffers)
    assert got.shape == tuple(ref.shape) and O.within(got, ref.numpy(), 1e-4).all()
    for fn, shape_x, shape_w, kw, tfn in (
            (conv1d, (2, 3, 17), (4, 3, 5), dict(stride=2, padding=2), F.conv1d),
            (conv3d, (1, 2, 5, 6, 4), (3, 2, 3, 2, 2), dict(padding=(1, 0, 1), dilation=(1, 1, 2)), F.conv3d)):
        xs, ws = rng.standard_normal(shape_x).astype(F32), rng.standard_normal(shape_w).astype(F32)
        s2 = Session()
        g = G.evaluate(fn(s2.from_numpy(xs), s2.from_numpy(ws), **kw).uop, s2.buffers)
        assert O.within(g, tfn(t(xs), t(ws), **kw).numpy(), 1e-4).all()


def test_plan_builder_emits_conv_steps():
    s, y, _ = _cnn(np.random.default_rng(1))
    sub = build_gpu_execution_submission(y.uop)
    steps = [st for st in sub.plan.steps if st.op.startswith("CONV")]
    assert [st.op for st in steps] == ["CONV2D", "CONV2D"]
    a = steps[0].arg
    assert (a["stride_h"], a["pad_w"], a["groups"], a["out_h"], a["has_bias"]) == (2, 1, 2, 7, True)


@pytest.mark.gpu
def test_conv_graph_on_the_walker_and_plan_route(bridge):
    rng = np.random.default_rng(2)
    s, y, _ = _cnn(rng)
    ref = G.evaluate(y.uop, s.buffers)
    gbt = GpuBufferTable(bridge)
    out = realize_hip(y.uop, s.buffers, gbt)
    assert O.within(out, ref, 1e-4).all(), O.report(out, ref, 1e-4)
    out2 = realize_tensor_plan_hip(y.uop, s.buffers, gbt)
    assert O.within(out2, ref, 1e-4).all(), O.report(out2, ref, 1e-4)
    gbt.release_all()
