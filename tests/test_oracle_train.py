"""Pins the oracle's LayerNorm backward and optimizer restatements on CPU.

Anchors outside the oracle's own formulas:
  * the reference's known answers for SGD_UPDATE, ADAMW_UPDATE_*,
    ADAM_UPDATE_* and LAYER_NORM(_BACKWARD_*) (packages/browsergrad-kernels/
    tests-browser/webgpu_real.test.ts:667-945), whose expected values the
    reference computes in double from the float32 inputs; restated here as
    data-driven float64 loops with the reference's tolerances;
  * torch.optim.SGD / Adam / AdamW run in float64 over several steps (L2
    decay folded into the gradient for SGD and Adam, decoupled for AdamW);
  * torch autograd of layer_norm in float64 for dX, dW and dB;
  * planted slips (coupled vs decoupled decay, a dropped term of dX, the
    bias correction left out) that one of the checks above must catch.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ops as O

F32 = np.float32

PARAM = np.array([1, -2, 3, -4], F32)
GRAD = np.array([0.5, -0.25, 0.75, -1], F32)
M0 = np.array([0.1, -0.2, 0.3, -0.4], F32)
V0 = np.array([0.01, 0.02, 0.03, 0.04], F32)


# ---------------------------------------------------------------- reference known answers


def test_sgd_known_answer():
    # webgpu_real.test.ts:667-711: lr 0.1, weight_decay 0.01, |err| < 1e-6
    got = O.sgd_update(PARAM, GRAD, 0.1, 0.01)
    for i in range(4):
        p, g = float(PARAM[i]), float(GRAD[i])
        assert abs(float(got[i]) - (p - 0.1 * (g + 0.01 * p))) < 1e-6


def _adam_expected(arg, decoupled):
    """The reference test's expected M / V / P loops (webgpu_real.test.ts:
    719-729 for AdamW, 794-804 for Adam): M and V stored to float32, P in double."""
    em, ev, ep = [], [], []
    for i in range(4):
        p, g = float(PARAM[i]), float(GRAD[i])
        ge = g if decoupled else g + arg["weight_decay"] * p
        m = float(F32(arg["beta1"] * float(M0[i]) + (1 - arg["beta1"]) * ge))
        v = float(F32(arg["beta2"] * float(V0[i]) + (1 - arg["beta2"]) * ge * ge))
        mh = m / (1 - arg["beta1"] ** arg["step"])
        vh = v / (1 - arg["beta2"] ** arg["step"])
        pn = p - arg["lr"] * (mh / (math.sqrt(vh) + arg["eps"]))
        if decoupled:
            pn -= arg["lr"] * arg["weight_decay"] * p
        em.append(m)
        ev.append(v)
        ep.append(float(F32(pn)))
    return em, ev, ep


ADAMW_ARG = dict(lr=0.01, beta1=0.8, beta2=0.95, eps=1e-6, weight_decay=0.02, step=3)
ADAM_ARG = dict(lr=0.02, beta1=0.75, beta2=0.9, eps=1e-6, weight_decay=0.03, step=4)


def test_adamw_known_answer():
    # webgpu_real.test.ts:713-786: M, V within 1e-6, PARAM within 1e-5
    a = ADAMW_ARG
    em, ev, ep = _adam_expected(a, decoupled=True)
    m = O.adamw_update_m(M0, GRAD, a["beta1"])
    v = O.adamw_update_v(V0, GRAD, a["beta2"])
    p = O.adamw_update_param(PARAM, m, v, a["lr"], a["beta1"], a["beta2"], a["eps"], a["step"], a["weight_decay"])
    assert np.max(np.abs(m - em)) < 1e-6
    assert np.max(np.abs(v - ev)) < 1e-6
    assert np.max(np.abs(p - ep)) < 1e-5


def test_adam_known_answer():
    # webgpu_real.test.ts:788-861
    a = ADAM_ARG
    em, ev, ep = _adam_expected(a, decoupled=False)
    m = O.adam_update_m(PARAM, GRAD, M0, a["beta1"], a["weight_decay"])
    v = O.adam_update_v(PARAM, GRAD, V0, a["beta2"], a["weight_decay"])
    p = O.adam_update_param(PARAM, m, v, a["lr"], a["beta1"], a["beta2"], a["eps"], a["step"])
    assert np.max(np.abs(m - em)) < 1e-6
    assert np.max(np.abs(v - ev)) < 1e-6
    assert np.max(np.abs(p - ep)) < 1e-5


LN_X = np.array([[1, 2, 4], [-1, 0.5, 3]], F32)
LN_W = np.array([0.75, -1.25, 1.5], F32)
LN_B = np.array([0.1, -0.2, 0.3], F32)
LN_DY = np.array([[0.25, -0.5, 1.0], [-1.5, 0.75, 0.5]], F32)


def _ln_expected(eps=1e-5):
    """webgpu_real.test.ts:873-903: per-row double loops."""
    y, dx = np.zeros((2, 3)), np.zeros((2, 3))
    dw, db = np.zeros(3), np.zeros(3)
    for r in range(2):
        xs = [float(v) for v in LN_X[r]]
        mean = sum(xs) / 3
        var = sum((v - mean) ** 2 for v in xs) / 3
        inv = 1 / math.sqrt(var + eps)
        xh = [float(F32((v - mean) * inv)) for v in xs]
        g = [float(F32(float(LN_DY[r, c]) * float(LN_W[c]))) for c in range(3)]
        sg, sgx = sum(g), sum(g[c] * xh[c] for c in range(3))
        for c in range(3):
            y[r, c] = xh[c] * float(LN_W[c]) + float(LN_B[c])
            dw[c] += float(LN_DY[r, c]) * xh[c]
            db[c] += float(LN_DY[r, c])
            dx[r, c] = (inv / 3) * (3 * g[c] - sg - xh[c] * sgx)
    return y, dx, dw, db


def test_layer_norm_forward_backward_known_answer():
    # webgpu_real.test.ts:863-945: y, dx, dw within 1e-5; db within 1e-6
    y, dx, dw, db = _ln_expected()
    assert np.max(np.abs(O.layer_norm(LN_X, LN_W, LN_B) - y)) < 1e-5
    assert np.max(np.abs(O.layer_norm_backward_input(LN_DY, LN_X, LN_W) - dx)) < 1e-5
    assert np.max(np.abs(O.layer_norm_backward_weight(LN_DY, LN_X) - dw)) < 1e-5
    assert np.max(np.abs(O.layer_norm_backward_bias(LN_DY) - db)) < 1e-6


# ---------------------------------------------------------------- torch cross-checks


def _torch_optimizer_steps(kind, p0, grads, **kw):
    p = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    opt = {"sgd": torch.optim.SGD, "adam": torch.optim.Adam, "adamw": torch.optim.AdamW}[kind]([p], **kw)
    for g in grads:
        p.grad = torch.tensor(g, dtype=torch.float64)
        opt.step()
    return p.detach().numpy()


@pytest.mark.parametrize("wd", [0.0, 0.05])
def test_optimizers_match_torch_over_steps(wd):
    rng = np.random.default_rng(5)
    p0 = rng.standard_normal(257).astype(F32)
    grads = [rng.standard_normal(257).astype(F32) for _ in range(5)]
    lr, b1, b2, eps = 0.01, 0.9, 0.99, 1e-8

    p = p0.copy()
    for g in grads:
        p = O.sgd_update(p, g, lr, wd)
    ref = _torch_optimizer_steps("sgd", p0, grads, lr=lr, weight_decay=wd)
    assert np.allclose(p, ref, rtol=1e-5, atol=1e-6)

    for kind in ("adam", "adamw"):
        p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
        for t, g in enumerate(grads, start=1):
            if kind == "adam":
                m = O.adam_update_m(p, g, m, b1, wd)
                v = O.adam_update_v(p, g, v, b2, wd)
                p = O.adam_update_param(p, m, v, lr, b1, b2, eps, t)
            else:
                m = O.adamw_update_m(m, g, b1)
                v = O.adamw_update_v(v, g, b2)
                p = O.adamw_update_param(p, m, v, lr, b1, b2, eps, t, wd)
        ref = _torch_optimizer_steps(kind, p0, grads, lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
        assert np.allclose(p, ref, rtol=1e-5, atol=1e-6), kind


def _torch_ln_grads(x, w, b, dy, eps=1e-5):
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    y = torch.nn.functional.layer_norm(xt, (x.shape[-1],), wt, bt, eps)
    y.backward(torch.tensor(dy, dtype=torch.float64))
    return xt.grad.numpy(), wt.grad.numpy(), bt.grad.numpy()


@pytest.mark.parametrize("rows,cols", [(7, 5), (33, 768), (4, 2049)])
def test_layer_norm_backward_matches_torch_autograd(rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    x = (rng.standard_normal((rows, cols)) * 2 + 0.5).astype(F32)
    w = rng.standard_normal(cols).astype(F32)
    b = rng.standard_normal(cols).astype(F32)
    dy = rng.standard_normal((rows, cols)).astype(F32)
    gx, gw, gb = _torch_ln_grads(x, w, b, dy)
    assert O.within(O.layer_norm_backward_input(dy, x, w), gx, 1e-4).all()
    assert O.within(O.layer_norm_backward_weight(dy, x), gw, 1e-4).all()
    assert O.within(O.layer_norm_backward_bias(dy), gb, 1e-4).all()


# ---------------------------------------------------------------- planted slips


def test_planted_training_slips_are_caught():
    a = ADAM_ARG
    _, _, ep = _adam_expected(a, decoupled=False)
    # coupled (Adam) vs decoupled (AdamW) weight decay
    m = O.adamw_update_m(M0, GRAD, a["beta1"])
    v = O.adamw_update_v(V0, GRAD, a["beta2"])
    wrong = O.adamw_update_param(PARAM, m, v, a["lr"], a["beta1"], a["beta2"], a["eps"], a["step"],
                                 a["weight_decay"])
    assert np.max(np.abs(wrong - ep)) > 1e-5
    # bias correction left out (step large enough that 1 - beta^step == 1)
    m = O.adam_update_m(PARAM, GRAD, M0, a["beta1"], a["weight_decay"])
    v = O.adam_update_v(PARAM, GRAD, V0, a["beta2"], a["weight_decay"])
    nocorr = O.adam_update_param(PARAM, m, v, a["lr"], a["beta1"], a["beta2"], a["eps"], 10 ** 6)
    assert np.max(np.abs(nocorr - ep)) > 1e-5
    # dX without the x_hat * sum(g * x_hat) term
    rng = np.random.default_rng(2)
    x, w, dy = (rng.standard_normal((4, 9)).astype(F32) for _ in range(3))
    gx, _, _ = _torch_ln_grads(x, w[0], np.zeros(9, F32), dy)
    inv, x_hat = O._ln_rows(x, 9, 1e-5)
    g = dy * w[0]
    dropped = (inv / F32(9)) * (F32(9) * g - g.sum(axis=1, keepdims=True))
    assert not O.within(dropped, gx, 1e-4).all()
    assert O.within(O.layer_norm_backward_input(dy, x, w[0]), gx, 1e-4).all()
