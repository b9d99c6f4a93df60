"""LayerNorm backward and optimizer updates on the HIP path against the oracle (GPU).

The optimizer kernels follow the oracle's float32 operation order with no
contraction and IEEE division / square root, so they are compared
bit-exactly.  LayerNorm backward reduces over rows or columns in another
order than NumPy's pairwise sums: dX uses the f32 abs-or-rel 1e-4 rule;
the column sums dW / dB are compared with 1e-4 abs-or-rel at moderate row
counts and, at the GPT-2 shape (8192 x 768), against float64 sums with a
bound of 1e-5 times the column's L1 mass.  The plan route runs the
reference's own test plans (webgpu_real.test.ts:667-945) with their
tolerances.
"""
from __future__ import annotations

import json
import math

import numpy as np
import pytest

from browsergrad_amd.errors import KernelError
from oracle import ops as O

pytestmark = pytest.mark.gpu

F32 = np.float32
TOL32 = 1e-4


def up(br, a):
    a = np.ascontiguousarray(a, dtype=F32)
    return br.upload(a, a.shape, "float32")


def fetch(br, h):
    y = br.to_numpy(h)
    br.release(h)
    return y


def _ulps(a, b):
    ai = np.asarray(a, F32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, F32).view(np.int32).astype(np.int64)
    return int(np.max(np.abs(ai - bi))) if ai.size else 0


# ---------------------------------------------------------------- optimizer kernels

ARGS = dict(lr=0.003, beta1=0.85, beta2=0.97, eps=1e-7, step=7)


def _oracle(op, ins, wd):
    a = ARGS
    if op == "SGD_UPDATE":
        return O.sgd_update(ins[0], ins[1], a["lr"], wd)
    if op == "ADAMW_UPDATE_M":
        return O.adamw_update_m(ins[0], ins[1], a["beta1"])
    if op == "ADAMW_UPDATE_V":
        return O.adamw_update_v(ins[0], ins[1], a["beta2"])
    if op == "ADAMW_UPDATE_PARAM":
        return O.adamw_update_param(ins[0], ins[2], ins[3], a["lr"], a["beta1"], a["beta2"], a["eps"], a["step"], wd)
    if op == "ADAM_UPDATE_M":
        return O.adam_update_m(ins[0], ins[1], ins[2], a["beta1"], wd)
    if op == "ADAM_UPDATE_V":
        return O.adam_update_v(ins[0], ins[1], ins[2], a["beta2"], wd)
    return O.adam_update_param(ins[0], ins[1], ins[2], a["lr"], a["beta1"], a["beta2"], a["eps"], a["step"])


ARITY = {"SGD_UPDATE": 2, "ADAMW_UPDATE_M": 2, "ADAMW_UPDATE_V": 2, "ADAMW_UPDATE_PARAM": 4,
         "ADAM_UPDATE_M": 3, "ADAM_UPDATE_V": 3, "ADAM_UPDATE_PARAM": 3}


@pytest.mark.parametrize("op", list(ARITY))
@pytest.mark.parametrize("n", [1, 7, 4099, (1 << 20) + 5])
@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_optimizer_update_bit_exact(bridge, rng, op, n, wd):
    ins = [rng.standard_normal(n).astype(F32) for _ in range(ARITY[op])]
    if op in ("ADAMW_UPDATE_PARAM",):
        ins[3] = np.abs(ins[3]) * F32(0.01)  # second moment >= 0
    if op == "ADAM_UPDATE_PARAM":
        ins[2] = np.abs(ins[2]) * F32(0.01)
    hs = [up(bridge, a) for a in ins]
    h = bridge.optimizer_update(op, hs, n, weight_decay=wd, **ARGS)
    y = fetch(bridge, h)
    for x in hs:
        bridge.release(x)
    ref = _oracle(op, ins, wd)
    assert y.shape == (n,)
    assert np.array_equal(y, ref), f"{op} n={n} wd={wd}: max {_ulps(y, ref)} ulp"


def test_optimizer_update_empty_and_errors(bridge):
    h0 = up(bridge, np.zeros(0, F32))
    h = bridge.optimizer_update("SGD_UPDATE", [h0, h0], 0, lr=0.1)
    assert fetch(bridge, h).size == 0
    p = up(bridge, np.ones(5, F32))
    q = up(bridge, np.ones(6, F32))
    with pytest.raises(KernelError, match="does not hold n elements"):
        bridge.optimizer_update("SGD_UPDATE", [p, q], 5, lr=0.1)
    with pytest.raises(KernelError, match="expects 4 inputs"):
        bridge.optimizer_update("ADAMW_UPDATE_PARAM", [p, p], 5, lr=0.1)
    with pytest.raises(KernelError, match="step must be >= 1"):
        bridge.optimizer_update("ADAM_UPDATE_PARAM", [p, p, p], 5, lr=0.1, step=0)
    with pytest.raises(KernelError, match="lr must be >= 0"):
        bridge.optimizer_update("SGD_UPDATE", [p, p], 5, lr=-1.0)
    with pytest.raises(KernelError, match="finite"):
        bridge.optimizer_update("ADAM_UPDATE_M", [p, p, p], 5, beta1=math.inf)
    for x in (h0, p, q):
        bridge.release(x)


def test_adamw_chain_matches_oracle_over_steps(bridge, rng):
    """Five AdamW steps with state kept resident on the device."""
    n = 300_001
    p = rng.standard_normal(n).astype(F32)
    hp, hm, hv = up(bridge, p), up(bridge, np.zeros(n, F32)), up(bridge, np.zeros(n, F32))
    m, v = np.zeros(n, F32), np.zeros(n, F32)
    kw = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.1)
    for t in range(1, 6):
        g = rng.standard_normal(n).astype(F32)
        hg = up(bridge, g)
        nm = bridge.optimizer_update("ADAMW_UPDATE_M", [hm, hg], n, step=t, **kw)
        nv = bridge.optimizer_update("ADAMW_UPDATE_V", [hv, hg], n, step=t, **kw)
        np_ = bridge.optimizer_update("ADAMW_UPDATE_PARAM", [hp, hg, nm, nv], n, step=t, **kw)
        for x in (hg, hm, hv, hp):
            bridge.release(x)
        hm, hv, hp = nm, nv, np_
        m = O.adamw_update_m(m, g, kw["beta1"])
        v = O.adamw_update_v(v, g, kw["beta2"])
        p = O.adamw_update_param(p, m, v, kw["lr"], kw["beta1"], kw["beta2"], kw["eps"], t, kw["weight_decay"])
    assert np.array_equal(fetch(bridge, hm), m)
    assert np.array_equal(fetch(bridge, hv), v)
    assert np.array_equal(fetch(bridge, hp), p)


# ---------------------------------------------------------------- LayerNorm backward kernels


# Up to 1024 columns the wavefront-per-row kernels; 4-aligned rows of 1028
# to 32768 the workgroup-per-row kernel (256 threads with 2, 4, 8 groups per
# thread, 1024 threads with 4 or 8; partial last groups); the rest the
# three-pass kernel.
@pytest.mark.parametrize("rows,cols", [(1, 1), (2, 3), (5, 100), (8, 768), (64, 1024), (3, 3000), (17, 257),
                                       (9, 1028), (5, 2048), (4, 4100), (3, 8192), (3, 12000), (2, 32768),
                                       (2, 32772), (3, 2050)])
def test_layer_norm_backward_input(bridge, rng, rows, cols):
    x = (rng.standard_normal((rows, cols)) * 3 + 1).astype(F32)
    w = rng.standard_normal(cols).astype(F32)
    dy = rng.standard_normal((rows, cols)).astype(F32)
    hx, hw, hdy = up(bridge, x), up(bridge, w), up(bridge, dy)
    y = fetch(bridge, bridge.layer_norm_backward_input(hdy, hx, hw, rows, cols, 1e-5))
    ref = O.layer_norm_backward_input(dy, x, w, 1e-5)
    assert y.shape == (rows, cols)
    assert O.within(y, ref, TOL32).all(), O.report(y, ref, TOL32)
    for h in (hx, hw, hdy):
        bridge.release(h)


# 4-aligned widths up to 1024 take the 16-byte kernel (every lane width
# 1..4 groups of 64, ragged rows and groups); the others the scalar ones.
@pytest.mark.parametrize("rows,cols", [(1, 1), (2, 3), (7, 5), (1, 4), (5, 100), (33, 260), (19, 1024), (100, 768),
                                       (517, 1030), (33, 4100), (9, 2048), (5, 12000), (3, 32768), (4, 32772),
                                       (6, 2050)])
def test_layer_norm_backward_weight_bias(bridge, rng, rows, cols):
    x = (rng.standard_normal((rows, cols)) * 2 - 0.5).astype(F32)
    dy = rng.standard_normal((rows, cols)).astype(F32)
    hx, hdy = up(bridge, x), up(bridge, dy)
    dw = fetch(bridge, bridge.layer_norm_backward_weight(hdy, hx, rows, cols, 1e-5))
    db = fetch(bridge, bridge.layer_norm_backward_bias(hdy, rows, cols))
    rw = O.layer_norm_backward_weight(dy, x, 1e-5)
    rb = O.layer_norm_backward_bias(dy)
    assert dw.shape == (cols,) and db.shape == (cols,)
    assert O.within(dw, rw, TOL32).all(), O.report(dw, rw, TOL32)
    assert O.within(db, rb, TOL32).all(), O.report(db, rb, TOL32)
    for h in (hx, hdy):
        bridge.release(h)


def test_layer_norm_backward_gpt2_shape_against_float64(bridge, rng):
    rows, cols = 8192, 768
    x = rng.standard_normal((rows, cols)).astype(F32)
    w = rng.standard_normal(cols).astype(F32)
    dy = rng.standard_normal((rows, cols)).astype(F32)
    hx, hw, hdy = up(bridge, x), up(bridge, w), up(bridge, dy)
    dx = fetch(bridge, bridge.layer_norm_backward_input(hdy, hx, hw, rows, cols, 1e-5))
    dw = fetch(bridge, bridge.layer_norm_backward_weight(hdy, hx, rows, cols, 1e-5))
    db = fetch(bridge, bridge.layer_norm_backward_bias(hdy, rows, cols))
    for h in (hx, hw, hdy):
        bridge.release(h)
    ref_dx = O.layer_norm_backward_input(dy, x, w, 1e-5)
    assert O.within(dx, ref_dx, TOL32).all(), O.report(dx, ref_dx, TOL32)
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=1, keepdims=True)
    xh = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(axis=1, keepdims=True) + 1e-5)
    terms_w = dy.astype(np.float64) * xh
    for got, terms in ((dw, terms_w), (db, dy.astype(np.float64))):
        bound = 1e-5 * np.abs(terms).sum(axis=0) + 1e-6
        err = np.abs(got - terms.sum(axis=0))
        assert np.all(err <= bound), float(np.max(err / bound))


def test_layer_norm_backward_columns_repeat_across_shapes(bridge, rng):
    """Column sums over 1 to 1024 partial rows (16-byte and 4-byte pass-1
    kernels, 256 to 1024 columns, single-block and ragged cases), called in a
    row twice: each must match float64 sums and repeat bit for bit, so a sum
    whose order depended on scheduling, or state left by an earlier call,
    would show."""
    shapes = [(16, 768), (256, 768), (300, 512), (4352, 256), (16384, 1024), (5, 4), (33, 260)]
    first = {}
    for rep in range(2):
        for rows, cols in shapes:
            r = np.random.default_rng(rows * 7 + cols)
            x = (r.standard_normal((rows, cols)) * 1.5 + 0.25).astype(F32)
            dy = r.standard_normal((rows, cols)).astype(F32)
            hx, hdy = up(bridge, x), up(bridge, dy)
            dw = fetch(bridge, bridge.layer_norm_backward_weight(hdy, hx, rows, cols, 1e-5))
            db = fetch(bridge, bridge.layer_norm_backward_bias(hdy, rows, cols))
            bridge.release(hx)
            bridge.release(hdy)
            if rep == 0:
                # float64 sums, bound 1e-5 x the column's L1 mass (as at the
                # GPT-2 shape: 16384-row f32 sums drift past 1e-4 relative
                # where the column nearly cancels).
                x64 = x.astype(np.float64)
                mu = x64.mean(axis=1, keepdims=True)
                xh = (x64 - mu) / np.sqrt(((x64 - mu) ** 2).mean(axis=1, keepdims=True) + 1e-5)
                for got, terms in ((dw, dy.astype(np.float64) * xh), (db, dy.astype(np.float64))):
                    bound = 1e-5 * np.abs(terms).sum(axis=0) + 1e-6
                    err = np.abs(got - terms.sum(axis=0))
                    assert np.all(err <= bound), (rows, cols, float(np.max(err / bound)))
                first[(rows, cols)] = (dw, db)
            else:
                assert np.array_equal(dw, first[(rows, cols)][0]), (rows, cols)
                assert np.array_equal(db, first[(rows, cols)][1]), (rows, cols)


def test_layer_norm_backward_errors(bridge):
    x = up(bridge, np.ones((2, 3), F32))
    w = up(bridge, np.ones(4, F32))
    with pytest.raises(KernelError, match="weight"):
        bridge.layer_norm_backward_input(x, x, w, 2, 3, 1e-5)
    with pytest.raises(KernelError, match="eps"):
        bridge.layer_norm_backward_weight(x, x, 2, 3, 0.0)
    with pytest.raises(KernelError, match="rows\\*cols"):
        bridge.layer_norm_backward_bias(x, 3, 3)
    h16 = bridge.upload(np.ones((2, 3), np.float16), (2, 3), "float16")
    with pytest.raises(KernelError, match="float32"):
        bridge.layer_norm_backward_bias(h16, 2, 3)
    for h in (x, w, h16):
        bridge.release(h)


# ---------------------------------------------------------------- the reference's test plans


def _plan(steps, root):
    buffers = [{"value_id": s["value_id"], "op": s["op"], "shape": s["shape"], "dtype": "float32",
                "bytes": 4 * int(np.prod(s["shape"])), "first_step": s["step"], "last_step": root,
                "materialize": s["value_id"] == root} for s in steps]
    return {"steps": steps, "buffers": buffers, "root_id": root, "materialization_boundary": "root",
            "peak_live_bytes": 0, "has_custom_ops": False}


def _buf(i, shape):
    return {"step": i, "value_id": i, "op": "BUFFER", "input_ids": [], "shape": list(shape), "dtype": "float32"}


def _load(i, src, shape):
    return {"step": i, "value_id": i, "op": "LOAD", "input_ids": [src], "shape": list(shape), "dtype": "float32"}


def _run(bridge, plan, arrays):
    data = [{"value_id": i, "data": np.ascontiguousarray(a, F32).tobytes()} for i, a in enumerate(arrays)]
    return np.frombuffer(bridge.run_tensor_plan(plan, data, "float32"), F32)


PARAM = np.array([1, -2, 3, -4], F32)
GRAD = np.array([0.5, -0.25, 0.75, -1], F32)
M0 = np.array([0.1, -0.2, 0.3, -0.4], F32)
V0 = np.array([0.01, 0.02, 0.03, 0.04], F32)


def test_plan_sgd_update(bridge):
    # webgpu_real.test.ts:667-711
    steps = [_buf(0, [4]), _buf(1, [4]), _load(2, 0, [4]), _load(3, 1, [4]),
             {"step": 4, "value_id": 4, "op": "SGD_UPDATE", "input_ids": [2, 3], "shape": [4], "dtype": "float32",
              "arg": {"lr": 0.1, "weight_decay": 0.01}}]
    y = _run(bridge, _plan(steps, 4), [PARAM, GRAD])
    for i in range(4):
        p, g = float(PARAM[i]), float(GRAD[i])
        assert abs(float(y[i]) - (p - 0.1 * (g + 0.01 * p))) < 1e-6
    assert np.array_equal(y, O.sgd_update(PARAM, GRAD, 0.1, 0.01))


def _adam_plan(kind, root_op, root_inputs, arg):
    if kind == "adamw":
        m_step = {"op": "ADAMW_UPDATE_M", "input_ids": [6, 5]}
        v_step = {"op": "ADAMW_UPDATE_V", "input_ids": [7, 5]}
    else:
        m_step = {"op": "ADAM_UPDATE_M", "input_ids": [4, 5, 6]}
        v_step = {"op": "ADAM_UPDATE_V", "input_ids": [4, 5, 7]}
    steps = [_buf(i, [4]) for i in range(4)] + [_load(4 + i, i, [4]) for i in range(4)]
    steps.append({"step": 8, "value_id": 8, "shape": [4], "dtype": "float32", "arg": arg, **m_step})
    steps.append({"step": 9, "value_id": 9, "shape": [4], "dtype": "float32", "arg": arg, **v_step})
    steps.append({"step": 10, "value_id": 10, "op": root_op, "input_ids": root_inputs, "shape": [4],
                  "dtype": "float32", "arg": arg})
    return _plan(steps, 10)


def test_plan_adamw_roots(bridge):
    # webgpu_real.test.ts:713-786
    arg = {"lr": 0.01, "beta1": 0.8, "beta2": 0.95, "eps": 1e-6, "weight_decay": 0.02, "step": 3}
    ins = [PARAM, GRAD, M0, V0]
    m = _run(bridge, _adam_plan("adamw", "ADAMW_UPDATE_M", [6, 5], arg), ins)
    v = _run(bridge, _adam_plan("adamw", "ADAMW_UPDATE_V", [7, 5], arg), ins)
    p = _run(bridge, _adam_plan("adamw", "ADAMW_UPDATE_PARAM", [4, 5, 8, 9], arg), ins)
    em = O.adamw_update_m(M0, GRAD, 0.8)
    ev = O.adamw_update_v(V0, GRAD, 0.95)
    ep = O.adamw_update_param(PARAM, em, ev, 0.01, 0.8, 0.95, 1e-6, 3, 0.02)
    assert np.array_equal(m, em) and np.array_equal(v, ev) and np.array_equal(p, ep)
    for i in range(4):
        pp, g = float(PARAM[i]), float(GRAD[i])
        mm = 0.8 * float(M0[i]) + 0.2 * g
        vv = 0.95 * float(V0[i]) + 0.05 * g * g
        mh, vh = mm / (1 - 0.8 ** 3), vv / (1 - 0.95 ** 3)
        pe = pp - 0.01 * (mh / (math.sqrt(vh) + 1e-6)) - 0.01 * 0.02 * pp
        assert abs(float(m[i]) - mm) < 1e-6 and abs(float(v[i]) - vv) < 1e-6 and abs(float(p[i]) - pe) < 1e-5


def test_plan_adam_roots(bridge):
    # webgpu_real.test.ts:788-861
    arg = {"lr": 0.02, "beta1": 0.75, "beta2": 0.9, "eps": 1e-6, "weight_decay": 0.03, "step": 4}
    ins = [PARAM, GRAD, M0, V0]
    m = _run(bridge, _adam_plan("adam", "ADAM_UPDATE_M", [4, 5, 6], arg), ins)
    v = _run(bridge, _adam_plan("adam", "ADAM_UPDATE_V", [4, 5, 7], arg), ins)
    p = _run(bridge, _adam_plan("adam", "ADAM_UPDATE_PARAM", [4, 8, 9], arg), ins)
    em = O.adam_update_m(PARAM, GRAD, M0, 0.75, 0.03)
    ev = O.adam_update_v(PARAM, GRAD, V0, 0.9, 0.03)
    ep = O.adam_update_param(PARAM, em, ev, 0.02, 0.75, 0.9, 1e-6, 4)
    assert np.array_equal(m, em) and np.array_equal(v, ev) and np.array_equal(p, ep)
    for i in range(4):
        pp, g = float(PARAM[i]), float(GRAD[i])
        ge = g + 0.03 * pp
        mm = 0.75 * float(M0[i]) + 0.25 * ge
        vv = 0.9 * float(V0[i]) + 0.1 * ge * ge
        mh, vh = mm / (1 - 0.75 ** 4), vv / (1 - 0.9 ** 4)
        pe = pp - 0.02 * (mh / (math.sqrt(vh) + 1e-6))
        assert abs(float(m[i]) - mm) < 1e-6 and abs(float(v[i]) - vv) < 1e-6 and abs(float(p[i]) - pe) < 1e-5


LN_X = np.array([[1, 2, 4], [-1, 0.5, 3]], F32)
LN_W = np.array([0.75, -1.25, 1.5], F32)
LN_B = np.array([0.1, -0.2, 0.3], F32)
LN_DY = np.array([[0.25, -0.5, 1.0], [-1.5, 0.75, 0.5]], F32)


def _ln_plan(root_op, shape, inputs, arg=None):
    arg = arg if arg is not None else {"normalized_shape": [3], "rows": 2, "cols": 3, "eps": 1e-5}
    steps = [_buf(0, [2, 3]), _buf(1, [3]), _buf(2, [3]), _buf(3, [2, 3]),
             _load(4, 0, [2, 3]), _load(5, 1, [3]), _load(6, 2, [3]), _load(7, 3, [2, 3]),
             {"step": 8, "value_id": 8, "op": root_op, "input_ids": inputs, "shape": shape, "dtype": "float32",
              "arg": arg}]
    return _plan(steps, 8)


def test_plan_layer_norm_forward_and_backward_roots(bridge):
    # webgpu_real.test.ts:863-945 (y, dx, dw within 1e-5; db within 1e-6)
    ins = [LN_X, LN_W, LN_B, LN_DY]
    y = _run(bridge, _ln_plan("LAYER_NORM", [2, 3], [4, 5, 6]), ins)
    dx = _run(bridge, _ln_plan("LAYER_NORM_BACKWARD_INPUT", [2, 3], [7, 4, 5]), ins)
    dw = _run(bridge, _ln_plan("LAYER_NORM_BACKWARD_WEIGHT", [3], [7, 4]), ins)
    db = _run(bridge, _ln_plan("LAYER_NORM_BACKWARD_BIAS", [3], [7]), ins)
    ey, edx, edw, edb = np.zeros((2, 3)), np.zeros((2, 3)), np.zeros(3), np.zeros(3)
    for r in range(2):
        xs = [float(v) for v in LN_X[r]]
        mean = sum(xs) / 3
        inv = 1 / math.sqrt(sum((v - mean) ** 2 for v in xs) / 3 + 1e-5)
        xh = [(v - mean) * inv for v in xs]
        g = [float(LN_DY[r, c]) * float(LN_W[c]) for c in range(3)]
        sg, sgx = sum(g), sum(g[c] * xh[c] for c in range(3))
        for c in range(3):
            ey[r, c] = xh[c] * float(LN_W[c]) + float(LN_B[c])
            edx[r, c] = (inv / 3) * (3 * g[c] - sg - xh[c] * sgx)
            edw[c] += float(LN_DY[r, c]) * xh[c]
            edb[c] += float(LN_DY[r, c])
    assert np.max(np.abs(y - ey.ravel())) < 1e-5
    assert np.max(np.abs(dx - edx.ravel())) < 1e-5
    assert np.max(np.abs(dw - edw)) < 1e-5
    assert np.max(np.abs(db - edb)) < 1e-6


def test_plan_argument_rules(bridge):
    ins = [PARAM, GRAD, M0, V0]
    # Adam defaults every field (lr 0.001, betas 0.9 / 0.999, eps 1e-8, step 1)
    p = _run(bridge, _adam_plan("adam", "ADAM_UPDATE_PARAM", [4, 8, 9], {}), ins)
    em = O.adam_update_m(PARAM, GRAD, M0, 0.9)
    ev = O.adam_update_v(PARAM, GRAD, V0, 0.999)
    assert np.array_equal(p, O.adam_update_param(PARAM, em, ev, 0.001, 0.9, 0.999, 1e-8, 1))
    # camelCase weightDecay
    steps = [_buf(0, [4]), _buf(1, [4]),
             {"step": 2, "value_id": 2, "op": "SGD_UPDATE", "input_ids": [0, 1], "shape": [4], "dtype": "float32",
              "arg": {"lr": 0.5, "weightDecay": 0.25}}]
    assert np.array_equal(_run(bridge, _plan(steps, 2), [PARAM, GRAD]), O.sgd_update(PARAM, GRAD, 0.5, 0.25))
    bad = json.loads(json.dumps(steps))
    bad[2]["arg"] = {"weight_decay": 0.1}
    with pytest.raises(KernelError, match="SGD_UPDATE.lr must be a finite number"):
        _run(bridge, _plan(bad, 2), [PARAM, GRAD])
    bad[2]["arg"] = {"lr": -0.1}
    with pytest.raises(KernelError, match="SGD_UPDATE.lr must be >= 0"):
        _run(bridge, _plan(bad, 2), [PARAM, GRAD])
    # AdamW requires beta1, beta2 and step
    with pytest.raises(KernelError, match="ADAMW_UPDATE_M.beta1 must be a finite number"):
        _run(bridge, _adam_plan("adamw", "ADAMW_UPDATE_M", [6, 5], {"beta2": 0.9, "step": 1}), ins)
    with pytest.raises(KernelError, match="ADAMW_UPDATE_M.step must be an integer"):
        _run(bridge, _adam_plan("adamw", "ADAMW_UPDATE_M", [6, 5], {"beta1": 0.9, "beta2": 0.9}), ins)
    with pytest.raises(KernelError, match="step must be >= 1"):
        _run(bridge, _adam_plan("adam", "ADAM_UPDATE_M", [4, 5, 6], {"step": 0}), ins)
    # LayerNorm argument and shape rules
    lnin = [LN_X, LN_W, LN_B, LN_DY]
    with pytest.raises(KernelError, match="cols must equal normalized_shape numel"):
        _run(bridge, _ln_plan("LAYER_NORM_BACKWARD_BIAS", [3], [7],
                              {"normalized_shape": [4], "rows": 2, "cols": 3}), lnin)
    with pytest.raises(KernelError, match="normalized_shape must be non-empty"):
        _run(bridge, _ln_plan("LAYER_NORM_BACKWARD_BIAS", [3], [7],
                              {"normalized_shape": [], "rows": 2, "cols": 3}), lnin)
    with pytest.raises(KernelError, match="LAYER_NORM_BACKWARD_WEIGHT.output shape mismatch at dim 0"):
        _run(bridge, _ln_plan("LAYER_NORM_BACKWARD_WEIGHT", [2], [7, 4]), lnin)
    with pytest.raises(KernelError, match="LAYER_NORM_BACKWARD_INPUT.weight expected rank 1"):
        _run(bridge, _ln_plan("LAYER_NORM_BACKWARD_INPUT", [2, 3], [7, 4, 4]), lnin)
    # eps defaults to 1e-5 when absent
    dx = _run(bridge, _ln_plan("LAYER_NORM_BACKWARD_INPUT", [2, 3], [7, 4, 5],
                               {"normalizedShape": [3], "rows": 2, "cols": 3}), lnin)
    ref = O.layer_norm_backward_input(LN_DY, LN_X, LN_W, 1e-5).ravel()
    assert O.within(dx, ref, TOL32).all()


def test_plan_adamw_param_root_fused_matches_unfused(bridge, rng):
    """A PARAM root whose M and V inputs are read by nothing else runs as one
    fused pass; its result equals the three-step chain bit for bit, and a
    plan where M has a second reader (no fusion) gives the same bytes."""
    n = (1 << 20) + 3
    p, g, m0 = (rng.standard_normal(n).astype(F32) for _ in range(3))
    v0 = (np.abs(rng.standard_normal(n)) * 0.01).astype(F32)
    arg = {"lr": 3e-4, "beta1": 0.9, "beta2": 0.95, "eps": 1e-8, "weight_decay": 0.1, "step": 12}
    ins = [p, g, m0, v0]

    def plan(extra_reader):
        steps = [_buf(i, [n]) for i in range(4)] + [_load(4 + i, i, [n]) for i in range(4)]
        steps.append({"step": 8, "value_id": 8, "op": "ADAMW_UPDATE_M", "input_ids": [6, 5], "shape": [n],
                      "dtype": "float32", "arg": arg})
        steps.append({"step": 9, "value_id": 9, "op": "ADAMW_UPDATE_V", "input_ids": [7, 5], "shape": [n],
                      "dtype": "float32", "arg": arg})
        root = 10
        if extra_reader:  # a dead second reader of M keeps the chain unfused
            steps.append({"step": 10, "value_id": 10, "op": "ADD", "input_ids": [8, 8], "shape": [n],
                          "dtype": "float32"})
            root = 11
        steps.append({"step": root, "value_id": root, "op": "ADAMW_UPDATE_PARAM", "input_ids": [4, 5, 8, 9],
                      "shape": [n], "dtype": "float32", "arg": arg})
        return _plan(steps, root)

    bridge.flushProfiles()
    fused = _run(bridge, plan(False), ins)
    labels = [q["label"] for q in bridge.flushProfiles()["passProfiles"]]
    unfused = _run(bridge, plan(True), ins)
    labels2 = [q["label"] for q in bridge.flushProfiles()["passProfiles"]]
    em = O.adamw_update_m(m0, g, 0.9)
    ev = O.adamw_update_v(v0, g, 0.95)
    ep = O.adamw_update_param(p, em, ev, 3e-4, 0.9, 0.95, 1e-8, 12, 0.1)
    assert np.array_equal(fused, ep) and np.array_equal(unfused, ep)
    if bridge.profiling:
        assert "adamw_update_fused" in labels and "adamw_update_m" not in labels
        assert "adamw_update_fused" not in labels2 and "adamw_update_m" in labels2


@pytest.mark.parametrize("wd_m,wd_v", [(0.0, 0.0), (0.03, 0.03), (0.03, 0.0)])
def test_plan_adam_param_root_fused_matches_oracle(bridge, rng, wd_m, wd_v):
    """The Adam chain (M and V over (param, grad, moment), PARAM over
    (param, m', v')) fuses the same way; each moment step keeps its own
    weight decay."""
    n = 300_007
    p, g, m0 = (rng.standard_normal(n).astype(F32) for _ in range(3))
    v0 = (np.abs(rng.standard_normal(n)) * 0.01).astype(F32)
    base = {"lr": 2e-3, "beta1": 0.8, "beta2": 0.99, "eps": 1e-7, "step": 5}
    steps = [_buf(i, [n]) for i in range(4)] + [_load(4 + i, i, [n]) for i in range(4)]
    steps.append({"step": 8, "value_id": 8, "op": "ADAM_UPDATE_M", "input_ids": [4, 5, 6], "shape": [n],
                  "dtype": "float32", "arg": {**base, "weight_decay": wd_m}})
    steps.append({"step": 9, "value_id": 9, "op": "ADAM_UPDATE_V", "input_ids": [4, 5, 7], "shape": [n],
                  "dtype": "float32", "arg": {**base, "weight_decay": wd_v}})
    steps.append({"step": 10, "value_id": 10, "op": "ADAM_UPDATE_PARAM", "input_ids": [4, 8, 9], "shape": [n],
                  "dtype": "float32", "arg": base})
    bridge.flushProfiles()
    got = _run(bridge, _plan(steps, 10), [p, g, m0, v0])
    labels = [q["label"] for q in bridge.flushProfiles()["passProfiles"]]
    em = O.adam_update_m(p, g, m0, 0.8, wd_m)
    ev = O.adam_update_v(p, g, v0, 0.99, wd_v)
    assert np.array_equal(got, O.adam_update_param(p, em, ev, 2e-3, 0.8, 0.99, 1e-7, 5))
    if bridge.profiling:
        assert labels.count("adam_update_fused") == 1 and "adam_update_m" not in labels
