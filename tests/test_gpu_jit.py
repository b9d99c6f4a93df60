"""The walker and the plan route on the GPU, against the graph oracle.

Parity bar (BASELINE / the reference's abs-or-rel rule,
semantic-core/src/kernel/attention-forward-model.ts:25-29): 1e-4 for float32
results of float32 graphs, 2e-2 where float16 arithmetic is involved.
Residency counts mirror
packages/browsergrad-jit/tests-integration/webgpu_realizer.test.ts:1026-1112.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

from browsergrad_amd.errors import KernelError
from browsergrad_amd.jit import configs
from browsergrad_amd.jit.amp import insert_cast_pass
from browsergrad_amd.jit.buffers import GpuBufferTable
from browsergrad_amd.jit.gpu_plan import build_gpu_execution_submission
from browsergrad_amd.jit.ir import toposort
from browsergrad_amd.jit.realize import (
    materialize_gpu_buffer, realize_hip, realize_tensor_plan_hip, realize_tensor_plan_hip_resident,
)
from browsergrad_amd.jit.tensor import Session, layer_norm, softmax
from oracle import graph as G
from oracle import ops as O

pytestmark = pytest.mark.gpu


@pytest.fixture
def table(bridge):
    gbt = GpuBufferTable(bridge)
    yield gbt
    gbt.release_all()


def _check(out, ref, tol):
    assert out.shape == ref.shape and out.dtype == ref.dtype, (out.shape, out.dtype, ref.shape, ref.dtype)
    rep = O.report(out.astype(np.float32), ref.astype(np.float32), tol)
    assert rep["pass"], rep


CASES = [("c1", 1.0, {}, 1e-4), ("c2", 1 / 16, {}, 1e-4), ("c3", 1 / 16, {"amp": False}, 1e-4),
         ("c3", 1 / 16, {}, 2e-2), ("c4", 1 / 16, {}, 2e-2), ("c5", 1 / 8, {}, 2e-2)]


@pytest.mark.parametrize("rewrites", [True, False], ids=["hip_rewrites", "reference_ops"])
@pytest.mark.parametrize("name,scale,kw,tol", CASES, ids=[f"{c[0]}{'_fp32' if c[2] else ''}" for c in CASES])
def test_config_parity_small(bridge, table, name, scale, kw, tol, rewrites):
    print(f"[case] {name} scale={scale} {kw} rewrites={rewrites}", flush=True)
    s, y = configs.BUILDERS[name](scale=scale, **kw)
    ref = G.evaluate(y.uop, s.buffers)
    alive = bridge.aliveHandleCount()
    out = realize_hip(y.uop, s.buffers, table, hip_rewrites=rewrites)
    _check(out, ref, tol)
    # every intermediate was released: only the table's seed buffers remain
    assert bridge.aliveHandleCount() == alive + table.stats()["handles_alive"]


def test_config_c4_bf16_extension(bridge, table):
    s, y = configs.c4(scale=1 / 16, dtype="bfloat16")
    ref = G.evaluate(y.uop, s.buffers)
    out = realize_hip(y.uop, s.buffers, table)
    assert out.dtype == np.uint16  # bfloat16 bit patterns
    _check(O.bf16_bits_to_f32(out), ref.astype(np.float32), 2e-2)


def test_full_size_c2_c3(bridge, table):
    for name, kw, tol in (("c2", {}, 1e-4), ("c3", {}, 2e-2)):
        print(f"[case] {name} full {kw}", flush=True)
        s, y = configs.BUILDERS[name](**kw)
        ref = G.evaluate(y.uop, s.buffers)
        out = realize_hip(y.uop, s.buffers, table)
        _check(out, ref, tol)
        table.release_all()


def test_full_size_c3_fp32_against_f64_truth(bridge, table):
    """K = 4096 float32 dot products: near-zero outputs put both the GPU and
    numpy above the 1e-4 absolute bar, so (per the parity rule for fp32 C3)
    both are measured against a float64 truth.  The GPU must stay inside the
    probabilistic rounding bound of a K-term float32 sum,
    |y - truth| <= 2 sqrt(K) u (|x| |w| + |b|) with u = 2^-24, elementwise;
    numpy's own float32 error is reported beside it."""
    s, y = configs.c3(amp=False)
    ref = G.evaluate(y.uop, s.buffers)
    out = realize_hip(y.uop, s.buffers, table)
    x, w, b = (s.buffers.get(n.inputs[0].arg).astype(np.float64) for n in toposort(y.uop) if n.op == "LOAD")
    truth = x @ w + b
    k = x.shape[1]
    bound = 2.0 * np.sqrt(k) * 2.0 ** -24 * (np.abs(x) @ np.abs(w) + np.abs(b))
    err_gpu = np.abs(out - truth)
    err_np = np.abs(ref - truth)
    print(f"[c3 fp32] max err gpu {err_gpu.max():.3e}  numpy f32 {err_np.max():.3e}  "
          f"min bound {bound.min():.3e}", flush=True)
    assert (err_gpu <= bound).all(), int((err_gpu > bound).sum())
    assert O.report(out, truth, 1e-4)["normwise"] < 1e-5


def test_full_size_c4_heads(bridge, table):
    s, y = configs.c4()
    out = realize_hip(y.uop, s.buffers, table)
    q, k, v = (s.buffers.get(n.inputs[0].arg) for n in toposort(y.uop)
               if n.op == "LOAD" and n.dtype == "float16")
    for bh in ((0, 0), (7, 15), (3, 9)):
        ref = O.sdpa_amp(q[bh][None, None], k[bh][None, None], v[bh][None, None], 0.125, True)[0, 0]
        _check(out[bh], ref, 2e-2)


def test_full_size_c5(bridge, table):
    s, y = configs.c5()
    ref = G.evaluate(y.uop, s.buffers)
    out = realize_hip(y.uop, s.buffers, table)
    _check(out, ref, 2e-2)


# ---- residency (webgpu_realizer.test.ts:1026-1112) ---------------------------------

def test_single_matmul_residency(bridge):
    rng = np.random.RandomState(0)
    a_np = rng.uniform(-1, 1, size=(3, 4)).astype(np.float32)
    b_np = rng.uniform(-1, 1, size=(4, 5)).astype(np.float32)
    s = Session()
    a, b = s.from_numpy(a_np), s.from_numpy(b_np)
    gbt = GpuBufferTable(bridge)
    c0 = dict(bridge.counters)
    y = realize_hip((a @ b).uop, s.buffers, gbt)
    d = {k: bridge.counters[k] - c0[k] for k in c0}
    assert np.max(np.abs(y - a_np @ b_np)) < 1e-6
    assert (d["upload"], d["matmul"], d["materialize"]) == (2, 1, 1)
    gbt.release_all()


def test_chained_matmul_residency(bridge):
    rng = np.random.RandomState(1)
    xs = [rng.uniform(-1, 1, size=sh).astype(np.float32) for sh in ((2, 3), (3, 4), (4, 5))]
    s = Session()
    x, w1, w2 = (s.from_numpy(t) for t in xs)
    gbt = GpuBufferTable(bridge)
    c0 = dict(bridge.counters)
    y = realize_hip(((x @ w1) @ w2).uop, s.buffers, gbt)
    d = {k: bridge.counters[k] - c0[k] for k in c0}
    assert np.max(np.abs(y - (xs[0] @ xs[1]) @ xs[2])) < 1e-5
    assert (d["upload"], d["matmul"], d["materialize"], d["release"]) == (3, 2, 1, 2)
    assert gbt.stats()["handles_alive"] == 3
    # second call: no re-upload
    realize_hip(((x @ w1) @ w2).uop, s.buffers, gbt)
    assert bridge.counters["upload"] - c0["upload"] == 3
    gbt.release_all()


# ---- plan route --------------------------------------------------------------------

PLAN_CASES = [("c1", 1.0, {}, 1e-4), ("c2", 1 / 16, {}, 1e-4), ("c3", 1 / 16, {"amp": False}, 1e-4),
              ("c3", 1 / 16, {}, 2e-2), ("c4", 1 / 8, {}, 2e-2), ("c5", 1 / 4, {}, 2e-2)]
PLAN_IDS = ["c1", "c2", "c3_fp32", "c3", "c4", "c5"]
# Kernel launches (profile scopes) of each config's plan after the
# executor's plan-level fusion: GEMM + bias (+ relu / residual) epilogues,
# one fused program for elementwise chains (+ trailing reduction), one
# attention kernel for the SDPA steps.
PLAN_LAUNCHES = {
    "c1": {"gemm_f32": 2},
    "c2": {"fused_reduce": 1},
    "c3_fp32": {"gemm_f32": 1},
    "c3": {"gemm_a_cast": 1, "gemm_b_cast": 1, "gemm_f16": 1},
    "c4": {"attention_f16": 1},
}


@pytest.mark.parametrize("name,scale,kw,tol", PLAN_CASES, ids=PLAN_IDS)
def test_plan_route_configs(bridge, table, name, scale, kw, tol):
    s, y = configs.BUILDERS[name](scale=scale, **kw)
    ref = G.evaluate(y.uop, s.buffers)
    alive = bridge.aliveHandleCount()
    bridge.set_profiling(True)
    n0 = len(bridge.flushProfiles()["passProfiles"])  # the list accumulates over the context's life
    try:
        out = realize_tensor_plan_hip(y.uop, s.buffers, table)
        labels = [p["label"] for p in bridge.flushProfiles()["passProfiles"][n0:]]
    finally:
        bridge.set_profiling(False)
    _check(out, ref, tol)
    assert bridge.aliveHandleCount() == alive  # plan inputs were host data, all released
    counts = {lb: labels.count(lb) for lb in set(labels)}
    key = PLAN_IDS[PLAN_CASES.index((name, scale, kw, tol))]
    if key in PLAN_LAUNCHES:
        assert counts == PLAN_LAUNCHES[key], counts
    else:  # c5: one attention, four GEMMs with their epilogues, two LayerNorms
        assert counts.get("attention_f16") == 1 and counts.get("gemm_f16") == 4, counts
        assert counts.get("layer_norm") == 2 and "softmax" not in counts and "fused_reduce" not in counts, counts
        assert counts.get("fused_elementwise", 0) == 1, counts  # the GELU program


@pytest.mark.parametrize("shapes", [((1, 2, 5, 4), (1, 2, 3, 4), (1, 2, 3, 6)),
                                    ((1, 2, 5, 4), (1, 1, 4, 4), (1, 1, 4, 4))],
                         ids=["dv_ne_dk", "broadcast_k_heads_sk_eq_d"])
def test_plan_route_unfusable_amp_sdpa(bridge, table, rng, shapes):
    """Autocast SDPA graphs the attention kernel does not take (value depth
    != key depth; one key head against two query heads with sk == d): the
    plan route runs their steps unfused and matches the graph oracle."""
    from browsergrad_amd.jit.tensor import autocast, scaled_dot_product_attention
    s = Session()
    q, k, v = (s.from_numpy(rng.standard_normal(sh, dtype=np.float32)) for sh in shapes)
    with autocast("float16"):
        y = scaled_dot_product_attention(q, k, v)
    ref = G.evaluate(y.uop, s.buffers)
    out = realize_tensor_plan_hip(y.uop, s.buffers, table)
    _check(out, ref, 2e-2)


def test_plan_route_semantic_and_resident(bridge, table):
    s, y = configs.c1(scale=1.0)
    ref = G.evaluate(y.uop, s.buffers)
    out = realize_tensor_plan_hip(y.uop, s.buffers, table)  # PERMUTE steps -> semantic route
    _check(out, ref, 1e-4)
    bid = realize_tensor_plan_hip_resident(y.uop, s.buffers, table)
    h = table.get(bid)
    assert bridge.semanticTensorPlanExecutionTrace(h)["preparation"]["requests"][0]["axes"] == [1, 0]
    got = materialize_gpu_buffer(bid, shape=y.shape, dtype="float32", buffers=s.buffers, gpu_buffer_table=table)
    _check(got, ref, 1e-4)
    assert np.array_equal(s.buffers.get(bid), got)


def test_plan_softmax_layernorm_reduce_broadcast(bridge, table, rng):
    s = Session()
    x = s.from_numpy(rng.standard_normal((4, 6, 40), dtype=np.float32))
    w = s.from_numpy(rng.standard_normal((40,), dtype=np.float32))
    b = s.from_numpy(rng.standard_normal((40,), dtype=np.float32))
    graphs = [
        softmax(x),
        layer_norm(x, 40, w, b),
        x.sum(axis=0),
        x.mean(axis=(0, 2), keepdims=True),
        x.sum(),
        x.permute(2, 0, 1),
        x + w,
        (x * x).max(axis=1),
    ]
    for gr in graphs:
        ref = G.evaluate(gr.uop, s.buffers)
        out = realize_tensor_plan_hip(gr.uop, s.buffers, table)
        _check(out, ref.astype(np.float32) if ref.dtype == np.float64 else ref, 1e-4)
        out2 = realize_hip(gr.uop, s.buffers, table)
        _check(out2, ref, 1e-4)


def _plan_for(y):
    sub = build_gpu_execution_submission(insert_cast_pass(y.uop))
    return sub.plan_summary(), sub.semantic_request_summary()


def test_plan_executor_refusals(bridge, rng):
    s = Session()
    a = s.from_numpy(rng.standard_normal((3, 4), dtype=np.float32))
    plan, req = _plan_for(a.T)
    data = {"value_id": 0, "data": s.buffers.get(toposort(a.uop)[0].arg).tobytes()}
    with pytest.raises(KernelError, match="valid JSON"):
        bridge.run_tensor_plan("{not json", [data], "float32")
    bad = json.loads(json.dumps(plan))
    bad["steps"][1]["input_ids"] = [7]
    with pytest.raises(KernelError, match="before production"):
        bridge.run_tensor_plan(bad, [data], "float32")
    with pytest.raises(KernelError, match="missing BUFFER input"):
        bridge.run_tensor_plan(plan, [], "float32")
    conv = json.loads(json.dumps(plan))
    conv["steps"][2]["op"] = "CONV2D"
    with pytest.raises(KernelError, match="CONV2D"):
        bridge.run_tensor_plan(conv, [data], "float32")
    # semantic table must match the PERMUTE steps one to one
    with pytest.raises(KernelError, match="expected exactly 1 request"):
        bridge.run_tensor_plan_semantic(plan, {**req, "requests": []}, [data], "float32")
    legacy_arg = json.loads(json.dumps(plan))
    legacy_arg["steps"][2]["arg"] = {"axes": [1, 0]}
    with pytest.raises(KernelError, match="erase legacy arg"):
        bridge.run_tensor_plan_semantic(legacy_arg, req, [data], "float32")
    # a resident root that is only a view of an input is refused
    plan_load, _ = _plan_for(a)
    with pytest.raises(KernelError, match="aliases an input buffer"):
        bridge.run_tensor_plan_resident(plan_load, [data], "float32")
    assert bridge.aliveHandleCount() >= 0


# ---- typed ATTENTION_FORWARD (_framework_contracts.py:2792-2932) -------------------

def test_attention_forward_typed(bridge, table, rng):
    from browsergrad_amd.errors import ShapeError
    from browsergrad_amd.jit.attention_forward import (
        execute_attention_forward_hip, infer_attention_forward_contract, validate_attention_forward_node,
    )
    from browsergrad_amd.jit.tensor import attention_forward
    s = Session()
    arrs = [rng.standard_normal((2, 3, 37, 64), dtype=np.float32) for _ in range(3)]
    q, k, v = (s.from_numpy(a) for a in arrs)
    y = attention_forward(q, k, v)
    ref = G.evaluate(y.uop, s.buffers)
    alive = bridge.aliveHandleCount()
    out = realize_hip(y.uop, s.buffers, table)
    _check(out, ref, 1e-4)
    c = validate_attention_forward_node(y.uop)
    _check(execute_attention_forward_hip(c, tuple(arrs), bridge), ref, 1e-4)
    assert bridge.aliveHandleCount() == alive + table.stats()["handles_alive"]
    # Scores that overflow float32 surface as a non-finite output and are refused.
    big = np.full((1, 1, 2, 4), 1e20, np.float32)
    c2 = infer_attention_forward_contract(big, big, big)
    with pytest.raises(ShapeError, match="output must remain finite"):
        execute_attention_forward_hip(c2, (big, big, big), bridge)
