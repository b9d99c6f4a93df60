"""Front end on CPU: IR, cast insertion, fusion, plan builder, HIP rewrites,
program compiler, and the graph oracle pinned against independent forms.

Reference behaviours mirrored (packages/browsergrad-jit/src/python):
_ir.py:277-330 (UOp validation), _amp.py:183-261 (cast placement),
_fusion.py:141-517 (matchers), _gpu_plan.py:285-666 (plan / side table).
"""
from __future__ import annotations

import json

import numpy as np
import pytest

from browsergrad_amd.jit import configs
from browsergrad_amd.jit.amp import insert_cast_pass
from browsergrad_amd.jit.fusion import fuse, get_last_report
from browsergrad_amd.jit.gpu_plan import GpuPlanUnsupported, build_gpu_execution_plan, build_gpu_execution_submission
from browsergrad_amd.jit.hip_fusion import ACT_GELU, ACT_RELU, hip_fuse
from browsergrad_amd.jit.ir import ShapeError, UOp, toposort
from browsergrad_amd.jit.program import ProgramTooLarge, compile_program
from browsergrad_amd.jit.realize import prepare
from browsergrad_amd.jit.tensor import Session, autocast, relu, softmax
from oracle import graph as G
from oracle import ops as O


def ops_of(root):
    return [n.op for n in toposort(root)]


# ---- IR ----------------------------------------------------------------------

def test_uop_validation_mirrors_reference():
    with pytest.raises(ValueError):
        UOp("NOPE", (), (), "float32")
    with pytest.raises(ShapeError):
        UOp("ADD", (), (2,), "float32")                       # non-leaf without inputs
    c = UOp("CONST", (), (), "float32", {"value": 1.0})
    with pytest.raises(ShapeError):
        UOp("CONST", (c,), (), "float32", {"value": 1.0})     # leaf with inputs
    with pytest.raises(ShapeError):
        UOp("NEG", (c,), (-1,), "float32")
    with pytest.raises(ValueError):
        UOp("NEG", (c,), (), "complex64")


def test_toposort_is_leaves_first_and_dedups_shared_nodes():
    s = Session()
    a = s.from_numpy(np.ones((2, 2), np.float32))
    b = a + a
    y = b * b
    order = toposort(y.uop)
    assert order[-1] is y.uop
    assert len(order) == len({id(n) for n in order}) == 4  # BUFFER, LOAD, ADD, MUL


# ---- cast insertion (A.3 / A.4 / A.5 of the config semantics) ------------------

def test_amp_c3_places_casts_like_the_reference():
    s, y = configs.c3(scale=1 / 64)
    g = insert_cast_pass(y.uop)
    add = g
    assert add.op == "ADD" and add.dtype == "float32"
    mm_cast, bias = add.inputs
    assert mm_cast.op == "CAST" and mm_cast.dtype == "float32" and mm_cast.arg["amp_inserted"]
    mm = mm_cast.inputs[0]
    assert mm.op == "MATMUL" and mm.dtype == "float16"
    assert all(i.op == "CAST" and i.dtype == "float16" for i in mm.inputs)
    assert bias.dtype == "float32"


def test_amp_noop_without_autocast_and_promotes_f64_constants():
    s, y = configs.c1(scale=0.25)
    assert insert_cast_pass(y.uop) is y.uop
    s2 = Session()
    x = s2.from_numpy(np.ones((4,), np.float32))
    with autocast():
        z = 0.5 * x                      # CONST float64 * f32
    assert z.dtype == "float64"          # the IR dtype numpy promotion gives
    g = insert_cast_pass(z.uop)
    assert g.dtype == "float32" and g.inputs[0].op == "CAST" and g.inputs[0].inputs[0].op == "CONST"


# ---- reference fusion --------------------------------------------------------

def test_softmax_template_fuses_and_chain_fuses():
    s = Session()
    x = s.from_numpy(np.zeros((3, 5), np.float32))
    g = fuse(softmax(x).uop)
    assert ops_of(g).count("FUSED_SOFTMAX") == 1 and "DIV" not in ops_of(g)
    assert get_last_report().fused[0].pattern == "softmax"
    a = s.from_numpy(np.ones((3, 5), np.float32))
    chain = ((a * 2.0) + a).exp()
    g2 = fuse(chain.uop)
    fe = [n for n in toposort(g2) if n.op == "FUSED_ELEMENTWISE"]
    assert len(fe) == 1 and [o[0] for o in fe[0].arg["ops"]] == ["MUL", "ADD", "EXP"]
    assert fe[0].arg["ops"][1][1] == 0  # the ADD reads step 0


def test_chain_breaks_at_shared_intermediate():
    s = Session()
    a = s.from_numpy(np.ones((4,), np.float32))
    t = a.exp()
    y = (t + t) * t  # t has three consumers -> not a chain interior
    g = fuse(y.uop)
    assert "EXP" in ops_of(g)


# ---- plan builder ----------------------------------------------------------------

def test_plan_fields_liveness_and_peak():
    s = Session()
    a = s.from_numpy(np.ones((2, 3), np.float32))
    b = s.from_numpy(np.ones((3, 4), np.float32))
    plan = build_gpu_execution_plan((a @ b).uop)
    summ = plan.summary()
    assert summ["ops"] == ["BUFFER", "LOAD", "BUFFER", "LOAD", "MATMUL"]
    assert [st["value_id"] for st in summ["steps"]] == [0, 1, 2, 3, 4]
    assert summ["steps"][4]["input_ids"] == [1, 3]
    bufs = {b["value_id"]: b for b in summ["buffers"]}
    assert bufs[1]["last_step"] == 4 and bufs[0]["last_step"] == 1 and bufs[4]["materialize"]
    # peak at step 3: LOAD a (24 B), BUFFER b (48 B, last read at 3), LOAD b (48 B);
    # step 4 holds 24 + 48 + 32
    assert summ["peak_live_bytes"] == 24 + 48 + 48
    json.dumps(summ)


def test_semantic_side_table_for_2d_permute_and_refusals():
    s, y = configs.c1(scale=0.25)
    sub = build_gpu_execution_submission(y.uop)
    req = sub.semantic_request_summary()
    assert req["schema"] == "browsergrad.jit.tensor-plan-semantic-requests"
    assert req["version"] == {"major": 1, "minor": 0}
    assert len(req["requests"]) == 2
    r0 = req["requests"][0]
    assert r0["kind"] == "dense-permutation-view-copy" and r0["dtype"] == "f32" and r0["axes"] == [1, 0]
    assert all(isinstance(e, str) for e in r0["inputShape"])
    assert all(st["arg"] is None for st in sub.plan_summary()["steps"] if st["op"] == "PERMUTE")
    # rank-4 PERMUTE (attention's k.transpose) is outside the initial side table
    s4 = Session()
    k = s4.from_numpy(np.ones((1, 2, 3, 4), np.float32))
    with pytest.raises(GpuPlanUnsupported):
        build_gpu_execution_submission(k.transpose(-1, -2).uop)


# ---- HIP rewrites ----------------------------------------------------------------

def _prepared(name, scale):
    s, y = configs.BUILDERS[name](scale=scale)
    return s, y, prepare(y.uop, s.buffers)


def test_rewrites_c1_two_linears_first_with_relu():
    s, y, g = _prepared("c1", 0.25)
    lin = [n for n in toposort(g) if n.op == "HIP_LINEAR"]
    assert len(lin) == 2 and sorted(n.arg["act"] for n in lin) == [0, ACT_RELU]
    assert all(n.arg["trans_b"] and not n.arg["round_out"] for n in lin)


def test_rewrites_c2_one_fused_reduce_program():
    s, y, g = _prepared("c2", 1 / 64)
    fused = [n for n in toposort(g) if n.op == "HIP_REDUCE_FUSED"]
    assert len(fused) == 1 and fused[0].arg["reduce"] == "sum" and len(fused[0].inputs) == 3
    p = fused[0].arg["program"]
    r = O.fused_program([np.float32(0.5), np.float32(2.0), np.float32(-0.25)][::1], p.ops, p.imms)
    a, b, c = 0.5, 2.0, -0.25
    assert np.isclose(r, max(a * b + c, 0.0) * np.exp(-a * a), rtol=1e-6)


def test_rewrites_c4_single_attention_kernel():
    s, y, g = _prepared("c4", 1 / 16)
    att = [n for n in toposort(g) if n.op == "HIP_ATTENTION"]
    assert ops_of(g).count("HIP_ATTENTION") == 1 and len([n for n in toposort(g) if n.op not in
                                                          ("BUFFER", "LOAD", "HIP_ATTENTION")]) == 0
    assert att[0].arg == {"scale": 0.125, "causal": True, "round_scores": True}


def test_rewrites_c5_block_structure():
    s, y, g = _prepared("c5", 1 / 8)
    ops = ops_of(g)
    assert ops.count("HIP_ATTENTION") == 1 and ops.count("LAYER_NORM") == 2
    lin = [n for n in toposort(g) if n.op == "HIP_LINEAR"]
    assert len(lin) == 4 and [n.arg["act"] for n in lin].count(ACT_GELU) == 1
    assert all(n.arg["round_out"] and n.arg["in_dtype"] == "float16" for n in lin)
    assert "EXP" not in ops and "DIV" not in ops and "MATMUL" not in ops
    # both residual adds ride on the out-projection and MLP-down epilogues
    res = [n for n in lin if n.arg.get("residual")]
    assert len(res) == 2 and all(len(n.inputs) == 4 and n.inputs[3].dtype == "float32" for n in res)
    assert "HIP_REDUCE_FUSED" not in ops, ops


def test_rewrites_preserve_values_on_cpu_oracle():
    """The rewritten graph's pieces are evaluated by the oracle only through
    the original graph; this checks that rewriting leaves the original graph
    untouched (a pass must not mutate shared nodes)."""
    s, y = configs.c2(scale=1 / 128)
    before = G.evaluate(y.uop, s.buffers)
    prepare(y.uop, s.buffers)
    after = G.evaluate(y.uop, s.buffers)
    assert np.array_equal(before, after)


# ---- program compiler ------------------------------------------------------------

def test_program_rounds_narrow_nodes_and_limits():
    s = Session()
    a = s.from_numpy(np.ones((4,), np.float16))
    y = (a + a) * a
    prog = compile_program([y.uop.inputs[0], y.uop], y.uop)
    assert [o[0] for o in prog.ops] == ["ADD", "ROUND_F16", "MUL", "ROUND_F16"]
    big = a
    for _ in range(20):
        big = big + a
    nodes = [n for n in toposort(big.uop) if n.op == "ADD"]
    with pytest.raises(ProgramTooLarge):
        compile_program(nodes, big.uop)


# ---- graph oracle pinned -----------------------------------------------------------

def test_graph_oracle_c2_matches_op_oracle_bit_exact():
    s, y = configs.c2(scale=1 / 64)
    ref = G.evaluate(y.uop, s.buffers)
    a, b, c = (s.buffers.get(n.inputs[0].arg) for n in toposort(y.uop) if n.op == "LOAD")
    assert np.array_equal(ref, O.c2_chain(a, b, c))


def test_graph_oracle_matmul_closed_forms():
    s = Session()
    a = s.from_numpy(np.array([[1, 2, 3], [4, 5, 6]], np.float32))
    b = s.from_numpy(np.array([[7, 8], [9, 10], [11, 12]], np.float32))
    assert G.evaluate((a @ b).uop, s.buffers).tolist() == [[58, 64], [139, 154]]  # reference.test.ts:42-50
    ones = s.from_numpy(np.ones((1, 4096), np.float32))
    col = s.from_numpy(np.ones((4096, 1), np.float32))
    with autocast():
        r = ones @ col
    out = G.evaluate(r.uop, s.buffers)
    assert out.dtype == np.float16 and out[0, 0] == 4096.0                      # amp.test.ts:47-66


def test_graph_oracle_c3_and_c4_match_op_oracle():
    s, y = configs.c3(scale=1 / 64)
    ref = G.evaluate(y.uop, s.buffers)
    x, w, b = (s.buffers.get(n.inputs[0].arg) for n in toposort(y.uop) if n.op == "LOAD")
    assert np.array_equal(ref, O.linear_amp(x, w, b))
    s4, y4 = configs.c4(scale=1 / 32)
    ref4 = G.evaluate(y4.uop, s4.buffers)
    q, k, v = (s4.buffers.get(n.inputs[0].arg) for n in toposort(y4.uop)
               if n.op == "LOAD" and n.dtype == "float16")
    assert np.array_equal(ref4, O.sdpa_amp(q, k, v, 0.125, True))


def test_graph_oracle_relu_is_where_form():
    s = Session()
    x = s.from_numpy(np.array([-1.0, 0.0, 2.0, np.nan], np.float32))
    out = G.evaluate(relu(x).uop, s.buffers)
    assert out[:3].tolist() == [0.0, 0.0, 2.0] and out[3] == 0.0  # where(nan > 0) is False


def test_graph_oracle_c5_matches_composed_op_oracle():
    s, y = configs.c5(scale=1 / 8)
    ref = G.evaluate(y.uop, s.buffers)
    arr = {n.inputs[0].arg.split("#")[0]: s.buffers.get(n.inputs[0].arg) for n in toposort(y.uop)
           if n.op == "LOAD" and not n.inputs[0].arg.startswith(("full", "causal"))}
    x = arr["x"]
    bsz, seq, emb = x.shape
    heads, hd = 2, 64

    def lin(t, w, b):
        return O.linear_amp(t, np.ascontiguousarray(w.T), b)

    h1 = O.layer_norm(x, arr["ln1_w"], arr["ln1_b"])
    qkv = lin(h1, arr["w_qkv"], arr["b_qkv"])
    sp = [qkv[..., i * emb:(i + 1) * emb].reshape(bsz, seq, heads, hd).transpose(0, 2, 1, 3) for i in range(3)]
    att = O.sdpa_amp(sp[0], sp[1], sp[2], 1.0 / np.sqrt(hd), True)
    att = att.transpose(0, 2, 1, 3).reshape(bsz, seq, emb)
    h = x + lin(att.astype(np.float32), arr["w_o"], arr["b_o"])
    h2 = O.layer_norm(h, arr["ln2_w"], arr["ln2_b"])
    up = O.gelu_tanh_f32(lin(h2, arr["w_up"], arr["b_up"]))
    out = h + lin(up, arr["w_down"], arr["b_down"])
    assert np.array_equal(ref, out)
