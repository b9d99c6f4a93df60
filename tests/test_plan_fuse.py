"""The tensor-plan executor's plan-level fusion, on the CPU.

bg_plan_inspect parses, validates and fuses a plan exactly as
bg_run_tensor_plan does, without a device, and reports the steps it would
run.  These tests pin which step groups become one launch (GEMM epilogues,
elementwise programs with a trailing reduction, SDPA as one attention
kernel) for the five BASELINE configs as the HIP route's plan builder
writes them, what must not fuse, and that malformed plans are refused with
the executor's messages (the same code path the GPU route runs).
"""
from __future__ import annotations

import json

import pytest

from browsergrad_amd import _native as N
from browsergrad_amd.errors import KernelError
from browsergrad_amd.jit import configs
from browsergrad_amd.jit.realize import _plan_submission

pytestmark = pytest.mark.skipif(not N.LIB_PATH.exists(), reason="libbghip.so not built")


def inspect(plan, req=None):
    from browsergrad_amd.bridge import inspect_tensor_plan
    return inspect_tensor_plan(plan, req)


def fused_ops(name, scale, **kw):
    s, y = configs.BUILDERS[name](scale=scale, **kw)
    plan, req, rj = _plan_submission(y.uop, s.buffers)
    out = inspect(plan, rj or None)
    return [st for st in out["steps"] if st["op"] not in ("BUFFER", "LOAD")], plan


def test_c1_two_gemms_with_bias_relu_epilogues():
    steps, _ = fused_ops("c1", 1.0)
    assert [st["op"] for st in steps] == ["+LINEAR", "+LINEAR"]
    assert [st["act"] for st in steps] == [1, 0]
    assert all(st["trans_b"] == 1 and st["bias"] == 1 for st in steps)  # W.T folded into the NT layout


def test_c2_is_one_fused_program_with_row_reduction():
    steps, plan = fused_ops("c2", 1 / 16)
    assert len(plan["steps"]) == 12
    assert [st["op"] for st in steps] == ["+PROGRAM"]
    assert steps[0]["reduce"] == 1 and steps[0]["n_ops"] == 9 and len(steps[0]["inputs"]) == 3


@pytest.mark.parametrize("amp", [False, True])
def test_c3_one_gemm_with_casts_folded(amp):
    steps, _ = fused_ops("c3", 1 / 16, amp=amp)
    assert [st["op"] for st in steps] == ["+LINEAR"]
    st = steps[0]
    assert st["bias"] == 1 and st["trans_b"] == 0
    assert (st["round"], st["a_dtype"], st["b_dtype"]) == ((1, 0, 0) if amp else (0, -1, -1))


def test_c4_is_one_attention_step():
    steps, _ = fused_ops("c4", 1 / 16)
    assert [st["op"] for st in steps] == ["+ATTENTION"]
    assert steps[0]["causal"] == 1 and abs(steps[0]["scale"] - 0.125) < 1e-7


def test_c5_block():
    steps, _ = fused_ops("c5", 1 / 16)
    ops = [st["op"] for st in steps]
    assert ops.count("+ATTENTION") == 1 and ops.count("+LINEAR") == 4 and ops.count("LAYER_NORM") == 2
    lin = [st for st in steps if st["op"] == "+LINEAR"]
    assert [st["residual"] for st in lin] == [0, 1, 0, 1]  # out-projection and MLP-down add the residual
    assert ops.count("+PROGRAM") == 1  # GELU: the whole tanh graph in one program
    assert "FUSED_SOFTMAX" not in ops and "MATMUL" not in ops and "CONST" not in ops


def _plan(steps, root):
    return {"steps": steps, "buffers": [], "root_id": root, "materialization_boundary": "root",
            "peak_live_bytes": 0, "has_custom_ops": False}


def _st(i, op, ins, shape, dtype="float32", arg=None):
    return {"step": i, "value_id": i, "op": op, "input_ids": ins, "shape": shape, "dtype": dtype, "arg": arg}


def test_values_read_outside_a_group_are_not_absorbed():
    # t = a * b is read by the ADD and is also the root's sibling output: the
    # reduction may not swallow it, since it is read twice.
    steps = [_st(0, "BUFFER", [], [4, 8]), _st(1, "BUFFER", [], [4, 8]),
             _st(2, "MUL", [0, 1], [4, 8]), _st(3, "EXP", [2], [4, 8]), _st(4, "ADD", [2, 3], [4, 8]),
             _st(5, "REDUCE", [4], [4], arg={"op": "sum", "axis": 1, "keepdims": False})]
    out = inspect(_plan(steps, 5))
    assert [s["op"] for s in out["steps"]] == ["BUFFER", "BUFFER", "+PROGRAM"]
    # root inside the chain: the MUL is the root and is read by EXP -> stays a step of its own
    steps2 = steps[:4]
    out2 = inspect(_plan(steps2, 2))
    assert [s["op"] for s in out2["steps"]] == ["BUFFER", "BUFFER", "MUL"]  # EXP is dead code
    # a reduction over a non-trailing axis is not fused into the program
    steps3 = steps[:5] + [_st(5, "REDUCE", [4], [8], arg={"op": "sum", "axis": 0, "keepdims": False})]
    ops3 = [s["op"] for s in inspect(_plan(steps3, 5))["steps"]]
    assert ops3 == ["BUFFER", "BUFFER", "+PROGRAM", "REDUCE"]


def test_matmul_without_epilogue_stays_plain():
    steps = [_st(0, "BUFFER", [], [4, 8]), _st(1, "BUFFER", [], [8, 3]), _st(2, "MATMUL", [0, 1], [4, 3])]
    assert [s["op"] for s in inspect(_plan(steps, 2))["steps"]] == ["BUFFER", "BUFFER", "MATMUL"]


def test_internal_opcodes_are_not_accepted_from_the_wire():
    steps = [_st(0, "BUFFER", [], [4]), _st(1, "+PROGRAM", [0], [4])]
    with pytest.raises(KernelError, match="not a plan opcode"):
        inspect(_plan(steps, 1))


@pytest.mark.parametrize("text,msg", [
    ("{", "valid JSON"),
    ("[]", "must be an object"),
    (json.dumps({"steps": 3}), "steps must be an array"),
    (json.dumps(_plan([_st(0, "ADD", [7, 8], [2])], 0)), "before production"),
    (json.dumps(_plan([_st(0, "BUFFER", [], [2] * 9)], 0)), "rank 9"),
    (json.dumps(_plan([_st(0, "BUFFER", [], [-1])], 0)), "negative extent"),
    (json.dumps(_plan([_st(0, "BUFFER", [], [2], dtype="int64")], 0)), "dtype"),
    (json.dumps(_plan([_st(0, "BUFFER", [], [2])], 5)), "root 5 missing"),
])
def test_malformed_plans_are_refused(text, msg):
    with pytest.raises(KernelError, match=msg):
        inspect(text)


def _amp_sdpa(qshape, kshape, vshape, seed=0):
    """An autocast SDPA graph (CAST(PERMUTE(K)) feeds Q K^T) of the given shapes."""
    from browsergrad_amd.jit.tensor import Session, autocast, scaled_dot_product_attention
    import numpy as np
    rng = np.random.default_rng(seed)
    s = Session()
    q, k, v = (s.from_numpy(rng.standard_normal(sh, dtype=np.float32)) for sh in (qshape, kshape, vshape))
    with autocast("float16"):
        y = scaled_dot_product_attention(q, k, v)
    return s, y


def _sdpa_steps_left_alone(y, s):
    plan, req, rj = _plan_submission(y.uop, s.buffers)
    out = inspect(plan, rj or None)
    by_id = {st["value_id"]: st for st in out["steps"]}
    ops = [st["op"] for st in out["steps"]]
    assert "+ATTENTION" not in ops
    # The K^T cast still reads the permuted K, and the permutation is still there.
    perms = [st for st in out["steps"] if st["op"] == "PERMUTE"]
    mm = [st for st in out["steps"] if st["op"] == "MATMUL"]
    assert len(mm) == 2, ops
    qk = mm[0]  # the first MATMUL in plan order is Q K^T
    kt = by_id[qk["inputs"][1]]
    assert kt["op"] == "CAST", kt
    src = by_id[kt["inputs"][0]]
    assert src["op"] == "PERMUTE" and src in perms, (kt, src)
    return plan, out


def test_sdpa_refused_when_value_depth_differs_leaves_plan_unchanged():
    # dv = 6 != dk = 4: not an attention the kernel runs.  Before the fix
    # the CAST(PERMUTE(K)) was already re-pointed at K when the shape check
    # turned the group away, so Q K^T read K unpermuted.
    s, y = _amp_sdpa((1, 2, 5, 4), (1, 2, 3, 4), (1, 2, 3, 6))
    _sdpa_steps_left_alone(y, s)


def test_sdpa_refused_for_broadcast_key_heads_with_sk_equal_d():
    # K with one head against two query heads, sk == d == 4: a wrongly
    # re-pointed cast would still make a shape-valid (and silently wrong)
    # Q K^T, so the plan itself must be unchanged.
    s, y = _amp_sdpa((1, 2, 5, 4), (1, 1, 4, 4), (1, 1, 4, 4))
    _sdpa_steps_left_alone(y, s)


def test_bf16_scalar_constant_is_inlined_rounded():
    # One bfloat16 CONST read by two fused groups: each program inlines it as
    # an immediate, which must be the value the unfused executor stores
    # (rounded to bfloat16), not the wire's double.
    c = 0.1  # bf16(0.1) = 0.10009765625
    steps = [_st(0, "BUFFER", [], [4, 8], dtype="bfloat16"),
             _st(1, "CONST", [], [1], dtype="bfloat16", arg={"value": c}),
             _st(2, "MUL", [0, 1], [4, 8], dtype="bfloat16"),
             _st(3, "REDUCE", [2], [4], dtype="bfloat16", arg={"op": "sum", "axis": 1, "keepdims": False}),
             _st(4, "ADD", [0, 1], [4, 8], dtype="bfloat16"),
             _st(5, "REDUCE", [4], [4], dtype="bfloat16", arg={"op": "sum", "axis": 1, "keepdims": False}),
             _st(6, "ADD", [3, 5], [4], dtype="bfloat16")]
    out = inspect(_plan(steps, 6))
    progs = [st for st in out["steps"] if st["op"] == "+PROGRAM"]
    assert progs, [st["op"] for st in out["steps"]]
    imms = [v for st in progs for v in st.get("imms", [])]
    assert imms and all(v == 0.10009765625 for v in imms), imms
