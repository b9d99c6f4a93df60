"""Certified exact-f32 GEMM and f32 attention entry points
(browsergrad_amd/semantic.py).

CPU: the input certificate's element rules against the reference's
decodeExactInput cases (browsergrad-semantic-core/src/kernel/
gemm-exact-input-artifact.ts:651-676: sign, NaN / infinity, subnormal,
non-integer, > 2^24) and the SHA-256 commitment.  GPU: bit-exact results
against int64 numpy products on certified inputs (including an output equal
to the inclusive limit 2^24, decided by the host check), refusal of a sum
above the limit, and f32 attention against the float64 oracle with the
semantic-core tolerance (abs-or-rel 1e-4, attention-forward-model.ts:25-29).
"""
from __future__ import annotations

import dataclasses
import threading

import numpy as np
import pytest

from browsergrad_amd.semantic import (
    canonical_hash, check_launches, check_layout, gemm_tile_order, parse_kernel_symbol,
    EXACT_F32_INTEGER_LIMIT, SemanticAttentionError, SemanticGemmError, certify_exact_f32_gemm_inputs,
    prepare_semantic_attention, prepare_semantic_gemm, run_prepared_semantic_attention_resident,
    run_prepared_semantic_gemm_resident, run_semantic_attention, run_semantic_attention_f32, run_semantic_gemm,
    run_semantic_gemm_exact_f32,
)
from oracle import ops as O

F32 = np.float32


@pytest.mark.parametrize("value,msg", [
    (-1.0, "nonnegative"), (-0.0, "canonical positive zero"), (np.nan, "NaN and infinity"),
    (np.inf, "NaN and infinity"), (1e-45, "subnormal"), (2.5, "integer-valued"),
    (float(EXACT_F32_INTEGER_LIMIT * 2), "exceeds the inclusive f32 integer limit"),
])
def test_certificate_rejects_each_inexact_input(value, msg):
    a = np.ones((2, 3), F32)
    a[1, 2] = value
    with pytest.raises(SemanticGemmError, match=msg) as e:
        certify_exact_f32_gemm_inputs(a, np.ones((3, 2), F32), 2, 2, 3)
    assert e.value.code == "BG-WEBGPU-GEMM-NUMERICAL-PROOF" and e.value.path == "$.inputs.lhs[1,2]"


def test_certificate_commits_to_the_bytes():
    a = np.arange(6, dtype=F32).reshape(2, 3)
    b = np.arange(6, dtype=F32).reshape(3, 2)
    cert = certify_exact_f32_gemm_inputs(a, b, 2, 2, 3)
    assert cert["inputs"]["lhs"]["allocationByteLength"] == 24 and len(cert["inputs"]["rhs"]["digest"]) == 64
    assert certify_exact_f32_gemm_inputs(a.tobytes(), b, 2, 2, 3) == cert
    b2 = b.copy()
    b2[0, 0] = 7
    with pytest.raises(SemanticGemmError, match="do not match") as e:
        run_semantic_gemm_exact_f32(None, cert, a, b2)
    assert e.value.code == "BG-WEBGPU-GEMM-INVALID-BINDING"


@pytest.mark.gpu
@pytest.mark.parametrize("m,n,k,hi", [(3, 5, 7, 9), (256, 384, 512, 15), (1000, 999, 1024, 3), (40, 3000, 4096, 2),
                                      (100, 3000, 1024, 3), (250, 2100, 2048, 2)])
def test_exact_gemm_is_bit_exact(bridge, m, n, k, hi):
    rng = np.random.default_rng(m + n + k)
    a = rng.integers(0, hi + 1, (m, k)).astype(F32)
    b = rng.integers(0, hi + 1, (k, n)).astype(F32)
    res = run_semantic_gemm_exact_f32(bridge, certify_exact_f32_gemm_inputs(a, b, m, n, k), a, b)
    got = np.frombuffer(res["destination"], F32).reshape(m, n)
    assert np.array_equal(got, (a.astype(np.int64) @ b.astype(np.int64)).astype(F32))
    t = res["trace"]
    assert t["multiplyAdds"] == m * n * k and t["numericalPreservation"] == "bit-exact-on-certified-inputs"
    # verified artifacts from the launches that ran, with their hashes
    arts = t["artifacts"]
    assert arts["layout"]["body"]["tensors"]["lhs"]["strides"] == [k, 1]
    assert arts["schedule"]["body"]["launches"][0]["family"] in ("gemm32_kernel", "gemm32_wide_k_kernel",
                                                                  "gemm_skinny_kernel")
    for name, key in (("layout", "layoutSemanticHash"), ("tile", "kernelSemanticHash"),
                      ("schedule", "scheduleSemanticHash")):
        assert t[key] == arts[name]["hash"] == canonical_hash(arts[name]["body"])
    assert len(t["backendPreparationHash"]) == 64 and t["inputCertificateSemanticHash"]
    # the same problem prepares the same artifacts
    again = run_semantic_gemm_exact_f32(bridge, certify_exact_f32_gemm_inputs(a, b, m, n, k), a, b)["trace"]
    assert again["backendPreparationHash"] == t["backendPreparationHash"]


@pytest.mark.gpu
def test_exact_gemm_limit_is_inclusive(bridge):
    # 4096 * 4096 = 2^24 exactly: accepted (host check), and exact
    a = np.full((2, 1), 4096, F32)
    b = np.full((1, 3), 4096, F32)
    res = run_semantic_gemm_exact_f32(bridge, certify_exact_f32_gemm_inputs(a, b, 2, 3, 1), a, b)
    assert np.all(np.frombuffer(res["destination"], F32) == float(EXACT_F32_INTEGER_LIMIT))
    # one more term crosses the limit: refused with the output's path
    a2 = np.full((2, 2), 4096, F32)
    b2 = np.full((2, 3), 4096, F32)
    b2[1] = 1
    with pytest.raises(SemanticGemmError, match="exceeds the inclusive f32 integer limit") as e:
        run_semantic_gemm_exact_f32(bridge, certify_exact_f32_gemm_inputs(a2, b2, 2, 3, 2), a2, b2)
    assert e.value.code == "BG-WEBGPU-GEMM-NUMERICAL-PROOF" and e.value.path.startswith("$.proof.output")


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [False, True])
def test_semantic_attention_f32(bridge, causal):
    rng = np.random.default_rng(5)
    b, h, sq, sk, d = 2, 3, 37, 53, 64
    q = rng.standard_normal((b, h, sq, d)).astype(F32)
    k = rng.standard_normal((b, h, sk, d)).astype(F32)
    v = rng.standard_normal((b, h, sk, d)).astype(F32)
    if causal:
        sk, k, v = sq, k[:, :, :sq], v[:, :, :sq]
    res = run_semantic_attention_f32(bridge, q.tobytes(), k.tobytes(), v.tobytes(), batch=b, heads=h, q_len=sq,
                                     k_len=sk, head_dim=d, causal=causal)
    got = np.frombuffer(res["destination"], F32).reshape(b, h, sq, d)
    ref = O.attention_f64(q, k, v, 1.0 / np.sqrt(d), causal=causal)
    assert O.within(got, ref, 1e-4).all(), O.report(got, ref, 1e-4)
    assert res["trace"]["mask"] == ("causal" if causal else "none")
    t = res["trace"]
    assert t["kernelSemanticHash"] == t["artifacts"]["tile"]["hash"]
    assert t["artifacts"]["tile"]["body"]["rows"] == b * h * sq
    assert t["artifacts"]["schedule"]["body"]["launches"][0]["family"] == "fa32_fwd_kernel"
    bad = q.copy()
    bad[0, 0, 0, 0] = np.inf
    with pytest.raises(SemanticAttentionError, match="finite"):
        run_semantic_attention_f32(bridge, bad, k, v, batch=b, heads=h, q_len=sq, k_len=sk, head_dim=d)


def test_gemm_tile_order_is_a_bijection():
    """The host restatement of the kernels' workgroup -> tile map covers every
    tile exactly once for every grid shape up to 48 x 48 tiles (both the
    XCD-remapped case, tile count % 8 == 0, and the plain one)."""
    for tm in range(1, 49):
        for tn in range(1, 49):
            seen = {gemm_tile_order(p, tm, tn) for p in range(tm * tn)}
            assert len(seen) == tm * tn and all(0 <= a < tm and 0 <= b < tn for a, b in seen), (tm, tn)


def _rec(kernel, grid, block=(256, 1, 1)):
    return {"kernel": kernel, "grid": list(grid), "block": list(block), "dynamicLds": 0, "staticLds": 32768,
            "vgprs": 128, "scratchBytesPerLane": 0}


def test_prepare_gemm_fixes_schedule_before_any_launch():
    """prepare_semantic_gemm needs no device: the schedule comes from the
    library's own launch decision (bg_matmul_launch_plan).  300 x 200 x 64
    is six 128 x 128 tiles in one launch; 64 x 128 x 784 (C1's shape) is one
    tile with K split over 25 slices plus the finishing pass."""
    p = prepare_semantic_gemm(300, 200, 64)
    assert p.plan["launches"] == [{"family": "gemm32_kernel", "templateArgs": [128, 128, 0, 1],
                                   "grid": [6, 1, 1], "block": [256, 1, 1]}]
    tile = p.tile["body"]
    assert (tile["tile"], tile["tilesM"], tile["tilesN"], tile["kSlices"]) == ({"m": 128, "n": 128, "k": 16}, 3, 2, 1)
    for art in (p.layout, p.tile, p.schedule):
        assert art["hash"] == canonical_hash(art["body"])
    assert p.layout["body"]["tensors"]["lhs"] == {"shape": [300, 64], "strides": [64, 1], "dtype": "float32",
                                                  "byteLength": 300 * 64 * 4}
    # a second preparation of the same problem hashes the same
    assert prepare_semantic_gemm(300, 200, 64).backendPreparationHash == p.backendPreparationHash
    assert prepare_semantic_gemm(300, 200, 65).backendPreparationHash != p.backendPreparationHash
    s = prepare_semantic_gemm(64, 128, 784)
    assert s.plan["launches"] == [{"family": "gemm32_wide_k_kernel", "templateArgs": [0, 0, 0],
                                   "grid": [8, 1, 1], "block": [1024, 1, 1]}]
    assert s.tile["body"]["kSlices"] == 16 and "wavefront order" in s.tile["body"]["accumulation"]
    assert s.schedule["body"]["tileOrder"] == "row-major"
    assert s.plannedTransientGpuBytes == 4 * (64 * 784 + 784 * 128 + 64 * 128)
    # 40 x 3000 x 4096: 24 column tiles of one 64-row block, K in 10 slices
    # of 448, the slices' partials summed by a second launch.
    k = prepare_semantic_gemm(40, 3000, 4096)
    assert k.plan["launches"] == [{"family": "gemm_skinny_kernel", "templateArgs": [0, 2, 0],
                                   "grid": [240, 1, 1], "block": [1024, 1, 1]},
                                  {"family": "gemm_skinny_finish_kernel", "templateArgs": [],
                                   "grid": [469, 1, 1], "block": [256, 1, 1]}]
    assert k.tile["body"]["kSlices"] == 10 and k.plan["workspaceBytes"] == 4 * 10 * 40 * 3000
    assert k.schedule["body"]["tileOrder"] == "row block y; column tile x // kSlices, K slice x % kSlices"
    # 200 rows: four 64-row blocks along grid y, K in 2 slices.
    k2 = prepare_semantic_gemm(200, 3000, 4096)
    assert [(e["family"], e["templateArgs"], e["grid"]) for e in k2.plan["launches"]] == [
        ("gemm_skinny_kernel", [0, 2, 0], [48, 4, 1]), ("gemm_skinny_finish_kernel", [], [2344, 1, 1])]
    assert k2.tile["body"]["tilesM"] == 4 and k2.plan["workspaceBytes"] == 4 * 2 * 200 * 3000


@pytest.mark.parametrize("kw,path", [
    ({"max_transient_working_set_bytes": 1 << 20}, "$.maxTransientWorkingSetBytes"),
    ({"max_workgroup_storage_bytes": 16 * 1024}, "$.maxWorkgroupStorageBytes"),
    ({"max_workgroup_invocations": 128}, "$.maxWorkgroupInvocations"),
])
def test_prepare_gemm_enforces_limits(kw, path):
    with pytest.raises(SemanticGemmError) as e:
        prepare_semantic_gemm(1024, 1024, 64, **kw)
    assert e.value.code == "BG-WEBGPU-GEMM-RESOURCE-LIMIT" and e.value.path == path


@pytest.mark.parametrize("kw", [{"max_transient_working_set_bytes": 0},
                                {"max_transient_working_set_bytes": (1 << 30) + 1},
                                {"max_workgroup_storage_bytes": True}, {"max_workgroup_invocations": 2048}])
def test_prepare_gemm_refuses_bad_limit_values(kw):
    with pytest.raises(SemanticGemmError, match="positive integer"):
        prepare_semantic_gemm(8, 8, 8, **kw)


def test_prepared_objects_are_required_and_resident_runs_are_closed():
    p = prepare_semantic_gemm(8, 8, 8)
    with pytest.raises(SemanticGemmError) as e:
        run_prepared_semantic_gemm_resident(p, {"lhs": 1, "rhs": 2})
    assert e.value.code == "BG-WEBGPU-GEMM-NUMERICAL-PROOF"
    forged = dataclasses.replace(p)  # same fields, not returned by prepare
    a = np.ones((8, 8), F32)
    cert = certify_exact_f32_gemm_inputs(a, a, 8, 8, 8)
    for bad in (forged, {"m": 8}):
        with pytest.raises(SemanticGemmError, match="returned by its prepare function") as e2:
            run_semantic_gemm(None, bad, cert, a, a)
        assert e2.value.code == "BG-WEBGPU-GEMM-INVALID-BINDING"
    with pytest.raises(SemanticGemmError, match="the preparation for 8 x 8 x 8"):
        b = np.ones((8, 4), F32)
        run_semantic_gemm(None, p, certify_exact_f32_gemm_inputs(a, b, 8, 4, 8), a, b)
    pa = prepare_semantic_attention(1, 1, 4, 4, 8)
    with pytest.raises(SemanticAttentionError) as e3:
        run_prepared_semantic_attention_resident(pa, None)
    assert e3.value.code == "BG-WEBGPU-ATTENTION-NUMERICAL-PROOF"


def test_cancel_and_wait_budget_are_checked_before_the_device():
    p = prepare_semantic_gemm(8, 8, 8)
    a = np.ones((8, 8), F32)
    cert = certify_exact_f32_gemm_inputs(a, a, 8, 8, 8)
    ev = threading.Event()
    ev.set()
    with pytest.raises(SemanticGemmError) as e:
        run_semantic_gemm(None, p, cert, a, a, cancel=ev)  # the bridge is never reached
    assert e.value.code == "BG-WEBGPU-GEMM-CANCELLED"
    for bad in (0, 5 * 60_000 + 1, 1.5):
        with pytest.raises(SemanticGemmError, match="positive integer") as e2:
            run_semantic_gemm(None, p, cert, a, a, timeout_ms=bad)
        assert e2.value.code == "BG-WEBGPU-GEMM-INVALID-BINDING"
    with pytest.raises(SemanticGemmError, match="is_set"):
        run_semantic_gemm(None, p, cert, a, a, cancel=object())


def test_prepare_attention():
    p = prepare_semantic_attention(2, 3, 37, 53, 64)
    assert p.plan["launches"] == [{"family": "fa32_fwd_kernel", "templateArgs": [64, 1], "grid": [6, 1, 1],
                                   "block": [256, 1, 1]}]
    t = p.tile["body"]
    assert (t["queriesPerWorkgroup"], t["keysPerTile"], t["paddedHeadDim"], t["rows"]) == (128, 64, 64, 2 * 3 * 37)
    assert prepare_semantic_attention(1, 1, 300, 300, 20).plan["launches"][0]["templateArgs"] == [32, 1]
    assert prepare_semantic_attention(1, 1, 300, 300, 7).plan["launches"][0]["templateArgs"] == [16, 0]
    assert prepare_semantic_attention(2, 3, 37, 53, 64).backendPreparationHash == p.backendPreparationHash
    assert prepare_semantic_attention(2, 3, 37, 53, 64, causal=False, scale=0.2).backendPreparationHash != \
        p.backendPreparationHash
    with pytest.raises(SemanticAttentionError, match="head dim 1..64") as e:
        prepare_semantic_attention(1, 1, 8, 8, 65)
    assert e.value.code == "BG-WEBGPU-ATTENTION-UNSUPPORTED-PROFILE"
    with pytest.raises(SemanticAttentionError, match="q_len <= k_len"):
        prepare_semantic_attention(1, 1, 9, 8, 16, causal=True)
    with pytest.raises(SemanticAttentionError) as e2:
        prepare_semantic_attention(1, 1, 8, 8, 64, max_workgroup_storage_bytes=32 * 1024)
    assert e2.value.code == "BG-WEBGPU-ATTENTION-RESOURCE-LIMIT"
    with pytest.raises(SemanticAttentionError) as e3:
        prepare_semantic_attention(64, 16, 2048, 2048, 64)  # 1 GiB+ of planned buffers
    assert e3.value.code == "BG-WEBGPU-ATTENTION-RESOURCE-LIMIT"


@pytest.mark.parametrize("name,args", [
    ("_ZN12_GLOBAL__N_113gemm32_kernelILi128ELi128ELb0ELb1EEEvNS_8GemmArgsE", [128, 128, 0, 1]),
    ("(anonymous namespace)::gemm32_kernel<128, 128, false, true>((anonymous namespace)::GemmArgs)",
     [128, 128, 0, 1]),
    ("_ZN12_GLOBAL__N_120gemm32_splitk_reduceILi0EEEvNS_8GemmArgsEi", None),
])
def test_parse_kernel_symbol(name, args):
    assert parse_kernel_symbol(name, "gemm32_kernel") == args


def test_parse_kernel_symbol_without_template_arguments():
    fin = "_ZN12_GLOBAL__N_125gemm_skinny_finish_kernelENS_8GemmArgsEiPKf"
    assert parse_kernel_symbol(fin, "gemm_skinny_finish_kernel") == []
    assert parse_kernel_symbol("(anonymous namespace)::gemm_skinny_finish_kernel((anonymous namespace)::GemmArgs, "
                               "int, float const*)", "gemm_skinny_finish_kernel") == []
    # neither the finishing kernel's name nor a longer one matches the main kernel's family
    assert parse_kernel_symbol(fin, "gemm_skinny_kernel") is None
    assert parse_kernel_symbol("_ZN12_GLOBAL__N_118gemm_skinny_kernelILi0ELi2ELb0EEEvNS_8GemmArgsEliPf",
                               "gemm_skinny_kernel") == [0, 2, 0]
    assert parse_kernel_symbol("_ZN12_GLOBAL__N_121xgemm_skinny_kernelENS_8GemmArgsE", "gemm_skinny_kernel") is None


def test_launch_log_must_match_the_prepared_schedule():
    p = prepare_semantic_gemm(300, 200, 64)
    good = [_rec("_ZN12_GLOBAL__N_113gemm32_kernelILi128ELi128ELb0ELb1EEEvNS_8GemmArgsE", [6, 1, 1])]
    check_launches(p.plan, good, "BG-WEBGPU-GEMM-VALIDATION")
    w = prepare_semantic_gemm(64, 128, 784)
    check_launches(w.plan, [_rec("_ZN12_GLOBAL__N_120gemm32_wide_k_kernelILi0ELb0ELb0EEEvNS_8GemmArgsE", [8, 1, 1],
                                 (1024, 1, 1))], "BG-WEBGPU-GEMM-VALIDATION")
    bad_grid = [dict(good[0], grid=[5, 1, 1])]
    bad_args = [dict(good[0], kernel=good[0]["kernel"].replace("ELb1EE", "ELb0EE"))]
    bad_block = [dict(good[0], block=[512, 1, 1])]
    other = [_rec("_ZN12_GLOBAL__N_120gemm32_wide_k_kernelILi0ELb0ELb0EEEvNS_8GemmArgsE", [6, 1, 1])]
    for bad in (bad_grid, bad_args, bad_block, other, good + good, []):
        with pytest.raises(SemanticGemmError) as e:
            check_launches(p.plan, bad, "BG-WEBGPU-GEMM-VALIDATION")
        assert e.value.code == "BG-WEBGPU-GEMM-VALIDATION"


def test_layout_is_checked_against_device_records():
    p = prepare_semantic_gemm(4, 6, 5)
    info = lambda shp: {"shape": tuple(shp), "dtype": "float32", "nbytes": 4 * int(np.prod(shp))}  # noqa: E731
    recs = {"lhs": info([4, 5]), "rhs": info([5, 6]), "output": info([4, 6])}
    check_layout(p.layout, recs, "BG-WEBGPU-GEMM-VALIDATION")
    for name, bad in (("rhs", info([6, 5])), ("output", dict(info([4, 6]), dtype="float16")),
                      ("lhs", dict(info([4, 5]), nbytes=84))):
        with pytest.raises(SemanticGemmError, match="does not match the prepared layout") as e:
            check_layout(p.layout, {**recs, name: bad}, "BG-WEBGPU-GEMM-VALIDATION")
        assert e.value.path == f"$.layout.{name}"


@pytest.mark.gpu
def test_prepared_gemm_runs_repeatably(bridge):
    """One prepared specialization, several runs: every run's launch log is
    the prepared schedule (the wide-K kernel for C1's 64 x 128 x 784), its device
    records match the layout, its results are exact, and the preparation
    hash in the trace is the same every time."""
    rng = np.random.default_rng(11)
    p = prepare_semantic_gemm(64, 128, 784)
    hashes = set()
    for _ in range(3):
        a = rng.integers(0, 4, (64, 784)).astype(F32)
        b = rng.integers(0, 4, (784, 128)).astype(F32)
        res = run_semantic_gemm(bridge, p, certify_exact_f32_gemm_inputs(a, b, 64, 128, 784), a, b,
                                timeout_ms=60_000)
        got = np.frombuffer(res["destination"], F32).reshape(64, 128)
        assert np.array_equal(got, (a.astype(np.int64) @ b.astype(np.int64)).astype(F32))
        assert res["trace"]["launchesMatchedPreparation"] is True
        hashes.add(res["trace"]["backendPreparationHash"])
    assert hashes == {p.backendPreparationHash}


@pytest.mark.gpu
def test_prepared_attention_runs_repeatably(bridge):
    rng = np.random.default_rng(12)
    p = prepare_semantic_attention(2, 2, 100, 100, 24, causal=True)
    hashes = set()
    for _ in range(2):
        q, k, v = (rng.standard_normal((2, 2, 100, 24)).astype(F32) for _ in range(3))
        res = run_semantic_attention(bridge, p, q, k, v)
        got = np.frombuffer(res["destination"], F32).reshape(2, 2, 100, 24)
        ref = O.attention_f64(q, k, v, 1.0 / np.sqrt(24), causal=True)
        assert O.within(got, ref, 1e-4).all(), O.report(got, ref, 1e-4)
        hashes.add(res["trace"]["backendPreparationHash"])
    assert hashes == {p.backendPreparationHash}
