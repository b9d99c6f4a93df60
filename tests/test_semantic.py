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

import numpy as np
import pytest

from browsergrad_amd.semantic import (
    canonical_hash, gemm_artifacts, gemm_tile_order,
    EXACT_F32_INTEGER_LIMIT, SemanticAttentionError, SemanticGemmError, certify_exact_f32_gemm_inputs,
    run_semantic_attention_f32, run_semantic_gemm_exact_f32,
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
@pytest.mark.parametrize("m,n,k,hi", [(3, 5, 7, 9), (256, 384, 512, 15), (1000, 999, 1024, 3)])
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
    assert arts["schedule"]["body"]["launches"][0]["kernel"].find("gemm32") >= 0
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


def _rec(kernel, grid):
    return {"kernel": kernel, "grid": grid, "block": [256, 1, 1], "dynamicLds": 0, "staticLds": 32768,
            "vgprs": 128, "scratchBytesPerLane": 0}


def test_gemm_artifacts_from_a_launch_log():
    log = [_rec("_ZN12_GLOBAL__N_113gemm32_kernelILi128ELi128ELb0ELb1EEEv8GemmArgs", [6, 1, 1])]
    arts = gemm_artifacts(log, 300, 200, 64)
    tile = arts["tile"]["body"]
    assert (tile["tile"], tile["tilesM"], tile["tilesN"], tile["kSlices"]) == ({"m": 128, "n": 128}, 3, 2, 1)
    assert arts["tile"]["hash"] == canonical_hash(tile)
    # split K: partial GEMM over 4 slices and the finishing pass
    log2 = [_rec("_ZN12_GLOBAL__N_113gemm32_kernelILi128ELi128ELb1ELb1EEEv8GemmArgs", [1, 4, 1]),
            _rec("_ZN12_GLOBAL__N_120gemm32_splitk_reduceILi0EEEv8GemmArgsi", [32, 1, 1])]
    t2 = gemm_artifacts(log2, 64, 128, 784)["tile"]["body"]
    assert t2["kSlices"] == 4 and "slice order" in t2["accumulation"]


@pytest.mark.parametrize("grid,m,n,msg", [
    ([5, 1, 1], 300, 200, "grid.x"),            # one tile short
    ([6, 1, 1], 300, 300, "grid.x"),            # wrong tile count for the shape
])
def test_gemm_artifacts_refuse_a_schedule_that_does_not_cover(grid, m, n, msg):
    log = [_rec("_ZN12_GLOBAL__N_113gemm32_kernelILi128ELi128ELb0ELb1EEEv8GemmArgs", grid)]
    with pytest.raises(SemanticGemmError, match=msg) as e:
        gemm_artifacts(log, m, n, 64)
    assert e.value.code == "BG-WEBGPU-GEMM-VALIDATION"
    with pytest.raises(SemanticGemmError, match="one GEMM kernel launch"):
        gemm_artifacts([], m, n, 64)
