"""Certified-numerics GEMM and attention entry points (the reference's
semantic GEMM / attention APIs, packages/browsergrad-kernels/src/
semantic_gemm.ts and semantic_attention.ts), on the HIP kernels.

Exact-f32 GEMM (semantic_gemm.ts:194-360 with the input certificate of
browsergrad-semantic-core/src/kernel/gemm-exact-input-artifact.ts):
``certify_exact_f32_gemm_inputs`` accepts lhs [m, k] and rhs [k, n] f32 only
when every element is a finite, non-negative (positive-zero), integer value
no larger than 2^24 and every output's sum of products stays within 2^24
(the profile "browsergrad.f32-exact-nonnegative-integer-gemm@1",
:25-26, 575-650); then any order of f32 additions gives the exact integer, so
the MFMA GEMM's result is bit-exact.  The certificate commits to the input
bytes with SHA-256 (as the reference's InputCommitment does, :41-45) and
``run_semantic_gemm_exact_f32`` refuses inputs that do not match it.

The sum bound is proved on the device instead of by the reference's
O(m n k) host loop: with non-negative terms the computed f32 sum is
monotone, so every computed output below 2^24 is the exact sum, and a
computed output >= 2^24 means the exact sum is >= 2^24; only in that case
does the host compute the exact int64 product to decide (the limit is
inclusive).

Attention (semantic_attention.ts:420; semantic-core
attention-forward-model.ts): dense rank-4 f32 scaled-dot-product attention
with an optional causal mask, online softmax, inputs and scaled scores
required finite; it runs on the f32 flash-attention kernel.

Verified artifacts (the reference composes layout, logical-tile and
schedule artifacts and reports their hashes in the trace,
semantic_gemm.ts:122-154, 193-214): each run here records the kernels the
library actually launched (bg_set_launch_log) and derives three artifacts
from them and from the problem:

* layout  -- every tensor's shape, element strides, dtype and byte length;
  checked dense row-major and sized exactly;
* logical tile -- the kernel's output tile (read from the launched kernel's
  template arguments), the tile grid and the K decomposition; checked to
  cover the output exactly once and the K range without gap;
* schedule -- the launches (kernel symbol, grid, workgroup, LDS, registers,
  scratch) and the workgroup-to-tile order; the GEMM's XCD-aware tile order
  is restated on the host and checked to be a bijection onto the tile grid.

Each artifact is canonical JSON (sorted keys, no spaces) hashed with
SHA-256; the trace carries the three hashes, the input certificate's hash
and a preparation hash over all of them.  An artifact whose check fails
raises BG-WEBGPU-GEMM-VALIDATION (attention: -ATTENTION-VALIDATION) before
any result is returned.
"""
from __future__ import annotations

import hashlib
import itertools
import json
import re
from typing import Any, Dict, List, Optional, Sequence

import numpy as np

EXACT_F32_INPUT_PROFILE = "browsergrad.f32-exact-nonnegative-integer-gemm@1"
EXACT_F32_INTEGER_LIMIT = 16_777_216
GEMM_PROFILE = "browsergrad.hip.gemm.exact-f32@1"
ATTENTION_PROFILE = "browsergrad.hip.attention.block-tiled-online-softmax-f32@1"
BACKEND_VERSION = "1.0.0"
_OPERATION_IDS = itertools.count(1)


class SemanticGemmError(Exception):
    """Error with the reference's code vocabulary (semantic_gemm.ts:161-191)."""

    def __init__(self, code: str, path: str, message: str) -> None:
        super().__init__(f"{code} at {path}: {message}")
        self.code = code
        self.path = path


class SemanticAttentionError(SemanticGemmError):
    """semantic_attention.ts:212-243 codes."""


def _f32_matrix(a: Any, rows: int, cols: int, path: str) -> np.ndarray:
    arr = np.frombuffer(a, dtype="<f4") if isinstance(a, (bytes, bytearray, memoryview)) else np.asarray(a)
    if arr.dtype != np.float32:
        raise SemanticGemmError("BG-WEBGPU-GEMM-INVALID-BINDING", path, f"expected float32 data, got {arr.dtype}")
    if arr.size != rows * cols:
        raise SemanticGemmError("BG-WEBGPU-GEMM-INVALID-BINDING", path,
                                f"expected {rows * cols} elements, got {arr.size}")
    return np.ascontiguousarray(arr.reshape(rows, cols))


def _check_exact_inputs(a: np.ndarray, path: str) -> None:
    """decodeExactInput (gemm-exact-input-artifact.ts:651-676) over a whole
    matrix: sign bit clear, finite, no nonzero subnormal, integer-valued,
    at most 2^24."""
    bits = a.view(np.uint32)
    bad = [
        ((bits >> 31) != 0, "exact f32 GEMM profile requires nonnegative inputs and canonical positive zero"),
        (((bits >> 23) & 0xFF) == 0xFF, "exact f32 GEMM profile rejects NaN and infinity"),
        ((((bits >> 23) & 0xFF) == 0) & ((bits & 0x7FFFFF) != 0),
         "exact f32 GEMM profile rejects nonzero subnormal and nonintegral inputs"),
    ]
    for mask, msg in bad:
        if mask.any():
            i = np.unravel_index(int(np.argmax(mask)), a.shape)
            raise SemanticGemmError("BG-WEBGPU-GEMM-NUMERICAL-PROOF", f"{path}[{i[0]},{i[1]}]", msg)
    with np.errstate(invalid="ignore"):
        nonint = a != np.floor(a)
    if nonint.any():
        i = np.unravel_index(int(np.argmax(nonint)), a.shape)
        raise SemanticGemmError("BG-WEBGPU-GEMM-NUMERICAL-PROOF", f"{path}[{i[0]},{i[1]}]",
                                "exact f32 GEMM profile requires integer-valued inputs")
    big = a > EXACT_F32_INTEGER_LIMIT
    if big.any():
        i = np.unravel_index(int(np.argmax(big)), a.shape)
        raise SemanticGemmError("BG-WEBGPU-GEMM-NUMERICAL-PROOF", f"{path}[{i[0]},{i[1]}]",
                                f"input integer {int(a[i])} exceeds the inclusive f32 integer limit "
                                f"{EXACT_F32_INTEGER_LIMIT}")


def _digest(a: np.ndarray) -> str:
    return hashlib.sha256(a.tobytes()).hexdigest()


def certify_exact_f32_gemm_inputs(lhs: Any, rhs: Any, m: int, n: int, k: int) -> Dict[str, Any]:
    """The input certificate of one exact-f32 GEMM (element checks on the
    host; the per-output sum bound is proved when the GEMM runs)."""
    for name, v in (("m", m), ("n", n), ("k", k)):
        if not isinstance(v, int) or v < 0:
            raise SemanticGemmError("BG-WEBGPU-GEMM-INVALID-BINDING", f"$.{name}", "must be a non-negative integer")
    a = _f32_matrix(lhs, m, k, "$.inputs.lhs")
    b = _f32_matrix(rhs, k, n, "$.inputs.rhs")
    _check_exact_inputs(a, "$.inputs.lhs")
    _check_exact_inputs(b, "$.inputs.rhs")
    return {
        "schema": "browsergrad.kernel.gemm-exact-f32-input",
        "profile": EXACT_F32_INPUT_PROFILE,
        "byteOrder": "little-endian",
        "exactIntegerLimit": EXACT_F32_INTEGER_LIMIT,
        "m": m, "n": n, "k": k,
        "inputs": {
            "lhs": {"algorithm": "sha256", "allocationByteLength": a.nbytes, "digest": _digest(a)},
            "rhs": {"algorithm": "sha256", "allocationByteLength": b.nbytes, "digest": _digest(b)},
        },
        "proof": {"products": "every-product-exact-f32", "partialSums": "every-subset-sum-exact-f32",
                  "f32Output": "bit-exact-on-certified-inputs"},
    }


# ---- verified artifacts --------------------------------------------------------

def canonical_hash(obj: Any) -> str:
    """SHA-256 of the canonical JSON of obj (sorted keys, no whitespace)."""
    return hashlib.sha256(json.dumps(obj, sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def _artifact(kind: str, body: Dict[str, Any], checks: List[str]) -> Dict[str, Any]:
    body = {"kind": kind, **body}
    return {"body": body, "hash": canonical_hash(body), "checks": checks}


def _fail(code: str, path: str, msg: str) -> None:
    cls = SemanticAttentionError if "ATTENTION" in code else SemanticGemmError
    raise cls(code, path, msg)


def layout_artifact(tensors: Dict[str, Dict[str, Any]], code: str) -> Dict[str, Any]:
    """Layout of dense row-major tensors {name: {shape, dtype}}; checked:
    strides are the dense row-major ones and the byte length is exact."""
    out = {}
    for name, t in sorted(tensors.items()):
        shape = [int(d) for d in t["shape"]]
        item = np.dtype(t["dtype"]).itemsize
        strides, acc = [], 1
        for d in reversed(shape):
            strides.insert(0, acc)
            acc *= d
        rec = {"shape": shape, "strides": strides, "dtype": t["dtype"], "byteLength": acc * item}
        if rec["byteLength"] != int(np.prod(shape, dtype=np.int64)) * item or (strides and strides[-1] != 1):
            _fail(code, f"$.layout.{name}", "layout is not dense row-major")
        out[name] = rec
    return _artifact("layout", {"tensors": out}, ["dense-row-major", "exact-byte-length"])


def gemm_tile_order(pid: int, tiles_m: int, tiles_n: int) -> tuple:
    """Host restatement of the GEMM kernels' workgroup -> tile map
    (k_gemm.hip tile_coords): workgroups go round-robin over the 8 XCDs, so
    the tiles of one XCD are made consecutive, then walked in groups of 4
    tile rows."""
    total = tiles_m * tiles_n
    if total % 8 == 0:
        per = total // 8
        pid = (pid % 8) * per + pid // 8
    g = 4
    group = pid // (g * tiles_n)
    first_m = group * g
    gsz = min(g, tiles_m - first_m)
    in_group = pid % (g * tiles_n)
    return first_m + in_group % gsz, in_group // gsz


_GEMM_KERNEL = re.compile(r"(gemm32_kernel|gemm16_lds_kernel|gemm16_kernel)ILi(\d+)ELi(\d+)E")


def gemm_artifacts(launches: Sequence[Dict[str, Any]], m: int, n: int, k: int) -> Dict[str, Dict[str, Any]]:
    """Logical-tile and schedule artifacts of one GEMM from its launch log."""
    code = "BG-WEBGPU-GEMM-VALIDATION"
    mains = [(r, _GEMM_KERNEL.search(r["kernel"])) for r in launches]
    mains = [(r, mt) for r, mt in mains if mt]
    if len(mains) != 1:
        _fail(code, "$.schedule", f"expected one GEMM kernel launch, saw {[r['kernel'] for r in launches]}")
    rec, mt = mains[0]
    bm, bn = int(mt.group(2)), int(mt.group(3))
    tiles_m, tiles_n = -(-m // bm), -(-n // bn)
    grid = rec["grid"]
    k_slices = int(grid[1])
    if grid[0] != tiles_m * tiles_n:
        _fail(code, "$.tile", f"grid.x {grid[0]} != {tiles_m} x {tiles_n} tiles of {bm}x{bn}")
    if not (tiles_m * bm >= m > (tiles_m - 1) * bm and tiles_n * bn >= n > (tiles_n - 1) * bn):
        _fail(code, "$.tile", "tile grid does not cover the output exactly once")
    seen = {gemm_tile_order(p, tiles_m, tiles_n) for p in range(tiles_m * tiles_n)}
    if len(seen) != tiles_m * tiles_n or not all(0 <= a < tiles_m and 0 <= b < tiles_n for a, b in seen):
        _fail(code, "$.schedule.tileOrder", "workgroup -> tile order is not a bijection onto the tile grid")
    tile = _artifact("logical-gemm-tile", {
        "m": m, "n": n, "k": k, "tile": {"m": bm, "n": bn}, "tilesM": tiles_m, "tilesN": tiles_n,
        "kSlices": k_slices,
        "accumulation": "f32; ascending k inside a slice; slices summed in slice order by a finishing pass"
                        if k_slices > 1 else "f32; ascending k",
    }, ["tiles-cover-output-once"])
    sched = _artifact("schedule", {
        "launches": [{kk: r[kk] for kk in ("kernel", "grid", "block", "dynamicLds", "staticLds", "vgprs",
                                          "scratchBytesPerLane")} for r in launches],
        "tileOrder": "xcd-round-robin-consecutive, groups of 4 tile rows",
    }, ["tile-order-bijection"])
    return {"tile": tile, "schedule": sched}


def attention_artifacts(launches: Sequence[Dict[str, Any]], rows: int) -> Dict[str, Dict[str, Any]]:
    """Logical-tile and schedule artifacts of the f32 attention kernel: one
    wavefront per query row, keys streamed in order."""
    code = "BG-WEBGPU-ATTENTION-VALIDATION"
    mains = [r for r in launches if "attention" in r["kernel"]]
    if len(mains) != 1:
        _fail(code, "$.schedule", f"expected one attention kernel launch, saw {[r['kernel'] for r in launches]}")
    r = mains[0]
    waves = int(r["block"][0]) // 64
    cover = int(r["grid"][0]) * waves
    if not (cover >= rows > cover - waves):
        _fail(code, "$.tile", f"{r['grid'][0]} workgroups x {waves} wavefronts do not cover {rows} query rows once")
    tile = _artifact("logical-attention-tile", {"queryRowsPerWavefront": 1, "wavefrontsPerWorkgroup": waves,
                                                "rows": rows, "keyOrder": "ascending, online softmax"},
                     ["rows-covered-once"])
    sched = _artifact("schedule", {
        "launches": [{kk: x[kk] for kk in ("kernel", "grid", "block", "dynamicLds", "staticLds", "vgprs",
                                          "scratchBytesPerLane")} for x in launches]}, ["one-launch"])
    return {"tile": tile, "schedule": sched}


def _trace_hashes(profile: str, layout: Dict[str, Any], arts: Dict[str, Dict[str, Any]],
                  certificate: Optional[Dict[str, Any]]) -> Dict[str, Any]:
    cert_hash = canonical_hash(certificate) if certificate is not None else None
    hashes = {"layoutSemanticHash": layout["hash"], "kernelSemanticHash": arts["tile"]["hash"],
              "scheduleSemanticHash": arts["schedule"]["hash"], "inputCertificateSemanticHash": cert_hash}
    hashes["backendPreparationHash"] = canonical_hash({"profile": profile, "version": BACKEND_VERSION, **hashes})
    hashes["artifacts"] = {"layout": layout, **arts}
    return hashes


def _run_logged(bridge: Any, fn):
    """Run fn() with the bridge's launch log on; returns (result, launches)."""
    bridge.set_launch_log(True)
    try:
        bridge.take_launch_log()  # drop anything older
        res = fn()
        return res, bridge.take_launch_log()
    finally:
        bridge.set_launch_log(False)


def _device_facts(bridge: Any) -> Dict[str, Any]:
    return {"backend": "hip", "architecture": "gfx950", "library": getattr(bridge, "version", lambda: "")()}


def run_semantic_gemm_exact_f32(bridge: Any, certificate: Dict[str, Any], lhs: Any, rhs: Any) -> Dict[str, Any]:
    """{"destination": f32 bytes of lhs @ rhs, "trace": {...}} for inputs
    matching ``certificate``; the GEMM runs on the f32 MFMA kernel."""
    if not isinstance(certificate, dict) or certificate.get("profile") != EXACT_F32_INPUT_PROFILE:
        raise SemanticGemmError("BG-WEBGPU-GEMM-UNSUPPORTED-PROFILE", "$.certificate",
                                f"expected a {EXACT_F32_INPUT_PROFILE} certificate")
    m, n, k = int(certificate["m"]), int(certificate["n"]), int(certificate["k"])
    a = _f32_matrix(lhs, m, k, "$.inputs.lhs")
    b = _f32_matrix(rhs, k, n, "$.inputs.rhs")
    for name, arr in (("lhs", a), ("rhs", b)):
        if _digest(arr) != certificate["inputs"][name]["digest"]:
            raise SemanticGemmError("BG-WEBGPU-GEMM-INVALID-BINDING", f"$.inputs.{name}",
                                    "input bytes do not match the certificate's commitment")
    launches: List[Dict[str, Any]] = []
    if m == 0 or n == 0:
        out = np.zeros((m, n), np.float32)
    else:
        ha = bridge.upload(a, a.shape, "float32")
        hb = bridge.upload(b, b.shape, "float32")
        try:
            if k == 0:
                out = np.zeros((m, n), np.float32)
            else:
                hc, launches = _run_logged(
                    bridge, lambda: bridge.matmul_ex(ha, hb, m=m, n=n, k=k, in_dtype="float32", out_dtype="float32"))
                try:
                    out = bridge.to_numpy(hc)
                finally:
                    bridge.release(hc)
        finally:
            bridge.release(ha)
            bridge.release(hb)
    if out.size and float(out.max()) >= EXACT_F32_INTEGER_LIMIT:
        exact = a.astype(np.int64) @ b.astype(np.int64)
        worst = int(exact.max())
        if worst > EXACT_F32_INTEGER_LIMIT:
            r, c = np.unravel_index(int(np.argmax(exact)), exact.shape)
            raise SemanticGemmError("BG-WEBGPU-GEMM-NUMERICAL-PROOF", f"$.proof.output[{r},{c}]",
                                    f"nonnegative product total {worst} exceeds the inclusive f32 integer limit "
                                    f"{EXACT_F32_INTEGER_LIMIT}")
    trace = {
        "operationId": f"hip-gemm-{next(_OPERATION_IDS)}",
        "backendProfile": GEMM_PROFILE,
        "backendVersion": BACKEND_VERSION,
        "executionTier": "mi355x-hip-mfma-f32",
        "numericalInputProfile": EXACT_F32_INPUT_PROFILE,
        "numericalPreservation": "bit-exact-on-certified-inputs",
        "inputCertificateDigests": {x: certificate["inputs"][x]["digest"] for x in ("lhs", "rhs")},
        "m": m, "n": n, "k": k,
        "multiplyAdds": m * n * k,
        "logicalBytesRead": 4 * (m * k + k * n),
        "logicalBytesWritten": 4 * m * n,
        "submitted": True,
        "device": _device_facts(bridge),
    }
    if launches:
        layout = layout_artifact({"lhs": {"shape": [m, k], "dtype": "float32"},
                                  "rhs": {"shape": [k, n], "dtype": "float32"},
                                  "output": {"shape": [m, n], "dtype": "float32"}}, "BG-WEBGPU-GEMM-VALIDATION")
        trace.update(_trace_hashes(GEMM_PROFILE, layout, gemm_artifacts(launches, m, n, k), certificate))
    return {"destination": np.ascontiguousarray(out, np.float32).tobytes(), "trace": trace}


def run_semantic_attention_f32(bridge: Any, query: Any, key: Any, value: Any, *, batch: int, heads: int,
                               q_len: int, k_len: int, head_dim: int, scale: Optional[float] = None,
                               causal: bool = False) -> Dict[str, Any]:
    """{"destination": f32 bytes [batch, heads, q_len, head_dim], "trace"}:
    softmax(q k^T * scale [causal]) v in f32 with online softmax.  Inputs
    must be finite (the finite-domain validation of semantic_attention.ts),
    and so must the result (non-finite scaled scores are refused)."""
    def arr(x: Any, s: int, path: str) -> np.ndarray:
        a = np.frombuffer(x, dtype="<f4") if isinstance(x, (bytes, bytearray, memoryview)) else np.asarray(x)
        if a.dtype != np.float32 or a.size != batch * heads * s * head_dim:
            raise SemanticAttentionError("BG-WEBGPU-ATTENTION-INVALID-BINDING", path,
                                         f"expected {batch * heads * s * head_dim} float32 elements")
        if not np.isfinite(a).all():
            raise SemanticAttentionError("BG-WEBGPU-ATTENTION-NUMERICAL-PROOF", path, "inputs must be finite f32")
        return np.ascontiguousarray(a.reshape(batch, heads, s, head_dim))

    q = arr(query, q_len, "$.inputs.query")
    k = arr(key, k_len, "$.inputs.key")
    v = arr(value, k_len, "$.inputs.value")
    sc = float(np.float32(scale if scale is not None else 1.0 / np.sqrt(head_dim)))
    if not (sc > 0 and np.isfinite(sc)):
        raise SemanticAttentionError("BG-WEBGPU-ATTENTION-NUMERICAL-PROOF", "$.scale", "scale must be positive finite")
    if causal and q_len > k_len:
        raise SemanticAttentionError("BG-WEBGPU-ATTENTION-INVALID-BINDING", "$.mask",
                                     "causal attention needs q_len <= k_len")
    hs = [bridge.upload(t, t.shape, "float32") for t in (q, k, v)]
    try:
        ho, launches = _run_logged(bridge, lambda: bridge.attention_ex(
            hs[0], hs[1], hs[2], batch=batch, heads=heads, sq=q_len, sk=k_len, d=head_dim, scale=sc,
            causal=causal, in_dtype="float32", out_dtype="float32"))
        try:
            out = bridge.to_numpy(ho)
        finally:
            bridge.release(ho)
    finally:
        for h in hs:
            bridge.release(h)
    if not np.isfinite(out).all():
        raise SemanticAttentionError("BG-WEBGPU-ATTENTION-NUMERICAL-PROOF", "$.output",
                                     "scaled scores or the result left the finite f32 domain")
    trace = {
        "operationId": f"hip-attention-{next(_OPERATION_IDS)}",
        "backendProfile": ATTENTION_PROFILE,
        "backendVersion": BACKEND_VERSION,
        "executionTier": "mi355x-hip-flash-attention-f32",
        "mask": "causal" if causal else "none",
        "scaleBits": f"{np.float32(sc).view(np.uint32):08x}",
        "batch": batch, "heads": heads, "queryLength": q_len, "keyLength": k_len, "headDim": head_dim,
        "logicalBytesRead": 4 * (q.size + k.size + v.size),
        "logicalBytesWritten": 4 * out.size,
        "submitted": True,
        "device": _device_facts(bridge),
    }
    shp = lambda s_: [batch, heads, s_, head_dim]  # noqa: E731
    layout = layout_artifact({"query": {"shape": shp(q_len), "dtype": "float32"},
                              "key": {"shape": shp(k_len), "dtype": "float32"},
                              "value": {"shape": shp(k_len), "dtype": "float32"},
                              "output": {"shape": shp(q_len), "dtype": "float32"}}, "BG-WEBGPU-ATTENTION-VALIDATION")
    trace.update(_trace_hashes(ATTENTION_PROFILE, layout, attention_artifacts(launches, batch * heads * q_len),
                               None))
    return {"destination": out.astype(np.float32).tobytes(), "trace": trace}


__all__ = ["certify_exact_f32_gemm_inputs", "run_semantic_gemm_exact_f32", "run_semantic_attention_f32",
           "SemanticGemmError", "SemanticAttentionError", "EXACT_F32_INPUT_PROFILE", "EXACT_F32_INTEGER_LIMIT",
           "canonical_hash", "layout_artifact", "gemm_artifacts", "attention_artifacts", "gemm_tile_order"]
