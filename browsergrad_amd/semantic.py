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

Prepare, then run (prepareSemanticGemmWgsl / runSemanticGemmWebGpu,
semantic_gemm.ts:194-420; prepareSemanticAttentionWgsl /
runSemanticAttentionWebGpu, semantic_attention.ts:245-520).
``prepare_semantic_gemm`` / ``prepare_semantic_attention`` ask the library
which kernels it will launch for the problem (bg_matmul_launch_plan /
bg_attention_launch_plan: host-only, no device) and build three artifacts
from that answer before anything runs:

* layout -- every tensor's shape, element strides, dtype and byte length
  (declared dense row-major; each run compares it with the bridge's records
  of the handles it actually used);
* logical tile -- the output tile, tile grid and K decomposition (GEMM) or
  query blocks, key tiles and padded head dim (attention); checked to cover
  the output once;
* schedule -- the launches (kernel, template arguments, grid, workgroup),
  LDS and workspace; the GEMM's XCD-aware tile order is restated on the host
  and checked to be a bijection onto the tile grid.

Each artifact is canonical JSON (sorted keys, no spaces) hashed with
SHA-256; the preparation hash covers all three and is the same for every
run of one prepared object.  Preparation enforces the caller's working-set
limit and this device's workgroup limits (RESOURCE-LIMIT).  A run takes
only prepared objects, uploads fresh copies of the validated host bytes,
honours a wait budget and a cancellation event, and refuses
(VALIDATION) when its launch log differs from the prepared schedule.  The
resident seams are closed, as in the reference: a host-side certificate
cannot prove what resident device buffers hold.
"""
from __future__ import annotations

import hashlib
import itertools
import json
import re
import time
import weakref
from dataclasses import dataclass
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


def layout_artifact(tensors: Dict[str, Dict[str, Any]]) -> Dict[str, Any]:
    """Declared layout of dense row-major tensors {name: {shape, dtype}}:
    shape, element strides, dtype and byte length.  A run checks it against
    the device records of the handles it actually used (check_layout)."""
    out = {}
    for name, t in sorted(tensors.items()):
        shape = [int(d) for d in t["shape"]]
        item = np.dtype(t["dtype"]).itemsize
        strides, acc = [], 1
        for d in reversed(shape):
            strides.insert(0, acc)
            acc *= d
        out[name] = {"shape": shape, "strides": strides, "dtype": t["dtype"], "byteLength": acc * item}
    return _artifact("layout", {"tensors": out}, ["declared-dense-row-major", "device-records-at-run"])


def check_layout(layout: Dict[str, Any], infos: Dict[str, Dict[str, Any]], code: str) -> None:
    """Compare the prepared layout with what the bridge recorded for the
    handles a run used ({name: handle_info()}: shape, dtype, nbytes)."""
    for name, rec in layout["body"]["tensors"].items():
        got = infos[name]
        if list(got["shape"]) != rec["shape"] or got["dtype"] != rec["dtype"] or int(got["nbytes"]) != rec["byteLength"]:
            _fail(code, f"$.layout.{name}",
                  f"device record {dict(shape=list(got['shape']), dtype=got['dtype'], nbytes=int(got['nbytes']))} "
                  f"does not match the prepared layout {rec}")


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


def launch_plan(kind: str, desc: Any) -> Dict[str, Any]:
    """The launches libbghip will make for a call (bg_matmul_launch_plan /
    bg_attention_launch_plan: host only, no device), as plain data."""
    import ctypes as C
    from . import _native as N
    lib = N.load_library()
    plan = N.LaunchPlan()
    err = C.create_string_buffer(512)
    fn = lib.bg_matmul_launch_plan if kind == "gemm" else lib.bg_attention_launch_plan
    rc = fn(C.byref(desc), C.byref(plan), err, len(err))
    if rc != N.BG_OK:
        _fail("BG-WEBGPU-GEMM-UNSUPPORTED-PROFILE" if kind == "gemm" else "BG-WEBGPU-ATTENTION-UNSUPPORTED-PROFILE",
              "$.launch", err.value.decode())
    launches = []
    for i in range(plan.n_launches):
        e = plan.launch[i]
        launches.append({"family": e.family.decode(), "templateArgs": [int(e.targs[j]) for j in range(e.n_targs)],
                         "grid": [int(x) for x in e.grid], "block": [int(x) for x in e.block]})
    return {"launches": launches, "tile": [plan.tile_m, plan.tile_n, plan.tile_k], "kSlices": plan.k_slices,
            "ldsBytes": int(plan.lds_bytes), "workspaceBytes": int(plan.workspace_bytes)}


_TARG = re.compile(r"L([a-z])(n?)(\d+)E")


def parse_kernel_symbol(name: str, family: str) -> Optional[List[int]]:
    """Template arguments of `family` in a launch-log kernel name, mangled
    (..15fa32_fwd_kernelILi64ELb1EEEv...) or demangled
    (fa32_fwd_kernel<64, true>(...)); [] for a kernel without template
    arguments; None when the name is another kernel."""
    m = re.search(re.escape(family) + r"I((?:L[a-z]n?\d+E)+)E", name)
    if m:
        return [(-1 if neg else 1) * int(v) for _, neg, v in _TARG.findall(m.group(1))]
    m = re.search(re.escape(family) + r"<([^<>]*)>", name)
    if m:
        vals = []
        for tok in m.group(1).split(","):
            tok = tok.strip()
            vals.append(1 if tok == "true" else 0 if tok == "false" else int(tok))
        return vals
    # A kernel without template arguments: mangled ..25name + E (end of the
    # nested name), or demangled name(...).
    if re.search(r"\d" + re.escape(family) + r"E", name) or re.search(
            r"(?:^|[^A-Za-z0-9_])" + re.escape(family) + r"\(", name):
        return []
    return None


def check_launches(plan: Dict[str, Any], launches: Sequence[Dict[str, Any]], code: str) -> None:
    """The run's launch log must be exactly the prepared schedule: the same
    kernels, in order, with the same template arguments, grids and
    workgroup sizes."""
    want = plan["launches"]
    if len(launches) != len(want):
        _fail(code, "$.schedule", f"prepared {len(want)} launch(es), the run made {len(launches)}: "
                                  f"{[r['kernel'] for r in launches]}")
    for i, (w, r) in enumerate(zip(want, launches)):
        args = parse_kernel_symbol(r["kernel"], w["family"])
        if args != w["templateArgs"] or list(r["grid"]) != w["grid"] or list(r["block"]) != w["block"]:
            _fail(code, f"$.schedule.launches[{i}]",
                  f"ran {r['kernel']} grid {list(r['grid'])} block {list(r['block'])}; prepared {w}")


def _positive(value: Any, default: int, ceiling: int, path: str, code: str) -> int:
    if value is None:
        return default
    if isinstance(value, bool) or not isinstance(value, int) or value <= 0 or value > ceiling:
        _fail(code, path, f"must be a positive integer no larger than {ceiling}")
    return int(value)


# Limits of a preparation.  Working set: the reference's bounds
# (semantic_gemm.ts:47-48).  Workgroup limits are this device's (gfx950: at
# most 1024 invocations and 160 KiB of LDS per workgroup), not WebGPU's
# (semantic_gemm.ts:43-46).  Run wait budget: semantic_gemm.ts:49-50.
DEFAULT_MAX_TRANSIENT_WORKING_SET_BYTES = 256 * 1024 * 1024
MAX_CONFIGURABLE_TRANSIENT_WORKING_SET_BYTES = 1024 * 1024 * 1024
DEVICE_MAX_WORKGROUP_INVOCATIONS = 1024
DEVICE_MAX_WORKGROUP_STORAGE_BYTES = 160 * 1024
DEFAULT_EXECUTION_TIMEOUT_MS = 30_000
MAX_EXECUTION_TIMEOUT_MS = 5 * 60_000


@dataclass(frozen=True, eq=False)
class PreparedSemanticGemm:
    """A prepared exact-f32 GEMM specialization (prepareSemanticGemmWgsl,
    semantic_gemm.ts:194-340): its artifacts and their hashes are fixed
    before anything runs; run_semantic_gemm checks each run against them."""
    m: int
    n: int
    k: int
    backendProfile: str
    backendVersion: str
    layout: Dict[str, Any]
    tile: Dict[str, Any]
    schedule: Dict[str, Any]
    plan: Dict[str, Any]
    backendPreparationHash: str
    workgroupStorageBytes: int
    plannedTransientGpuBytes: int
    plannedTransientHostBytes: int
    plannedTransientWorkingSetBytes: int
    maxTransientWorkingSetBytes: int


@dataclass(frozen=True, eq=False)
class PreparedSemanticAttention:
    """A prepared f32 attention specialization (prepareSemanticAttentionWgsl,
    semantic_attention.ts:245-413)."""
    batch: int
    heads: int
    q_len: int
    k_len: int
    head_dim: int
    scale: float
    causal: bool
    backendProfile: str
    backendVersion: str
    layout: Dict[str, Any]
    tile: Dict[str, Any]
    schedule: Dict[str, Any]
    plan: Dict[str, Any]
    backendPreparationHash: str
    workgroupStorageBytes: int
    plannedTransientGpuBytes: int
    plannedTransientHostBytes: int
    plannedTransientWorkingSetBytes: int
    maxTransientWorkingSetBytes: int


_PREPARED: "weakref.WeakSet[Any]" = weakref.WeakSet()


def _require_prepared(prepared: Any, cls: type, code: str) -> None:
    if not isinstance(prepared, cls) or prepared not in _PREPARED:
        _fail(code, "$.prepared", f"expected a {cls.__name__} returned by its prepare function")


def _workgroup_limits(plan: Dict[str, Any], max_inv: Any, max_lds: Any, code: str) -> int:
    inv = _positive(max_inv, DEVICE_MAX_WORKGROUP_INVOCATIONS, DEVICE_MAX_WORKGROUP_INVOCATIONS,
                    "$.maxWorkgroupInvocations", code)
    lds = _positive(max_lds, DEVICE_MAX_WORKGROUP_STORAGE_BYTES, DEVICE_MAX_WORKGROUP_STORAGE_BYTES,
                    "$.maxWorkgroupStorageBytes", code)
    for i, l in enumerate(plan["launches"]):
        n = l["block"][0] * l["block"][1] * l["block"][2]
        if n > inv:
            _fail(code.replace("VALIDATION", "RESOURCE-LIMIT"), "$.maxWorkgroupInvocations",
                  f"launch {i} ({l['family']}) uses {n} invocations per workgroup; limit is {inv}")
    if plan["ldsBytes"] > lds:
        _fail(code.replace("VALIDATION", "RESOURCE-LIMIT"), "$.maxWorkgroupStorageBytes",
              f"the kernel stages {plan['ldsBytes']} bytes in LDS per workgroup; limit is {lds}")
    return int(plan["ldsBytes"])


def prepare_semantic_gemm(m: int, n: int, k: int, *, max_transient_working_set_bytes: Optional[int] = None,
                          max_workgroup_invocations: Optional[int] = None,
                          max_workgroup_storage_bytes: Optional[int] = None) -> PreparedSemanticGemm:
    """Fix the kernels, tile schedule and working set of an m x n x k
    exact-f32 GEMM before any launch, check them (tiles cover the output
    once, the XCD tile order is a bijection, device and caller limits), and
    hash them.  Needs libbghip.so but no device."""
    from . import _native as N
    code = "BG-WEBGPU-GEMM-VALIDATION"
    for name, v in (("m", m), ("n", n), ("k", k)):
        if isinstance(v, bool) or not isinstance(v, int) or v <= 0:
            _fail("BG-WEBGPU-GEMM-INVALID-BINDING", f"$.{name}", "must be a positive integer")
    cap = _positive(max_transient_working_set_bytes, DEFAULT_MAX_TRANSIENT_WORKING_SET_BYTES,
                    MAX_CONFIGURABLE_TRANSIENT_WORKING_SET_BYTES, "$.maxTransientWorkingSetBytes",
                    "BG-WEBGPU-GEMM-RESOURCE-LIMIT")
    d = N.MatmulDesc()
    d.batch, d.m, d.n, d.k = 1, m, n, k
    d.lda, d.ldb, d.ldc = k, n, n
    d.trans_b, d.in_dtype, d.out_dtype = 0, N.BG_F32, N.BG_F32
    plan = launch_plan("gemm", d)
    lds = _workgroup_limits(plan, max_workgroup_invocations, max_workgroup_storage_bytes, code)
    main = plan["launches"][0]
    bm, bn, bk = plan["tile"]
    tiles_m, tiles_n = -(-m // bm), -(-n // bn)
    wide = main["family"] == "gemm32_wide_k_kernel"
    skinny = main["family"] == "gemm_skinny_kernel"
    slices = plan["kSlices"]
    # The skinny kernel runs each column tile once per K slice (grid x) and
    # row block (grid y).
    per_launch = tiles_n * slices if skinny else tiles_m * tiles_n
    if main["grid"][0] != per_launch or (skinny and main["grid"][1] != tiles_m) or not (
            tiles_m * bm >= m > (tiles_m - 1) * bm and tiles_n * bn >= n > (tiles_n - 1) * bn):
        _fail(code, "$.tile", f"{main['grid'][0]} workgroups do not cover {m} x {n} once with {bm} x {bn} tiles")
    # Workgroup -> tile: the wide-K kernel walks tiles row-major; the skinny
    # one takes row block y and, for workgroup x, column tile x // kSlices
    # and K slice x % kSlices; the others use the XCD-aware order restated
    # by gemm_tile_order.
    if wide or skinny:
        order = lambda p: (p // tiles_n, p % tiles_n)  # noqa: E731
    else:
        order = lambda p: gemm_tile_order(p, tiles_m, tiles_n)  # noqa: E731
    seen = {order(p) for p in range(tiles_m * tiles_n)}
    if len(seen) != tiles_m * tiles_n or not all(0 <= a < tiles_m and 0 <= b < tiles_n for a, b in seen):
        _fail(code, "$.schedule.tileOrder", "workgroup -> tile order is not a bijection onto the tile grid")
    if wide and (slices != main["block"][0] // 64 or len(plan["launches"]) != 1 or plan["workspaceBytes"] != 0):
        _fail(code, "$.tile.kSlices", f"{slices} in-workgroup K slices need one wavefront each and one launch")
    if skinny and (bm > 64 or len(plan["launches"]) != (2 if slices > 1 else 1)
                   or plan["workspaceBytes"] != (4 * slices * m * n if slices > 1 else 0)):
        _fail(code, "$.tile.kSlices", f"{slices} K slices need one f32 partial each and a summing launch")
    if not wide and not skinny and (slices != 1 or len(plan["launches"]) != 1):
        _fail(code, "$.tile.kSlices", "the tiled kernel runs the whole K range in one launch")
    layout = layout_artifact({"lhs": {"shape": [m, k], "dtype": "float32"},
                              "rhs": {"shape": [k, n], "dtype": "float32"},
                              "output": {"shape": [m, n], "dtype": "float32"}})
    tile = _artifact("logical-gemm-tile", {
        "m": m, "n": n, "k": k, "tile": {"m": bm, "n": bn, "k": bk}, "tilesM": tiles_m, "tilesN": tiles_n,
        "kSlices": slices,
        "accumulation": ("f32; each of the workgroup's wavefronts sums a contiguous run of 8-wide k chunks in "
                         "ascending order; the partials are added in wavefront order through LDS")
                        if wide else
                        ("f32; per K slice, four wavefronts sum every fourth 8-deep k step in ascending order and "
                         "are added in wavefront order through LDS; the slices' partials are added in slice order")
                        if skinny else "f32; ascending k",
    }, ["tiles-cover-output-once", "k-slices-one-per-wavefront"])
    schedule = _artifact("schedule", {
        "launches": plan["launches"], "ldsBytes": plan["ldsBytes"], "workspaceBytes": plan["workspaceBytes"],
        "tileOrder": "row-major" if wide else "row block y; column tile x // kSlices, K slice x % kSlices"
                     if skinny
                     else "xcd-round-robin-consecutive, groups of 4 tile rows",
    }, ["tile-order-bijection", "within-workgroup-limits"])
    gpu = 4 * (m * k + k * n + m * n) + plan["workspaceBytes"]
    host = 4 * (m * k + k * n) + 2 * 4 * m * n  # certified input copies, readback, returned bytes
    if gpu + host > cap:
        _fail("BG-WEBGPU-GEMM-RESOURCE-LIMIT", "$.maxTransientWorkingSetBytes",
              f"planned owned host and GPU buffers require {gpu + host} bytes; limit is {cap}")
    prep_hash = canonical_hash({"profile": GEMM_PROFILE, "version": BACKEND_VERSION, "layout": layout["hash"],
                                "tile": tile["hash"], "schedule": schedule["hash"], "workgroupStorageBytes": lds})
    prepared = PreparedSemanticGemm(m, n, k, GEMM_PROFILE, BACKEND_VERSION, layout, tile, schedule, plan, prep_hash,
                                    lds, gpu, host, gpu + host, cap)
    _PREPARED.add(prepared)
    return prepared


def prepare_semantic_attention(batch: int, heads: int, q_len: int, k_len: int, head_dim: int, *,
                               scale: Optional[float] = None, causal: bool = False,
                               max_transient_working_set_bytes: Optional[int] = None,
                               max_workgroup_invocations: Optional[int] = None,
                               max_workgroup_storage_bytes: Optional[int] = None) -> PreparedSemanticAttention:
    """Fix the kernel, query/key tiling and working set of a dense f32
    attention before any launch, check that the query blocks cover every
    row once and the limits hold, and hash the artifacts."""
    from . import _native as N
    code = "BG-WEBGPU-ATTENTION-VALIDATION"
    for name, v in (("batch", batch), ("heads", heads), ("q_len", q_len), ("k_len", k_len),
                    ("head_dim", head_dim)):
        if isinstance(v, bool) or not isinstance(v, int) or v <= 0:
            _fail("BG-WEBGPU-ATTENTION-INVALID-BINDING", f"$.{name}", "must be a positive integer")
    sc = float(np.float32(scale if scale is not None else 1.0 / np.sqrt(head_dim)))
    if not (sc > 0 and np.isfinite(sc)):
        _fail("BG-WEBGPU-ATTENTION-NUMERICAL-PROOF", "$.scale", "scale must be positive finite")
    if causal and q_len > k_len:
        _fail("BG-WEBGPU-ATTENTION-INVALID-BINDING", "$.mask", "causal attention needs q_len <= k_len")
    cap = _positive(max_transient_working_set_bytes, DEFAULT_MAX_TRANSIENT_WORKING_SET_BYTES,
                    MAX_CONFIGURABLE_TRANSIENT_WORKING_SET_BYTES, "$.maxTransientWorkingSetBytes",
                    "BG-WEBGPU-ATTENTION-RESOURCE-LIMIT")
    d = N.AttentionDesc()
    d.batch, d.heads, d.sq, d.sk, d.d = batch, heads, q_len, k_len, head_dim
    d.scale, d.causal = sc, 1 if causal else 0
    d.in_dtype = d.out_dtype = N.BG_F32
    plan = launch_plan("attention", d)
    lds = _workgroup_limits(plan, max_workgroup_invocations, max_workgroup_storage_bytes, code)
    main = plan["launches"][0]
    bq, bk, dp = plan["tile"]
    nqb = int(main["grid"][1])
    if main["grid"][0] != batch * heads or not (nqb * bq >= q_len > (nqb - 1) * bq) or dp < head_dim:
        _fail(code, "$.tile", f"grid {main['grid']} of {bq}-query blocks does not cover {batch * heads} heads x "
                              f"{q_len} rows once")
    shp = lambda s_: [batch, heads, s_, head_dim]  # noqa: E731
    layout = layout_artifact({"query": {"shape": shp(q_len), "dtype": "float32"},
                              "key": {"shape": shp(k_len), "dtype": "float32"},
                              "value": {"shape": shp(k_len), "dtype": "float32"},
                              "output": {"shape": shp(q_len), "dtype": "float32"}})
    tile = _artifact("logical-attention-tile", {
        "queriesPerWorkgroup": bq, "queriesPerWavefront": 32, "keysPerTile": bk, "paddedHeadDim": dp,
        "rows": batch * heads * q_len, "queryBlocks": nqb,
        "keyOrder": "ascending; online softmax with an exact running max per 32 keys",
        "mask": "causal" if causal else "none",
    }, ["rows-covered-once", "head-dim-fits-padding"])
    schedule = _artifact("schedule", {"launches": plan["launches"], "ldsBytes": plan["ldsBytes"],
                                      "workgroupOrder": "heaviest query blocks first"},
                         ["one-launch", "within-workgroup-limits"])
    inputs = 4 * batch * heads * head_dim * (q_len + 2 * k_len)
    out_b = 4 * batch * heads * q_len * head_dim
    gpu, host = inputs + out_b, inputs + 2 * out_b
    if gpu + host > cap:
        _fail("BG-WEBGPU-ATTENTION-RESOURCE-LIMIT", "$.maxTransientWorkingSetBytes",
              f"planned owned host and GPU buffers require {gpu + host} bytes; limit is {cap}")
    prep_hash = canonical_hash({"profile": ATTENTION_PROFILE, "version": BACKEND_VERSION, "layout": layout["hash"],
                                "tile": tile["hash"], "schedule": schedule["hash"], "workgroupStorageBytes": lds,
                                "scaleBits": f"{np.float32(sc).view(np.uint32):08x}"})
    prepared = PreparedSemanticAttention(batch, heads, q_len, k_len, head_dim, sc, bool(causal), ATTENTION_PROFILE,
                                         BACKEND_VERSION, layout, tile, schedule, plan, prep_hash, lds, gpu, host,
                                         gpu + host, cap)
    _PREPARED.add(prepared)
    return prepared


class _Deadline:
    """Caller wait budget and cancellation of one run (the reference's
    timeoutMs / AbortSignal, semantic_gemm.ts:110-120): checked before the
    upload, before the launch and once the result is back; a cancelled or
    late run returns no result."""

    def __init__(self, timeout_ms: Any, cancel: Any, kind: str) -> None:
        self.code = f"BG-WEBGPU-{kind}"
        self.ms = _positive(timeout_ms, DEFAULT_EXECUTION_TIMEOUT_MS, MAX_EXECUTION_TIMEOUT_MS, "$.timeoutMs",
                            f"{self.code}-INVALID-BINDING")
        if cancel is not None and not callable(getattr(cancel, "is_set", None)):
            _fail(f"{self.code}-INVALID-BINDING", "$.cancel", "cancel must provide is_set() (threading.Event)")
        self.cancel = cancel
        self.t0 = time.monotonic()

    def check(self) -> None:
        if self.cancel is not None and self.cancel.is_set():
            _fail(f"{self.code}-CANCELLED", "$.cancel", "the run was cancelled")
        if (time.monotonic() - self.t0) * 1e3 > self.ms:
            _fail(f"{self.code}-TIMEOUT", "$.timeoutMs", f"the run exceeded the caller wait budget of {self.ms} ms")


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


def _trace_hashes(prepared: Any, certificate: Optional[Dict[str, Any]]) -> Dict[str, Any]:
    return {"layoutSemanticHash": prepared.layout["hash"], "kernelSemanticHash": prepared.tile["hash"],
            "scheduleSemanticHash": prepared.schedule["hash"],
            "inputCertificateSemanticHash": canonical_hash(certificate) if certificate is not None else None,
            "backendPreparationHash": prepared.backendPreparationHash,
            "artifacts": {"layout": prepared.layout, "tile": prepared.tile, "schedule": prepared.schedule},
            "plannedTransientWorkingSetBytes": prepared.plannedTransientWorkingSetBytes,
            "maxTransientWorkingSetBytes": prepared.maxTransientWorkingSetBytes}


def run_prepared_semantic_gemm_resident(prepared: PreparedSemanticGemm, inputs: Any) -> None:
    """Closed, as in the reference (semantic_gemm.ts:341-356): a certificate
    over host bytes cannot prove what resident device buffers hold now."""
    _require_prepared(prepared, PreparedSemanticGemm, "BG-WEBGPU-GEMM-INVALID-BINDING")
    _fail("BG-WEBGPU-GEMM-NUMERICAL-PROOF", "$.inputs",
          "resident GEMM requires trusted input provenance; a host-byte certificate cannot prove current "
          "device buffer contents")


def run_semantic_gemm(bridge: Any, prepared: PreparedSemanticGemm, certificate: Dict[str, Any], lhs: Any, rhs: Any,
                      *, timeout_ms: Optional[int] = None, cancel: Any = None) -> Dict[str, Any]:
    """{"destination": f32 bytes of lhs @ rhs, "trace"} for certified inputs
    on a prepared specialization (runSemanticGemmWebGpu,
    semantic_gemm.ts:358-420): fresh uploads of the certified bytes, the
    prepared launches only (the launch log must match the schedule), the
    device records of every handle checked against the prepared layout."""
    _require_prepared(prepared, PreparedSemanticGemm, "BG-WEBGPU-GEMM-INVALID-BINDING")
    dl = _Deadline(timeout_ms, cancel, "GEMM")
    if not isinstance(certificate, dict) or certificate.get("profile") != EXACT_F32_INPUT_PROFILE:
        raise SemanticGemmError("BG-WEBGPU-GEMM-UNSUPPORTED-PROFILE", "$.certificate",
                                f"expected a {EXACT_F32_INPUT_PROFILE} certificate")
    m, n, k = prepared.m, prepared.n, prepared.k
    if (int(certificate["m"]), int(certificate["n"]), int(certificate["k"])) != (m, n, k):
        raise SemanticGemmError("BG-WEBGPU-GEMM-INVALID-BINDING", "$.certificate",
                                f"certificate is for {certificate['m']} x {certificate['n']} x {certificate['k']}, "
                                f"the preparation for {m} x {n} x {k}")
    a = _f32_matrix(lhs, m, k, "$.inputs.lhs")
    b = _f32_matrix(rhs, k, n, "$.inputs.rhs")
    for name, arr in (("lhs", a), ("rhs", b)):
        if _digest(arr) != certificate["inputs"][name]["digest"]:
            raise SemanticGemmError("BG-WEBGPU-GEMM-INVALID-BINDING", f"$.inputs.{name}",
                                    "input bytes do not match the certificate's commitment")
    dl.check()
    ha = bridge.upload(a, a.shape, "float32")
    hb = bridge.upload(b, b.shape, "float32")
    try:
        dl.check()
        hc, launches = _run_logged(
            bridge, lambda: bridge.matmul_ex(ha, hb, m=m, n=n, k=k, in_dtype="float32", out_dtype="float32"))
        try:
            check_launches(prepared.plan, launches, "BG-WEBGPU-GEMM-VALIDATION")
            check_layout(prepared.layout, {"lhs": bridge.handle_info(ha), "rhs": bridge.handle_info(hb),
                                           "output": bridge.handle_info(hc)}, "BG-WEBGPU-GEMM-VALIDATION")
            out = bridge.to_numpy(hc)
        finally:
            bridge.release(hc)
    finally:
        bridge.release(ha)
        bridge.release(hb)
    dl.check()
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
        "physicalTile": prepared.tile["body"]["tile"],
        "dispatchWorkgroups": prepared.plan["launches"][0]["grid"],
        "multiplyAdds": m * n * k,
        "logicalBytesRead": 4 * (m * k + k * n),
        "logicalBytesWritten": 4 * m * n,
        "submitted": True,
        "device": _device_facts(bridge),
        "launchesMatchedPreparation": True,
    }
    trace.update(_trace_hashes(prepared, certificate))
    return {"destination": np.ascontiguousarray(out, np.float32).tobytes(), "trace": trace}


def run_semantic_gemm_exact_f32(bridge: Any, certificate: Dict[str, Any], lhs: Any, rhs: Any) -> Dict[str, Any]:
    """One-shot form: prepare for the certificate's shape, then run."""
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
    if m == 0 or n == 0 or k == 0:  # nothing to launch: the exact result is zeros
        return {"destination": np.zeros((m, n), np.float32).tobytes(),
                "trace": {"operationId": f"hip-gemm-{next(_OPERATION_IDS)}", "backendProfile": GEMM_PROFILE,
                          "backendVersion": BACKEND_VERSION, "m": m, "n": n, "k": k, "multiplyAdds": 0,
                          "submitted": False, "numericalInputProfile": EXACT_F32_INPUT_PROFILE}}
    return run_semantic_gemm(bridge, prepare_semantic_gemm(m, n, k), certificate, a, b)


def run_prepared_semantic_attention_resident(prepared: PreparedSemanticAttention, inputs: Any) -> None:
    """Closed like the GEMM's resident seam: finiteness of resident buffers
    cannot be proved at this boundary."""
    _require_prepared(prepared, PreparedSemanticAttention, "BG-WEBGPU-ATTENTION-INVALID-BINDING")
    _fail("BG-WEBGPU-ATTENTION-NUMERICAL-PROOF", "$.inputs",
          "resident attention requires trusted input provenance; host-side validation cannot prove current "
          "device buffer contents")


def run_semantic_attention(bridge: Any, prepared: PreparedSemanticAttention, query: Any, key: Any, value: Any, *,
                           timeout_ms: Optional[int] = None, cancel: Any = None) -> Dict[str, Any]:
    """{"destination": f32 bytes [batch, heads, q_len, head_dim], "trace"}:
    softmax(q k^T * scale [causal]) v in f32 on a prepared specialization
    (runSemanticAttentionWebGpu, semantic_attention.ts:420-520).  Inputs must
    be finite, and so must the result."""
    _require_prepared(prepared, PreparedSemanticAttention, "BG-WEBGPU-ATTENTION-INVALID-BINDING")
    dl = _Deadline(timeout_ms, cancel, "ATTENTION")
    batch, heads, q_len, k_len, head_dim = (prepared.batch, prepared.heads, prepared.q_len, prepared.k_len,
                                            prepared.head_dim)

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
    dl.check()
    hs = [bridge.upload(t, t.shape, "float32") for t in (q, k, v)]
    try:
        dl.check()
        ho, launches = _run_logged(bridge, lambda: bridge.attention_ex(
            hs[0], hs[1], hs[2], batch=batch, heads=heads, sq=q_len, sk=k_len, d=head_dim, scale=prepared.scale,
            causal=prepared.causal, in_dtype="float32", out_dtype="float32"))
        try:
            check_launches(prepared.plan, launches, "BG-WEBGPU-ATTENTION-VALIDATION")
            check_layout(prepared.layout, {"query": bridge.handle_info(hs[0]), "key": bridge.handle_info(hs[1]),
                                           "value": bridge.handle_info(hs[2]), "output": bridge.handle_info(ho)},
                         "BG-WEBGPU-ATTENTION-VALIDATION")
            out = bridge.to_numpy(ho)
        finally:
            bridge.release(ho)
    finally:
        for h in hs:
            bridge.release(h)
    dl.check()
    if not np.isfinite(out).all():
        raise SemanticAttentionError("BG-WEBGPU-ATTENTION-NUMERICAL-PROOF", "$.output",
                                     "scaled scores or the result left the finite f32 domain")
    trace = {
        "operationId": f"hip-attention-{next(_OPERATION_IDS)}",
        "backendProfile": ATTENTION_PROFILE,
        "backendVersion": BACKEND_VERSION,
        "executionTier": "mi355x-hip-mfma-f32-attention",
        "mask": "causal" if prepared.causal else "none",
        "scaleBits": f"{np.float32(prepared.scale).view(np.uint32):08x}",
        "batch": batch, "heads": heads, "queryLength": q_len, "keyLength": k_len, "headDim": head_dim,
        "logicalBytesRead": 4 * (q.size + k.size + v.size),
        "logicalBytesWritten": 4 * out.size,
        "submitted": True,
        "device": _device_facts(bridge),
        "launchesMatchedPreparation": True,
    }
    trace.update(_trace_hashes(prepared, None))
    return {"destination": out.astype(np.float32).tobytes(), "trace": trace}


def run_semantic_attention_f32(bridge: Any, query: Any, key: Any, value: Any, *, batch: int, heads: int,
                               q_len: int, k_len: int, head_dim: int, scale: Optional[float] = None,
                               causal: bool = False) -> Dict[str, Any]:
    """One-shot form: prepare for the problem, then run."""
    prepared = prepare_semantic_attention(batch, heads, q_len, k_len, head_dim, scale=scale, causal=causal)
    return run_semantic_attention(bridge, prepared, query, key, value)


__all__ = ["certify_exact_f32_gemm_inputs", "prepare_semantic_gemm", "run_semantic_gemm",
           "run_prepared_semantic_gemm_resident", "run_semantic_gemm_exact_f32", "prepare_semantic_attention",
           "run_semantic_attention", "run_prepared_semantic_attention_resident", "run_semantic_attention_f32",
           "PreparedSemanticGemm", "PreparedSemanticAttention", "SemanticGemmError", "SemanticAttentionError",
           "EXACT_F32_INPUT_PROFILE", "EXACT_F32_INTEGER_LIMIT", "canonical_hash", "layout_artifact",
           "check_layout", "check_launches", "parse_kernel_symbol", "launch_plan", "gemm_tile_order"]
