"""The C ABI (include/bghip.h) on CPU: the library loads, exports every
declared entry point, and its host-only functions behave (no GPU calls).

The library is built by __graft_entry__.build() / python -m browsergrad_amd.build;
these tests skip with a message when it has not been built yet.
"""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

from browsergrad_amd import _native as N

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "bghip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bg_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not N.LIB_PATH.exists():
        pytest.skip(f"{N.LIB_PATH} not built (run python -m browsergrad_amd.build)")
    return N.load_library()


def test_header_declares_the_bridge_surface():
    names = declared_functions()
    # realizer.ts:77-280 methods, as C entry points
    for must in ("bg_upload", "bg_materialize", "bg_release", "bg_matmul", "bg_fused_elementwise", "bg_cast",
                 "bg_flash_attention", "bg_run_tensor_plan", "bg_alive_handles", "bg_resource_snapshot",
                 "bg_flush_profiles"):
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared in bghip.h but not exported: {missing}"


def test_ctypes_signatures_cover_the_header():
    # every declared function has a ctypes signature in browsergrad_amd/_native.py
    assert set(declared_functions()) <= set(N.SIGNATURES)


def test_host_only_functions(lib):
    assert lib.bg_version().decode().startswith("bghip")
    assert lib.bg_dtype_from_name(b"float32") == N.BG_F32
    assert lib.bg_dtype_from_name(b"float16") == N.BG_F16
    assert lib.bg_dtype_from_name(b"bfloat16") == N.BG_BF16
    assert lib.bg_dtype_from_name(b"complex64") == -1
    assert [lib.bg_dtype_size(t) for t in (N.BG_F32, N.BG_F16, N.BG_BF16, N.BG_BOOL)] == [4, 2, 2, 1]
    assert lib.bg_dtype_size(99) == -1
    # NULL arguments are refused before any HIP call
    assert lib.bg_ctx_create(0, 0, None) == N.BG_E_INVALID
    assert lib.bg_last_error(None).decode() == "HIP bridge: null context"
    assert lib.bg_ctx_destroy(None) == N.BG_OK


def test_struct_layouts_match_header():
    # field counts / sizes of the descriptors the bindings pass by pointer
    assert C.sizeof(N.FusedOp) == 16
    assert C.sizeof(N.MatmulDesc) == 3 * 8 + 12 * 8 + 6 * 4
    assert C.sizeof(N.PassProfile) == 48 + 8 + 8 + 8
    assert C.sizeof(N.OptimArgs) == 6 * 8
    assert C.sizeof(N.ConvDesc) == 4 * 4 + 4 * 8 + 7 * 3 * 8 + 3 * 8
    assert C.sizeof(N.LaunchPlanEntry) == 48 + 4 + 8 * 4 + 3 * 4 + 3 * 8
    assert C.sizeof(N.LaunchPlan) == 6 * 4 + 2 * 8 + 4 * C.sizeof(N.LaunchPlanEntry)


def test_fused_codegen_compiles_every_opcode(lib):
    """hipRTC-compiles generated fused kernels covering every opcode, input
    dtype, broadcast kind, vector width and reduction (no device needed)."""
    buf = C.create_string_buffer(4096)
    failures = lib.bg_fused_codegen_selftest(buf, 4096)
    assert failures == 0, buf.value.decode()


def test_fused_ex_descriptor_cache_passes_each_calls_handles():
    """HipRealizerBridge.fused_ex reuses one ctypes descriptor per program
    structure; every call must still pass its own input handles, and a change
    of structure (ops, shape, immediates, reduction) must get its own
    descriptor.  Checked on the CPU against a stand-in for the library that
    records what bg_fused_ex receives (no GPU call)."""
    import numpy as np  # noqa: F401

    from browsergrad_amd.bridge import HipRealizerBridge

    seen = []

    class RecordingLib:
        def bg_fused_ex(self, ctx, dptr, out):
            d = C.cast(dptr, C.POINTER(N.FusedDesc)).contents
            seen.append({
                "inputs": [int(d.inputs[i]) for i in range(d.n_inputs)],
                "ops": [(d.ops[i].code, d.ops[i].a, d.ops[i].b) for i in range(d.n_ops)],
                "shape": [int(d.shape[i]) for i in range(d.rank)],
                "imms": [float(d.imms[i]) for i in range(d.n_imms)],
                "reduce": int(d.reduce_op),
            })
            C.cast(out, C.POINTER(N.handle_t)).contents.value = 100 + len(seen)
            return N.BG_OK

    br = HipRealizerBridge.__new__(HipRealizerBridge)
    br._lib = RecordingLib()
    br._ctx = None
    br._fused_descs = {}
    ops = [("MUL", -1, -2, 0), ("ADD", 0, -3, 0)]
    assert br.fused_ex([1, 2, 3], ops, (4, 8), "float32") == 101
    assert br.fused_ex([7, 8, 9], ops, (4, 8), "float32") == 102
    assert br.fused_ex([7, 8, 9], ops, (4, 8), "float32", imms=[2.5], reduce=1) == 103
    assert br.fused_ex([4, 5], [("ADD", -1, -2, 0)], (16,), "float32") == 104
    assert [s["inputs"] for s in seen] == [[1, 2, 3], [7, 8, 9], [7, 8, 9], [4, 5]]
    assert seen[0]["ops"] == seen[1]["ops"] == [(N.OPS["MUL"], -1, -2), (N.OPS["ADD"], 0, -3)]
    assert seen[2]["imms"] == [2.5] and seen[2]["reduce"] == 1 and seen[1]["reduce"] == 0
    assert seen[3]["shape"] == [16] and seen[3]["ops"] == [(N.OPS["ADD"], -1, -2)]
    assert len(br._fused_descs) == 3
