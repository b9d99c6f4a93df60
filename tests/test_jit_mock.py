"""The HIP walker on the NumPy MockBridge (CPU): parity, residency and
refusals of the front end without a GPU.

The GPU tier runs the same walker against libbghip (tests/test_gpu_jit.py);
here the bridge is tests/mock_bridge.py, whose arithmetic is the oracle's, so
these tests pin the walker's own logic: cast insertion, the HIP rewrites
(GEMM epilogues with residuals, fused attention with strided QKV views,
elementwise + reduce programs), handle bookkeeping and release, and the
GpuBufferTable residency counts of the reference's MockBridge tests
(webgpu_realizer.test.ts:1026-1112).
"""
from __future__ import annotations

import numpy as np
import pytest

from browsergrad_amd.errors import JitNotImplementedError, KernelError
from browsergrad_amd.jit import configs
from browsergrad_amd.jit.buffers import GpuBufferTable
from browsergrad_amd.jit.ir import UOp
from browsergrad_amd.jit.realize import realize_hip
from browsergrad_amd.jit.tensor import Session
from mock_bridge import MockHipBridge
from oracle import graph as G
from oracle import ops as O

CASES = [("c1", 1.0, {}, 1e-4), ("c2", 1 / 16, {}, 1e-4), ("c3", 1 / 16, {"amp": False}, 1e-4),
         ("c3", 1 / 16, {}, 2e-2), ("c4", 1 / 16, {}, 2e-2), ("c5", 1 / 8, {}, 2e-2)]


def _check(out, ref, tol):
    assert out.shape == ref.shape and out.dtype == ref.dtype, (out.shape, out.dtype, ref.shape, ref.dtype)
    rep = O.report(out.astype(np.float32), ref.astype(np.float32), tol)
    assert rep["pass"], rep


@pytest.mark.parametrize("rewrites", [True, False], ids=["hip_rewrites", "reference_ops"])
@pytest.mark.parametrize("name,scale,kw,tol", CASES, ids=[f"{c[0]}{'_fp32' if c[2] else ''}" for c in CASES])
def test_walker_parity_on_mock(name, scale, kw, tol, rewrites):
    br = MockHipBridge()
    table = GpuBufferTable(br)
    s, y = configs.BUILDERS[name](scale=scale, **kw)
    ref = G.evaluate(y.uop, s.buffers)
    out = realize_hip(y.uop, s.buffers, table, hip_rewrites=rewrites)
    _check(out, ref, tol)
    # every intermediate was released: only the table's seed buffers (and their cached casts) remain
    assert br.aliveHandleCount() == table.stats()["handles_alive"]
    table.release_all()
    assert br.aliveHandleCount() == 0


def test_walker_c4_bf16_on_mock():
    br = MockHipBridge()
    s, y = configs.c4(scale=1 / 16, dtype="bfloat16")
    ref = G.evaluate(y.uop, s.buffers)
    out = realize_hip(y.uop, s.buffers, GpuBufferTable(br))
    assert out.dtype == np.uint16
    _check(O.bf16_bits_to_f32(out), ref.astype(np.float32), 2e-2)


def test_single_matmul_residency():
    br = MockHipBridge()
    rng = np.random.RandomState(0)
    a_np = rng.uniform(-1, 1, size=(3, 4)).astype(np.float32)
    b_np = rng.uniform(-1, 1, size=(4, 5)).astype(np.float32)
    s = Session()
    a, b = s.from_numpy(a_np), s.from_numpy(b_np)
    gbt = GpuBufferTable(br)
    y = realize_hip((a @ b).uop, s.buffers, gbt)
    assert np.max(np.abs(y - a_np @ b_np)) < 1e-6
    c = br.counters
    assert (c["upload"], c["matmul"], c["materialize"]) == (2, 1, 1)


def test_chained_matmul_residency_and_no_reupload():
    br = MockHipBridge()
    rng = np.random.RandomState(1)
    xs = [rng.uniform(-1, 1, size=sh).astype(np.float32) for sh in ((2, 3), (3, 4), (4, 5))]
    s = Session()
    x, w1, w2 = (s.from_numpy(t) for t in xs)
    gbt = GpuBufferTable(br)
    y = realize_hip(((x @ w1) @ w2).uop, s.buffers, gbt)
    c = br.counters
    assert np.max(np.abs(y - (xs[0] @ xs[1]) @ xs[2])) < 1e-5
    assert (c["upload"], c["matmul"], c["materialize"], c["release"]) == (3, 2, 1, 2)
    assert gbt.stats()["handles_alive"] == 3
    realize_hip(((x @ w1) @ w2).uop, s.buffers, gbt)
    assert br.counters["upload"] == 3  # seeds stay resident
    gbt.release_all()
    assert br.aliveHandleCount() == 0


def test_handle_rules():
    br = MockHipBridge()
    h1 = br.upload(np.ones(3, np.float32), (3,), "float32")
    h2 = br.upload(np.ones(3, np.float32), (3,), "float32")
    assert (h1, h2) == (1, 2)
    br.release(h1)
    br.release(h1)  # idempotent
    h3 = br.upload(np.ones(3, np.float32), (3,), "float32")
    assert h3 == 3  # ids are never reused
    with pytest.raises(KernelError, match="materialize: unknown or released handle 1"):
        br.materialize(h1, (3,), "float32")


def test_walker_refusals():
    br = MockHipBridge()
    s = Session()
    x = s.from_numpy(np.ones((2, 2), np.float32))
    custom = UOp("CUSTOM", (x.uop,), (2, 2), "float32", {"op": "wgsl_kernel"})
    with pytest.raises(JitNotImplementedError, match="CUSTOM"):
        realize_hip(custom, s.buffers, GpuBufferTable(br))
    # nothing leaked by the refused walk
    assert br.aliveHandleCount() == 1  # the uploaded seed, owned by the table


def test_residual_epilogue_rides_on_the_gemm():
    """x + linear(h) is one matmul_ex call with the residual, bit-identical to
    the unfused ADD on the mock (same f32 additions in the same order)."""
    br = MockHipBridge()
    s, y = configs.c5(scale=1 / 8)
    fused = realize_hip(y.uop, s.buffers, GpuBufferTable(br))
    plain = realize_hip(y.uop, s.buffers, GpuBufferTable(MockHipBridge()), hip_rewrites=False)
    _check(fused, plain, 2e-2)


def test_gpu_buffer_table_bookkeeping():
    """The table's own contract (_gpu_buffer_table.py:35-131): idempotent
    upload, refused second register, detach hands the handle over without a
    release, replace/release give handles back, stats stay consistent."""
    from browsergrad_amd.jit.buffers import BufferTableError
    br = MockHipBridge()
    t = GpuBufferTable(br)
    a = np.arange(6, dtype=np.float32)
    h1 = t.upload("a", a, (6,), "float32")
    assert t.upload("a", a, (6,), "float32") == h1  # no second upload
    assert t.stats() == {"handles_alive": 1, "uploaded_bytes": 24, "registered_ids": 1}
    with pytest.raises(BufferTableError, match="resident already"):
        t.register("a", h1)
    hb = br.upload(a, (6,), "float32")
    t.register("b", hb)
    assert t.has("b") and t.get("b") == hb and t.get("zzz") is None
    assert t.detach("b") == hb and not t.has("b")
    assert br.aliveHandleCount() == 2  # detach does not release
    with pytest.raises(BufferTableError, match="nothing to detach"):
        t.detach("b")
    br.release(hb)
    hc = br.upload(a, (6,), "float32")
    t.replace("a", hc)  # h1 is released
    assert br.aliveHandleCount() == 1 and t.get("a") == hc
    t.release("missing")  # ignored
    t.upload("d", a.tobytes(), (6,), "float32")
    assert t.stats() == {"handles_alive": 2, "uploaded_bytes": 48, "registered_ids": 2}
    t.release_all()
    assert br.aliveHandleCount() == 0 and t.stats()["handles_alive"] == 0
    with pytest.raises(BufferTableError, match="needs a bridge"):
        GpuBufferTable(None)
