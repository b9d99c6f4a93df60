"""bg_matmul_noalloc, the GEMM entry point that allocates nothing, against
bg_matmul_ex on the GPU.

Both run the same kernels; only the scratch differs (the context's growable
slots vs the fixed per-GPU array), so the outputs must be bit-identical.  Each
case uses scratch (split-K partials, the re-laid-out B of x @ w, the f32
product before a separate GELU pass) and runs twice in a row on the fixed
array, the second time with a smaller problem.  Operands and results of the
no-allocation calls are caller-owned device memory (torch tensors); the
library's handle table and pool must not change across those calls.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from browsergrad_amd import _native as N

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

_TORCH = {"float32": torch.float32, "float16": torch.float16}


def _desc(m, n, k, trans_b, in_dtype, out_dtype, round_out, act, a=0, b=0, bias=0):
    d = N.MatmulDesc()
    d.a, d.b, d.bias = a, b, bias
    d.batch, d.m, d.n, d.k = 1, m, n, k
    d.lda = k
    d.ldb = k if trans_b else n
    d.ldc = n
    d.stride_a, d.stride_b, d.stride_c = m * k, n * k, m * n
    d.trans_b = 1 if trans_b else 0
    d.in_dtype = N.DTYPE_CODES[in_dtype]
    d.out_dtype = N.DTYPE_CODES[out_dtype]
    d.round_f16 = 1 if round_out else 0
    d.act = act
    return d


def _inputs(rng, m, n, k, trans_b, in_dtype):
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (n, k) if trans_b else (k, n)).astype(np.float32)
    bias = rng.uniform(-0.5, 0.5, (n,)).astype(np.float32)
    dt = np.float32 if in_dtype == "float32" else np.float16
    return a.astype(dt), b.astype(dt), bias


def _with_handles(bridge, a, b, bias, m, n, k, trans_b, in_dtype, out_dtype, round_out, act):
    ha, hb = bridge.upload(a, a.shape, in_dtype), bridge.upload(b, b.shape, in_dtype)
    hbias = bridge.upload(bias, bias.shape, "float32")
    h = bridge.matmul_ex(ha, hb, m=m, n=n, k=k, trans_b=trans_b, in_dtype=in_dtype, out_dtype=out_dtype,
                         bias=hbias, round_out=round_out, act=act)
    y = bridge.to_numpy(h)
    for x in (h, ha, hb, hbias):
        bridge.release(x)
    return y


def _snapshot(bridge):
    s = bridge.resourceSnapshot()
    return (bridge.aliveHandleCount(), s["currentOwnedGpuBytes"], torch.cuda.memory_allocated())


def _no_alloc(bridge, a, b, bias, m, n, k, trans_b, in_dtype, out_dtype, round_out, act):
    ta = torch.from_numpy(a).cuda()
    tb = torch.from_numpy(b).cuda()
    tbias = torch.from_numpy(bias).cuda()
    tc = torch.full((m, n), float("nan"), dtype=_TORCH[out_dtype], device="cuda")
    torch.cuda.synchronize()
    before = _snapshot(bridge)
    d = _desc(m, n, k, trans_b, in_dtype, out_dtype, round_out, act)
    rc = bridge._lib.bg_matmul_noalloc(bridge._ctx, C.byref(d), ta.data_ptr(), tb.data_ptr(), tbias.data_ptr(),
                                       tc.data_ptr())
    assert rc == N.BG_OK, bridge._lib.bg_last_error(bridge._ctx).decode()
    bridge.synchronize()
    assert _snapshot(bridge) == before
    return tc.cpu().numpy()


# (label, m, n, k, trans_b, in, out, round_out, act, smaller (m, n, k))
CASES = [
    ("f32 long-K split-K partials", 64, 128, 784, True, "float32", "float32", False, N.ACT_RELU, (48, 100, 640)),
    ("f16 x @ w, B re-laid out", 512, 384, 768, False, "float16", "float16", True, N.ACT_NONE, (200, 96, 320)),
    ("f16 GELU after the product", 100, 96, 100, True, "float16", "float16", True, N.ACT_GELU_TANH, (70, 40, 36)),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_matches_matmul_ex_twice(bridge, case):
    _, m, n, k, trans_b, in_dt, out_dt, rnd, act, smaller = case
    rng = np.random.default_rng(42)
    for (mm, nn, kk) in ((m, n, k), smaller):
        a, b, bias = _inputs(rng, mm, nn, kk, trans_b, in_dt)
        ref = _with_handles(bridge, a, b, bias, mm, nn, kk, trans_b, in_dt, out_dt, rnd, act)
        got = _no_alloc(bridge, a, b, bias, mm, nn, kk, trans_b, in_dt, out_dt, rnd, act)
        assert got.dtype == ref.dtype and got.shape == ref.shape
        assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), (mm, nn, kk)


def test_noalloc_refuses_scratch_beyond_its_limit(bridge):
    """x @ w at 4096 x 4096 x 4096 in f16 needs a 32 MiB re-laid-out B: refused
    with a clear message before anything runs (C keeps its contents)."""
    m = n = k = 4096
    ta = torch.zeros((m, k), dtype=torch.float16, device="cuda")
    tb = torch.zeros((k, n), dtype=torch.float16, device="cuda")
    tc = torch.full((m, n), 7.0, dtype=torch.float16, device="cuda")
    torch.cuda.synchronize()
    d = _desc(m, n, k, False, "float16", "float16", False, N.ACT_NONE)
    rc = bridge._lib.bg_matmul_noalloc(bridge._ctx, C.byref(d), ta.data_ptr(), tb.data_ptr(), None, tc.data_ptr())
    assert rc == N.BG_E_UNSUPPORTED
    msg = bridge._lib.bg_last_error(bridge._ctx).decode()
    assert "scratch" in msg and str(16 << 20) in msg, msg
    bridge.synchronize()
    assert bool((tc == 7.0).all())


def test_noalloc_refuses_handles_in_the_descriptor(bridge):
    d = _desc(8, 8, 8, True, "float32", "float32", False, N.ACT_NONE, a=1)
    t = torch.zeros(64, dtype=torch.float32, device="cuda")
    rc = bridge._lib.bg_matmul_noalloc(bridge._ctx, C.byref(d), t.data_ptr(), t.data_ptr(), None, t.data_ptr())
    assert rc == N.BG_E_INVALID
    assert "must be 0" in bridge._lib.bg_last_error(bridge._ctx).decode()
