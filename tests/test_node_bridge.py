"""createHipRealizerBridge (the Node host of the bridge, browsergrad_amd/node).

CPU: the N-API addon loads, exports its functions, and refuses to open a
context without a HIP device (no CPU fallback).  GPU: tests/node/bridge_test.js
runs the reference's known answers through the Node bridge.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
ADDON = ROOT / "browsergrad_amd" / "node" / "bghip.node"
NODE = shutil.which("node")

needs_addon = pytest.mark.skipif(NODE is None or not ADDON.exists(),
                                 reason="node or the built addon (python -m browsergrad_amd.build) is missing")


def _node(script: str, timeout: int = 120) -> subprocess.CompletedProcess:
    return subprocess.run([NODE, "-e", script], cwd=ROOT, capture_output=True, text=True, timeout=timeout)


@needs_addon
def test_addon_loads_and_exports():
    r = _node("const m = require('./browsergrad_amd/node');"
              "const n = require('./browsergrad_amd/node/bghip.node');"
              "console.log(JSON.stringify({api: Object.keys(m), native: Object.keys(n).sort(), v: m.version()}));")
    assert r.returncode == 0, r.stderr
    out = r.stdout.strip()
    for name in ("createHipRealizerBridge", "KernelError", "ctxCreate", "upload", "materialize", "matmul",
                 "fusedElementwise", "cast", "flashAttention", "conv", "runTensorPlan", "aliveHandles",
                 "resourceSnapshot", "flushProfiles", "materializeAsync", "runTensorPlanAsync"):
        assert name in out
    assert "bghip" in out


@pytest.mark.gpu
@needs_addon
def test_node_bridge_on_gpu():
    r = subprocess.run([NODE, str(ROOT / "tests" / "node" / "bridge_test.js")], cwd=ROOT, capture_output=True,
                       text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "[node] ok" in r.stdout
