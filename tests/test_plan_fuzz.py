"""Sanitizer fuzz of the tensor-plan reader, validator and fuser (CPU).

tests/fuzz/Makefile builds browsergrad_amd/csrc/plan.cpp and plan_fuse.cpp
for the host only with AddressSanitizer and UndefinedBehaviorSanitizer, with
the harness tests/fuzz/plan_fuzz.cpp.  The seeds are the HIP route's plans
of the five BASELINE configs (with the semantic side table where one
travels); each is checked unmutated (it must be accepted) and under seeded
mutations (byte flips, truncations, splices, out-of-range numbers, token
swaps), which must end as refusals, never as a sanitizer report.
"""
from __future__ import annotations

import json
import os
import shutil
import subprocess
from pathlib import Path

import pytest

from browsergrad_amd.jit import configs
from browsergrad_amd.jit.realize import _plan_submission

FUZZ = Path(__file__).resolve().parent / "fuzz"
pytestmark = pytest.mark.skipif(not os.path.exists("/opt/rocm/bin/hipcc") or shutil.which("make") is None,
                                reason="hipcc / make not available")


def test_plan_reader_under_asan_ubsan(tmp_path):
    out = tmp_path / "build"
    r = subprocess.run(["make", "-s", "-C", str(FUZZ), f"OUT={out}"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    seeds = []
    for name, kw, scale in (("c1", {}, 1.0), ("c2", {}, 1 / 16), ("c3", {}, 1 / 16), ("c4", {}, 1 / 16),
                            ("c5", {}, 1 / 16)):
        s, y = configs.BUILDERS[name](scale=scale, **kw)
        plan, _, req_json = _plan_submission(y.uop, s.buffers)
        p = tmp_path / f"{name}.json"
        p.write_text(json.dumps(plan, separators=(",", ":")))
        if req_json:
            Path(str(p) + ".req").write_text(req_json)
        seeds.append(str(p))
    env = dict(os.environ, UBSAN_OPTIONS="print_stacktrace=1", ASAN_OPTIONS="detect_leaks=1")
    r = subprocess.run([str(out / "plan_fuzz"), "3000", *seeds], capture_output=True, text=True, timeout=600,
                       env=env)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "no sanitizer report" in r.stdout
    accepted, refused = (int(w) for w in r.stdout.split()[1:4:2])
    assert accepted >= 5 and refused > 1000, r.stdout
