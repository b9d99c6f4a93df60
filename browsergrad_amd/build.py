"""Build libbghip.so (HIP, gfx950) and the Node addon in-tree.

Usage: python -m browsergrad_amd.build [--jobs N] [--no-node]

Every HIP/C++ source under browsergrad_amd/csrc is compiled with hipcc for
gfx950 into _build/ and linked into browsergrad_amd/libbghip.so.  The N-API
addon (browsergrad_amd/node/bghip.node) links against that library with an
$ORIGIN rpath so both travel together.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
LIB = PKG / "libbghip.so"
NODE_DIR = PKG / "node"
NODE_ADDON = NODE_DIR / "bghip.node"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("BG_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: elementwise chains must round per op like NumPy.
# -packed-fp32-ops disabled: packed FP32 forms are avoided on these boxes.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-Wno-unused-result",
]


# Per-source additions to HIP_FLAGS (none at present).
FILE_FLAGS: dict[str, list[str]] = {}


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line  # host pass does not know the feature
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def compile_sources(jobs: int = 8) -> list[Path]:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    objs = []

    def one(src: Path) -> Path:
        obj = BUILD / (src.name + ".o")
        cmd = [HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
        if src.suffix == ".cpp":
            cmd[1:1] = ["-x", "hip"]
        _run(cmd)
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(one, sources))
    return objs


def link_library(objs: list[Path]) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs),
          "-o", str(tmp), "-Wl,-soname,libbghip.so", "-lhiprtc"])
    os.replace(tmp, LIB)
    return LIB


def build_node_addon() -> Path | None:
    inc = Path("/usr/include/node")
    src = NODE_DIR / "bghip_napi.cpp"
    if not (inc / "node_api.h").exists() or not src.exists():
        return None
    cxx = shutil.which("g++") or "g++"
    tmp = NODE_ADDON.with_suffix(".node.tmp")
    _run([cxx, "-O2", "-std=c++17", "-shared", "-fPIC", f"-I{inc}", f"-I{ROOT / 'include'}",
          str(src), "-o", str(tmp), f"-L{PKG}", "-lbghip",
          "-Wl,-rpath,$ORIGIN/..", "-Wl,--allow-shlib-undefined"])
    os.replace(tmp, NODE_ADDON)
    return NODE_ADDON


def build(jobs: int = 8, node: bool = True) -> None:
    objs = compile_sources(jobs)
    link_library(objs)
    if node:
        build_node_addon()


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--no-node", action="store_true")
    a = ap.parse_args()
    build(a.jobs, node=not a.no_node)
    print(f"built {LIB}")


if __name__ == "__main__":
    main()
