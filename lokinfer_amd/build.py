"""Builds liblokinfer_hip.so (gfx950) in-tree from lokinfer_amd/csrc with hipcc.

Usage: python -m lokinfer_amd.build [-j N]. Objects go to _build/ (git-ignored); the shared library lands
next to this file so that it travels with the source tree.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
LIB = PKG / "liblokinfer_hip.so"
ARCH = "gfx950"


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build the gfx950 backend)")


def common_flags() -> list[str]:
    return [
        "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
        # Packed-FP32 VALU forms are kept out of the generated code (compiler-chosen v_pk_* f32 ops).
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", str(ROOT / "include"), "-I", str(CSRC),
        "-Wno-unused-command-line-argument",
    ]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.parent.name + "_" + src.name + ".o")
    cmd = [hipcc(), *common_flags(), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [hipcc(), *common_flags(), "-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")) + list((CSRC / "rt").glob("*.cpp")))
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    build(a.j, verbose=True)
