"""Build ``libg4rollout.so`` (gfx950) from ``csrc/`` with hipcc, in-tree.

Each source compiles to an object under ``<repo>/_build/`` (git-ignored), then one shared library
is linked next to this file. All device code is built with packed-FP32 instruction selection
disabled (``-packed-fp32-ops``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "libg4rollout.so"
BUILD_DIR = PKG_DIR.parent / "_build"
ARCH = "gfx950"

CXXFLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def build(verbose: bool = False) -> Path:
    """Compile every ``csrc/*.hip`` / ``csrc/*.cpp`` and link ``libg4rollout.so``; returns its path."""

    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    procs = []
    objects = []
    for src in sources:
        obj = BUILD_DIR / (src.name + ".o")
        objects.append(obj)
        cmd = [hipcc, *CXXFLAGS, "-c", str(src), "-o", str(obj)]
        procs.append((src, cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for src, cmd, p in procs:
        out, _ = p.communicate()
        out = "\n".join(line for line in out.splitlines() if "is not a recognized feature for this target" not in line)
        if p.returncode != 0:
            failed.append(f"{src.name}:\n{' '.join(cmd)}\n{out}")
        elif verbose and out.strip():
            print(out, file=sys.stderr)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n\n".join(failed))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objects), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
