"""Build libssa_hip.so (the HIP kernels and their C ABI) for gfx950, in the package directory.

Both sources are compiled with ``-ffp-contract=off``: the selection and insertion decisions
(select.h, shared by both files) must be reproducible bit for bit, and the attention loops
spell out their fused multiply-adds. Both are linked into one shared library next to this
file, which ``ssa_amd._lib`` loads.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
INCLUDE = PKG.parent.parent / "include"
LIB = PKG / "libssa_hip.so"
ARCH = os.environ.get("SSA_OFFLOAD_ARCH", "gfx950")

COMMON = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
          # packed fp32 instructions are kept out of every kernel
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-fhip-fp32-correctly-rounded-divide-sqrt", f"-I{INCLUDE}"]
SOURCES = {"attention.hip": ["-ffp-contract=off"], "index.hip": ["-ffp-contract=off"]}


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if c and (os.path.isabs(c) and os.path.exists(c) or not os.path.isabs(c)):
            return c
    raise RuntimeError("hipcc not found")


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        msg = "\n".join(line for line in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in line)
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{msg}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link ``libssa_hip.so``; returns its path."""
    hipcc = _hipcc()
    objdir = PKG / "_obj"
    objdir.mkdir(exist_ok=True)
    objs = []
    for src, extra in SOURCES.items():
        obj = objdir / (src.replace(".hip", ".o"))
        cmd = [hipcc, *COMMON, *extra, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, "-shared", f"--offload-arch={ARCH}", *objs, "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
