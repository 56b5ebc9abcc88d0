"""Build libssa_hip.so (the HIP kernels and their C ABI) for gfx950, in the package directory.

Every source is compiled with ``-ffp-contract=off``: the selection and insertion decisions
(select.h, shared by the decode and index kernels) must be reproducible bit for bit, and the
attention loops spell out their fused multiply-adds. The sources compile in parallel and are
linked into one shared library next to this file, which ``ssa_amd._lib`` loads.
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
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
SOURCES = {name: ["-ffp-contract=off"] for name in
           ("decode_bf16.hip", "decode_f16.hip", "decode_f32.hip", "attention.hip", "index.hip", "model.hip")}


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if c and (os.path.isabs(c) and os.path.exists(c) or not os.path.isabs(c)):
            return c
    raise RuntimeError("hipcc not found")


def _run(cmd: list[str]) -> str:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        msg = "\n".join(line for line in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in line)
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{msg}")
    return r.stderr


# The step kernel's resident workgroups per compute unit. With insert-ahead its grid is one
# workgroup per compute unit plus a stager per head, so a kernel that fits only one wave per SIMD
# (registers or LDS) leaves the stagers waiting for a whole workgroup to finish, which lengthens
# every step by that workgroup's runtime. The build refuses such a kernel for the caches, head
# sizes and query groups of the decode configurations it serves (2-byte K/V, d <= 128, up to 4
# query heads per KV head); fp32 caches hold twice the row registers and are a parity path.
_KERNEL = re.compile(r"Function Name: _ZN3ssa13decode_kernelI(\w+?)Li(\d+)ELi(\d+)ELb(\d)ELb(\d)ELb(\d)ELi(\d+)E")
_OCC = re.compile(r"Occupancy \[waves/SIMD\]: (\d+)")


def decode_occupancy(remarks: str) -> dict:
    """{(dtype, d, GMAX, dense, select, ahead, slot capacity): waves per SIMD} from the compiler's
    kernel-resource-usage remarks of a decode translation unit."""
    out = {}
    for block in remarks.split("Function Name: ")[1:]:
        m = _KERNEL.match("Function Name: " + block)
        o = _OCC.search(block)
        if m and o:
            out[(m.group(1), int(m.group(2)), int(m.group(3)), *(int(m.group(i)) for i in (4, 5, 6, 7)))] = int(o.group(1))
    return out


def _check_occupancy(remarks: str, src: str) -> None:
    occ = decode_occupancy(remarks)
    if not occ:
        raise RuntimeError(f"{src}: no resource-usage remarks for decode_kernel")
    low = {k: v for k, v in occ.items() if k[0] != "f" and k[1] <= 128 and k[2] <= 4 and v < 2}
    if low:
        raise RuntimeError(f"{src}: decode kernels below 2 waves per SIMD: {sorted(low)}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link ``libssa_hip.so``; returns its path."""
    hipcc = _hipcc()
    objdir = PKG / "_obj"
    objdir.mkdir(exist_ok=True)
    cmds, objs = [], []
    for src, extra in SOURCES.items():
        obj = objdir / (src.replace(".hip", ".o"))
        remarks = ["-Rpass-analysis=kernel-resource-usage"] if src.startswith("decode_") else []
        cmds.append([hipcc, *COMMON, *extra, *remarks, "-c", str(CSRC / src), "-o", str(obj)])
        objs.append(str(obj))
        if verbose:
            print(" ".join(cmds[-1]), flush=True)
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as pool:
        logs = list(pool.map(_run, cmds))
    for src, log in zip(SOURCES, logs):
        if src.startswith("decode_"):
            _check_occupancy(log, src)
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, "-shared", f"--offload-arch={ARCH}", *objs, "-o", str(tmp)])
    os.replace(tmp, LIB)
    _write_build_info(hipcc)
    return LIB


def _write_build_info(hipcc: str) -> None:
    """Record the source revision the library was built from (read by ``ssa_amd.stamp`` where
    the tree has no git metadata)."""
    import json
    import time
    root = str(PKG.parents[1])
    try:
        rev = {"sha": subprocess.check_output(["git", "-C", root, "rev-parse", "HEAD"], text=True,
                                              stderr=subprocess.DEVNULL).strip(),
               "dirty": bool(subprocess.check_output(["git", "-C", root, "status", "--porcelain",
                                                      "--untracked-files=no"], text=True,
                                                     stderr=subprocess.DEVNULL).strip())}
    except (OSError, subprocess.CalledProcessError):
        rev = {"sha": "nogit"}
    try:
        ver = subprocess.run([hipcc, "--version"], capture_output=True, text=True).stdout.splitlines()[0]
    except (OSError, IndexError):
        ver = hipcc
    (PKG / "BUILD_INFO.json").write_text(json.dumps({"git_sha": rev.get("sha"), "dirty": rev.get("dirty"), "arch": ARCH,
                                      "built_at": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
                                      "hipcc": ver}) + "\n")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
