"""Result-file provenance stamp (mirrors src/ssa/harness/stamp.py:35-45 of the reference).

Every result dict gets a header: the source revision, the GPU and the torch / ROCm versions.
The revision is ``git rev-parse HEAD`` when the tree is a git checkout; a copied tree (the GPU
machine receives the working tree without its ``.git``) falls back to the revision recorded by
``ssa_amd.build`` when it compiled ``libssa_hip.so`` (``BUILD_INFO.json`` beside the library),
so a number can always be traced to the sources of the library that produced it.
"""

from __future__ import annotations

import json
import platform
import subprocess
from pathlib import Path

import torch

BUILD_INFO = Path(__file__).resolve().parent / "BUILD_INFO.json"


def git_revision(root: Path | None = None) -> dict:
    """``{"sha": ..., "dirty": bool}`` of the checkout at ``root``, or ``{"sha": "nogit"}``."""
    root = root or Path(__file__).resolve().parents[2]
    try:
        sha = subprocess.check_output(["git", "-C", str(root), "rev-parse", "HEAD"], stderr=subprocess.DEVNULL,
                                      text=True).strip()
        dirty = bool(subprocess.check_output(["git", "-C", str(root), "status", "--porcelain", "--untracked-files=no"],
                                             stderr=subprocess.DEVNULL, text=True).strip())
        return {"sha": sha, "dirty": dirty}
    except Exception:
        return {"sha": "nogit"}


def build_info() -> dict:
    try:
        return json.loads(BUILD_INFO.read_text())
    except (OSError, ValueError):
        return {}


def _gpu_info() -> dict:
    if not torch.cuda.is_available():
        return {"name": None, "arch": None, "driver": None}
    p = torch.cuda.get_device_properties(0)
    return {"name": torch.cuda.get_device_name(0), "arch": getattr(p, "gcnArchName", None),
            "compute_units": p.multi_processor_count, "memory_GB": round(p.total_memory / 2 ** 30, 1),
            "driver": getattr(torch.version, "hip", None)}


def stamp(payload: dict) -> dict:
    """Return ``payload`` merged under a reproducibility header."""
    rev = git_revision()
    built = build_info()
    if rev.get("sha") == "nogit" and built.get("git_sha"):
        rev = {"sha": built["git_sha"], "dirty": built.get("dirty"), "from": "BUILD_INFO.json"}
    return {
        "git_sha": rev.get("sha"),
        "git_dirty": rev.get("dirty"),
        "library_built": {k: built.get(k) for k in ("git_sha", "dirty", "built_at", "hipcc") if k in built},
        "torch_version": torch.__version__,
        "hip_version": getattr(torch.version, "hip", None),
        "python_version": platform.python_version(),
        "platform": platform.platform(),
        "gpu": _gpu_info(),
        **payload,
    }
