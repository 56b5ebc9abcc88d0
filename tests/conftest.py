"""Shared pytest setup: import paths, the ``gpu`` marker, and small input factories.

Tests marked ``gpu`` need an AMD GPU (run on the MI355X box with ``-m gpu``); everything else
runs on the CPU (``-m "not gpu"``).
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "sparse-kv-reads_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (HIP) and the built libssa_hip.so")


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    import torch
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
