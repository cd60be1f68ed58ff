"""Shared pytest configuration.

GPU tests are marked ``gpu`` and need an MI355X (gfx950) with the in-tree
libpisa_hip.so; everything else runs on the CPU.
"""
from __future__ import annotations

import pathlib
import sys

import pytest

REPO_ROOT = pathlib.Path(__file__).resolve().parents[1]
PACKAGE_DIR = REPO_ROOT / "comfyui-rdna35-attention_amd"
for path in (REPO_ROOT, PACKAGE_DIR):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def _gpu_ready() -> bool:
    try:
        import torch

        return torch.cuda.is_available() and torch.version.hip is not None
    except Exception:  # pragma: no cover - torch import problems
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_ready():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
