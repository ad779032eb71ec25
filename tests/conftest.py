"""Shared pytest setup.

* Puts the package directory (flash-attention-cuda_amd/) and the repo root
  (for the CPU oracle) on sys.path.
* Registers the ``gpu`` marker (pytest.ini of the reference:1-4); GPU tests
  are skipped when no HIP device is visible.
"""

import os
import sys

import pytest

REPO_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO_ROOT, "flash-attention-cuda_amd")
for p in (PKG_DIR, REPO_ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test requires a HIP (MI355X) device")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="HIP device required")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
