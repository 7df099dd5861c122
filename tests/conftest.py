"""Shared pytest set-up.

* puts the repository root (for ``oracle``) and the package directory (for
  ``import w4a16``) on ``sys.path``, the way the reference's conftest puts
  ``src/`` there (reference: w4a16-kernel/tests/conftest.py:14-17);
* registers the ``gpu`` marker: tests that need an MI355X (HIP device) carry it,
  everything else runs on the CPU;
* seeds torch once per session (reference conftest.py:31-33).
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
PKG_DIR = os.path.join(ROOT, "w4a16-dequant-fused-matmul-kernel_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X / gfx950)")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()


@pytest.fixture(scope="session", autouse=True)
def _seed() -> None:
    import torch

    torch.manual_seed(0)


@pytest.fixture(scope="session")
def lib():
    """The built C-ABI library (ctypes handle).  Fails loudly if it is missing."""
    from w4a16 import _lib

    return _lib.load()
