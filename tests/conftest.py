"""Shared pytest setup.

* Puts the repository root (for `oracle`) and rocm-kernel-select_amd/ (for the
  `amd_tuned_torch` package) on sys.path.
* Registers the `gpu` marker: tests that need an MI355X.  `-m "not gpu"` runs everywhere.
* Disables the selector's on-disk winner cache so test runs never write into the package.
"""
from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "rocm-kernel-select_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

os.environ.setdefault("AMD_TUNED_TORCH_KERNEL_SELECT_CACHE", "0")

import pytest  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)
