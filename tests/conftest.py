"""Test configuration: import paths, the ``gpu`` marker, shared helpers."""

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_PARENT = REPO / "specdiff-ae_amd"
for p in (str(REPO), str(PKG_PARENT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device); run with -m gpu")


@pytest.fixture(scope="session")
def dsv_lib():
    """libdsv.so, built in-tree on first use when it is missing."""
    from diffspec_mi355x import _build, _ext

    if not _ext.lib_path().exists():
        _build.build()
    return _ext.load()


@pytest.fixture(scope="session")
def gpu(dsv_lib):
    """The ROCm device the GPU tests run on; fails (never skips) without one."""
    import torch

    assert torch.cuda.is_available(), "GPU tests need a ROCm device (run them on the MI355X box)"
    return torch.device("cuda:0")
