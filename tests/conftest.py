"""Shared pytest setup: import paths, the ``gpu`` marker, GPU fixtures."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "kernel-rush-kawk_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box with -m gpu)")


@pytest.fixture(scope="session")
def device():
    """The GPU.  A test that asks for it is only ever selected with ``-m gpu``,
    so a missing GPU is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    return torch.device("cuda:0")
