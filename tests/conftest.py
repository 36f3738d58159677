"""Shared pytest setup.

* ``gpu`` marks tests that need an MI355X; everything else runs on the CPU.
* The repository root (for ``oracle``) and ``tilemix-cuda_amd`` (for the
  ``tilemix`` binding package) are put on sys.path.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for path in (ROOT, ROOT / "tilemix-cuda_amd", ROOT / "tests"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle

    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def tm():
    """The HIP binding; fails loudly (no fallback) when the library is missing."""
    import tilemix

    tilemix.library()
    return tilemix


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    torch.cuda.init()
    return torch.device("cuda:0")
