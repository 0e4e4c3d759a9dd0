"""Test configuration: import paths and the ``gpu`` marker.

The product package lives in ``twilight-cpu-gpu-offloading_amd/`` and is
imported as ``headinfer`` (the reference's package name), exactly as the
reference's scripts import it after putting ``source/headinfer`` on sys.path.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "twilight-cpu-gpu-offloading_amd"
for p in (str(ROOT), str(PKG_DIR)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    return torch.device("cuda", 0)
