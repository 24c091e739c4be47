"""pytest configuration: the ``gpu`` marker and import paths.

Tests marked ``gpu`` need a ROCm device and the built library; the rest run on
any CPU (oracle pinning, host logic, C-ABI loading and argument checks).
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and libwal2026_amd.so")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda", 0)
