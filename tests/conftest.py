"""Shared pytest configuration: markers, import paths, seeding."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "pyramid-forcing_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity tests of the HIP kernels")
    config.addinivalue_line("markers", "slow: long-running case")


@pytest.fixture(autouse=True)
def _seed():
    import numpy as np
    np.random.seed(int(os.environ.get("PKV_TEST_SEED", "0")))
    try:
        import torch
        torch.manual_seed(int(os.environ.get("PKV_TEST_SEED", "0")))
    except ImportError:
        pass
    yield


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False
