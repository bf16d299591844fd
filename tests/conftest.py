import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fast-familywise-loss_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (ROOT, ORACLE, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs the HIP kernels on an MI355X (gfx950)")


@pytest.fixture(scope="session")
def dev():
    import torch
    # GPU tests fail (never skip) without a GPU, so a missing device cannot pass silently
    assert torch.cuda.is_available(), "GPU tests need a ROCm device (run them with -m gpu on an MI355X)"
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def ext(dev):
    import fwloss
    return fwloss
