import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "freetoken-rs_amd"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (run on the MI355X box)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gemv():
    """The HIP library on cuda:0 (GPU tests only)."""
    import torch
    import ft_hip
    assert torch.cuda.is_available(), "GPU test run without a GPU"
    g = ft_hip.Q4Gemv(0)
    yield g
    g.close()
