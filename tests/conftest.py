import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs libkq kernels")


@pytest.fixture(scope="session")
def gpu():
    """The torch device the GPU tests allocate on. Skips when no GPU is
    visible; never falls back to the CPU."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from kernels_amd import kq
    kq.lib()  # loud failure if libkq is missing
    return torch.device("cuda:0")
