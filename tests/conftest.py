import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libmiikv.so")


@pytest.fixture(scope="session")
def gpu():
    """Skip nothing: a gpu-marked test on a box without a GPU must fail loudly."""
    import torch
    assert torch.cuda.is_available(), "gpu-marked test run without a GPU"
    import miinfer_amd
    miinfer_amd.lib()
    return torch.device("cuda:0")
