import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libqr_attn on cuda:0)")


@pytest.fixture(scope="session")
def gpu():
    """Fails (never skips) when a test marked gpu runs without a usable GPU."""
    import torch

    assert torch.cuda.is_available(), "GPU test needs a ROCm device"
    torch.cuda.set_device(0)
    import qauntrunner_amd

    qauntrunner_amd.load()
    return torch.device("cuda:0")
