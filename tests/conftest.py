import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


@pytest.fixture(scope="session")
def gpu():
    """torch with a visible HIP device; GPU tests fail (not skip) without one."""
    import torch
    assert torch.cuda.is_available(), "GPU test started without a visible HIP device"
    return torch
