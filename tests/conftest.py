import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")
    config.addinivalue_line("markers", "slow: exhaustive CPU check (tens of seconds)")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu():
    """torch on cuda:0; a GPU test without a GPU is an error, not a skip."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    torch.cuda.init()
    return torch
