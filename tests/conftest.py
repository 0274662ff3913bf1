import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); runs the C-ABI kernels")


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.skip("GPU required")
    return torch.device("cuda")


@pytest.fixture(autouse=True)
def _restore_config():
    from sparsetriton_amd.config import _STATE

    saved = dict(_STATE)
    yield
    _STATE.clear()
    _STATE.update(saved)
