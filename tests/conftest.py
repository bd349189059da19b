import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libviktor_hip.so")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN


def gpu_available():
    import torch
    return torch.cuda.is_available() and torch.version.hip is not None
