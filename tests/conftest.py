import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")
    config.addinivalue_line("markers", "slow: long CPU reference run")


@pytest.fixture(scope="session")
def P():
    """The CPU checkers (oracle/pyoracle.py)."""
    import pyoracle
    pyoracle.build()
    return pyoracle


@pytest.fixture(scope="session")
def qa():
    """The product's ctypes view (qwen-asr_amd/__init__.py)."""
    return importlib.import_module("qwen-asr_amd")


@pytest.fixture(scope="session")
def gpu(qa):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    qa.lib()   # loud failure if the HIP library is missing
    return torch
