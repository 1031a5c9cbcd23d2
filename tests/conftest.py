import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def golden():
    import json

    base = os.path.join(ROOT, "tests", "golden")

    def load(name):
        with open(os.path.join(base, name)) as f:
            return json.load(f)

    return load


@pytest.fixture(scope="session")
def torch_cuda():
    """The GPU tests' torch handle.  Skips only when no GPU is visible."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch
