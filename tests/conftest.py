import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
for p in (HERE, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "ref: needs the vendored-ggml reference build (oracle/_ref)")


@pytest.fixture(scope="session")
def dev():
    """The GPU device; a gpu-marked test on a machine without one is an error,
    not a skip (the product path has no CPU fallback)."""
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("GPU test run without a GPU")
    return torch.device("cuda:0")
