import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_ROOT = os.path.join(ROOT, "adaptive-splash-attention_amd")
for _p in (ROOT, PKG_ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture
def pairing():
    """Set the forward's pairing mode for one test (asa_set_pairing: which
    forward kernel runs for 16-bit inputs), restoring the default after it."""
    from splash_attention import _lib

    yield _lib.set_pairing
    _lib.set_pairing("auto")
