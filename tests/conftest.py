import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def cuda():
    """The GPU device; the native library must be loadable (no fallback)."""
    import torch
    from xllms_amd import _lib
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    _lib.backend()
    return torch.device("cuda:0")
