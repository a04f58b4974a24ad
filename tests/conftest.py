import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "deepseek-v4-flash-offload_amd")
for _p in (PKG, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The ROCm device; a GPU test on a box without one fails loudly."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test requested but torch.cuda.is_available() is False")
    from dsv4_hip import _lib
    _lib.lib()  # raises if the HIP library is missing
    return torch.device("cuda:0")
