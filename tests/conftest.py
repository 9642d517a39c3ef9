import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; calls the HIP library through its C ABI")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; GPU tests fail (not skip) when the library or device is missing."""
    import torch

    import femtochat_amd._lib as L

    L.lib()  # raises if the library is not built
    assert torch.cuda.is_available(), "GPU test run without a visible HIP device"
    return torch.device("cuda", 0)
