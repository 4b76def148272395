import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built extension")


@pytest.fixture(scope="session")
def hip():
    """The philtorch_amd package, with the HIP extension required and loaded."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    import philtorch_amd

    philtorch_amd.require_extension()
    return philtorch_amd
