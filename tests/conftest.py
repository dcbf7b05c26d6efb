import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libdcengine.so")


@pytest.fixture(scope="session")
def eng():
    """The drop-in nn_engine module (initialises the HIP device; no fallback)."""
    from directcompute_torch_amd import nn_engine
    return nn_engine
