import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) and the built libnnhip.so")


@pytest.fixture(scope="session")
def ctx():
    """One device context (HIP stream) for all GPU tests of a session."""
    import gpu_util
    c = gpu_util.nnhip.Context(0)
    yield c
    c.close()
