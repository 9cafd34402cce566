import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libobjeta_hip.so)")


@pytest.fixture(scope="session")
def backend():
    """One HIP context for all GPU tests. Fails (does not skip) if the library or the
    GPU is missing: GPU tests must exercise the native path."""
    from objeta_amd import HipBackend

    be = HipBackend(0, 2)
    yield be
    be.close()


@pytest.fixture(scope="session")
def quant(backend):
    from objeta_amd import QuantBackend

    return QuantBackend(backend)
