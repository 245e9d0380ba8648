import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import g4o
    g4o.lib()
    return g4o


@pytest.fixture(scope="session")
def gpu():
    """The HIP library, initialised on device 0 (GPU tests fail loudly without it)."""
    import g4run_amd as G
    G.init(0)
    return G
