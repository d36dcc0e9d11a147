import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def hip():
    """One device context for the GPU tests of a session."""
    from yaxus_amd.backend import HipBackend

    b = HipBackend(0)
    yield b
    b.close()
