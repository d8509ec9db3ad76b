import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and runs the HIP path")


@pytest.fixture(scope="session")
def hip():
    """libpktito_amd with its device opened; the HIP path only, never a CPU one."""
    import libpktito_amd as pk
    pk.init()
    return pk
