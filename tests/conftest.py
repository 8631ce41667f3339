import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the miaie C ABI")


@pytest.fixture(scope="session")
def ctx():
    """One miaie context on device 0 for the whole GPU session."""
    import aiehlc_amd as mi

    c = mi.Context(0)
    yield c
    c.close()
