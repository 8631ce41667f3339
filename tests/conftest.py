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


def pytest_collection_modifyitems(config, items):
    """The host-sanitized libraries (MIAIE_LIB_DIR=.../lib_san) are for the
    CPU tests only: ASan's allocator in the same process as the HIP runtime
    is not a supported GPU configuration, so GPU tests are skipped there."""
    lib_dir = os.environ.get("MIAIE_LIB_DIR", "")
    if "lib_san" not in lib_dir:
        return
    skip = pytest.mark.skip(reason="MIAIE_LIB_DIR selects the host-sanitized build: CPU tests only")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
