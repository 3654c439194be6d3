import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def dev():
    """The one GPU, opened through the C ABI.  GPU tests fail (not skip) when
    the HIP library or the device is missing: the HIP path has no fallback."""
    import fuel_amd

    d = fuel_amd.RocmDevice(0)
    yield d
    d.close()
