import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP path")


@pytest.fixture(scope="session")
def runtime():
    """The rocm backend's runtime. A GPU test fails, rather than skips, when
    the library or the device is missing: there is no other path."""
    import turboembed_amd as T
    rt = T.Runtime()
    assert rt.device_count() >= 1, "no gfx950 device listed by the rocm backend"
    return rt


@pytest.fixture(scope="session")
def context(runtime):
    ctx = runtime.context(0)
    yield ctx
    ctx.close()
