import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o
    o.lib()
    return o


@pytest.fixture(autouse=True)
def _release_device_buffers(request):
    yield
    if request.node.get_closest_marker("gpu"):
        from tests import gpu_util
        if gpu_util.LIVE:
            gpu_util.release_all()
