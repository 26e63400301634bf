import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gpu():
    """The C-ABI library on a GPU box; fails loudly when either is missing."""
    from vai_amd import _capi
    lib = _capi.lib()
    if _capi.device_count() < 1:
        pytest.fail("no HIP device visible: GPU tests must run on the MI355X box")
    _capi.check(lib.vai_set_device(0), "set_device")
    return _capi
