import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("fused-lncc_amd", "oracle", "tests", os.path.join("tests", "golden")):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    config.addinivalue_line("markers", "slow: CPU test that takes tens of seconds")


import pytest  # noqa: E402


@pytest.fixture
def force_dchunk():
    """Calling force_dchunk(n) makes the library split D into chunks of n output planes for the
    launches this test makes on its thread (fl_test_set_dchunk); the planner decides again after."""
    from fused_lncc import _lib

    def set_planes(n):
        _lib.check(_lib.load().fl_test_set_dchunk(int(n)))

    yield set_planes
    _lib.load().fl_test_set_dchunk(0)
