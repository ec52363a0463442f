"""Shared test configuration.

Markers: ``gpu`` -- needs a gfx950 device and the built libmmp_hip.so; the
driver runs ``-m "not gpu"`` on CPU and ``-m gpu`` on an MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs an MI355X (gfx950) GPU")


@pytest.fixture(autouse=True)
def _reset_config():
    """Each test starts from the default configuration (the reference's
    tests reset float64 handling the same way, tests/conftest.py:135-142)."""
    from macmetalpy_amd._config import set_config
    set_config(float64_behavior="cpu_fallback", fusion=True, warn_on_downcast=True,
               fast_math=False, native_dispatch=True)
    yield
    set_config(float64_behavior="cpu_fallback", fusion=True, warn_on_downcast=True,
               fast_math=False, native_dispatch=True)


@pytest.fixture(autouse=True)
def _no_device_wait_timeouts(request):
    """After every GPU test: no split reduction or scan may have run out of
    its bounded cross-workgroup wait (that would make its result suspect)."""
    yield
    if request.node.get_closest_marker("gpu") is None:
        return
    from macmetalpy_amd._backend import HipBackend
    flags = HipBackend().wait_status()
    assert flags == 0, f"device-side wait ran out during this test (flags {flags:#x})"
