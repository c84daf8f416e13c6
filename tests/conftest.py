"""pytest configuration: the ``gpu`` marker and import paths.

Tests marked ``gpu`` need an MI355X (gfx950) and the built libkan_hip.so;
everything else runs on the CPU.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture
def routes():
    """Restores every routing switch of libkan_hip.so (kan_hip_set_route)
    after the test; the test sets them through _lib.set_route."""
    from torchsplinekan_amd import _lib
    saved = {name: _lib.get_route(name) for name in _lib.ROUTES}
    yield _lib
    for name, value in saved.items():
        _lib.set_route(name, value)
