"""Shared test setup.

Markers: `gpu` tests need a real MI355X and the built HIP library; everything
else runs on the CPU (oracle checks, ABI/export checks, host logic).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and build/libtinytorch.so")


@pytest.fixture(scope="session")
def tlib():
    """The GPU library, with a hard failure when no GPU is usable."""
    import tinytorch_amd
    tinytorch_amd.require_gpu()
    return tinytorch_amd.lib()


@pytest.fixture(scope="session")
def orc():
    import orc as _orc
    return _orc
