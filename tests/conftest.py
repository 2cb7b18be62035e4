"""Test configuration: the `gpu` marker and import paths.

CPU tests (`-m "not gpu"`) pin the oracle against golden vectors and check the
host side of the C ABI; GPU tests (`-m gpu`) are the parity tests proper and
call libmxfp4hip through its C ABI.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mpp-4.1-fp4-fp8-block_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def dev():
    """One libmxfp4hip context for the whole GPU session."""
    import mxfp4hip
    d = mxfp4hip.Device(0)
    yield d
    d.close()
