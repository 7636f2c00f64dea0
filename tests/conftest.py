"""Shared pytest setup: import paths for the package binding and the oracle, the `gpu`
marker, and a session fixture that initialises device 0 through the C ABI."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "switch-l4t-gpu_amd")
for p in (PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs through libswitchgpu.so on device 0)")


@pytest.fixture(scope="session")
def gpu():
    """The binding, with device 0 initialised (every embedded code object loaded)."""
    import sgpu

    sgpu.init(0)
    return sgpu


@pytest.fixture(scope="session")
def sg():
    import sgpu

    return sgpu


@pytest.fixture(scope="session")
def og():
    import oracle

    return oracle
