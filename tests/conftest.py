"""Test configuration: the `gpu` marker and the device context.

Tests marked `gpu` need an MI355X (gfx950) and run with `pytest -m gpu`; the others run on any
host (`pytest -m "not gpu"`) and never touch a device.
"""

import os
import sys

import pytest

TESTS = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(TESTS)
for path in (ROOT, TESTS):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libtmhip.so")


@pytest.fixture(scope="session")
def ctx():
    from transmuter_amd import Context

    c = Context(0)
    yield c
    c.synchronize()
    c.close()
