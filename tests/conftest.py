import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on the device)")


@pytest.fixture(scope="session")
def kgx():
    return importlib.import_module("katago-rs_amd")


@pytest.fixture(scope="session")
def synth():
    return importlib.import_module("katago-rs_amd.synth")


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    return o
