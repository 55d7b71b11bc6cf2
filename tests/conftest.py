import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (runs on the MI355X box)")


@pytest.fixture(scope="session")
def plugin():
    from pjrtx_amd.pjrt import plugin as get
    return get()


@pytest.fixture(scope="session")
def client(plugin):
    from pjrtx_amd.pjrt import Client
    if plugin.device_count() == 0:
        pytest.fail("GPU test ran on a host without a visible HIP device")
    c = Client()
    yield c
