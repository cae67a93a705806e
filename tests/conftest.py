"""Shared fixtures. `gpu` marks tests that need an MI355X; every other test runs on the CPU."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def oracle():
    import oracle_lib
    return oracle_lib.Oracle()


@pytest.fixture(scope="session")
def ctx():
    from modelspec_amd import api
    if api.device_count() < 1:
        pytest.fail("no HIP device is visible to a gpu-marked test")
    c = api.Context(0)
    yield c
    c.close()
