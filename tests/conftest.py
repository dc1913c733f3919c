"""Shared test setup: the `gpu` marker, import paths and device fixtures."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("orbi-streammoe_amd", "oracle", "tests"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def ctx():
    import osm_hip

    if osm_hip.device_count() < 1:
        pytest.fail("no HIP device visible to libosm_hip.so")
    c = osm_hip.Context(0)
    yield c
    c.close()
