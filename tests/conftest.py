"""Shared pytest setup: the `gpu` marker, import paths, seeded input generators."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llama-cpp-ascend310b4-addon_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C ABI on the device)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def mi():
    import ggml_mi355x
    ggml_mi355x.lib()
    return ggml_mi355x


@pytest.fixture(scope="session")
def gpu(mi):
    n = mi.device_count()
    if n < 1:
        pytest.fail("gpu-marked test run without a HIP device: " + mi.last_error())
    return mi
