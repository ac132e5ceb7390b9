import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "xdna.cpp_amd"))
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def reflib():
    from oracle import RefLib
    if not RefLib.available():
        pytest.skip("oracle/_ref/libxdna_ref.so not built (reference sources absent)")
    return RefLib()


@pytest.fixture(scope="session")
def lib():
    import mi355x
    return mi355x.load()


@pytest.fixture(scope="session")
def ctx():
    import mi355x
    if mi355x.device_count() < 1:
        pytest.fail("no HIP device visible: GPU tests need the MI355X")
    c = mi355x.Context(0)
    yield c
    c.close()
