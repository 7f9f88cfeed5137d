"""Test configuration: the `gpu` marker and shared fixtures.

`gpu` tests run the HIP library on an MI355X and compare it with the CPU
oracle; everything else runs on any machine (oracle vs reference build,
golden vectors, host logic, ABI checks).
"""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X; runs the HIP library")


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import load_reference
    r = load_reference()
    if r is None:
        pytest.skip("reference build oracle/_ref/libref.so is absent")
    return r


@pytest.fixture(scope="session")
def lib():
    from inference_c_amd import load_library
    return load_library()


@pytest.fixture(scope="session")
def sdk():
    """The HIP library on a GPU. A gpu test without a device fails: the
    library has no CPU path to fall back to."""
    from inference_c_amd import Sdk
    s = Sdk()
    if not s.available:
        pytest.fail("no HIP device available to a gpu-marked test")
    return s
