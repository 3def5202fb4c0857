import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (a HIP device) and the built library")


@pytest.fixture(scope="session")
def oracle():
    import _oracle
    return _oracle.Oracle()


@pytest.fixture(scope="session")
def kref():
    import _oracle
    ref = _oracle.ReferenceOracle.load()
    if ref is None:
        pytest.skip("oracle/_ref/libkref.so not built (reference checkout absent)")
    return ref


@pytest.fixture(scope="session")
def gpu():
    """The product library on device 0. Fails (does not skip) without a device."""
    import kunlunk200_lib_amd as kl
    kl.load()
    count = kl.device_count()
    assert count >= 1, "gpu-marked test needs a HIP device"
    return kl


@pytest.fixture(scope="session")
def kl():
    """The product library, loaded (no device needed)."""
    import kunlunk200_lib_amd as kl
    kl.load()
    return kl


@pytest.fixture
def knobs():
    """Sets library route/tile knobs (kunlun_set_tuning) for one test and
    restores the environment's values afterwards."""
    import kunlunk200_lib_amd as kl
    touched = set()

    def set_knob(name, value):
        kl.set_tuning(name, value)
        touched.add(name)

    yield set_knob
    for name in touched:
        kl.set_tuning(name, None)
