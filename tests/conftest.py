import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); parity of the HIP path")


@pytest.fixture(scope="session")
def orc():
    from oracle.bindings import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.bindings import Reference

    if not Reference.available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return Reference()


@pytest.fixture(scope="session")
def ref_gen1():
    from oracle.bindings import RefGen1

    if not RefGen1.available():
        pytest.skip("oracle/_ref/libref_gen1.so not built (reference sources absent)")
    return RefGen1()


@pytest.fixture(scope="session")
def gpu():
    """The native library on a visible device.  Fails (does not skip) when the
    library or the device is missing: GPU tests must exercise the HIP path."""
    import laii_amd as la

    la.load()
    la.require_gpu()
    return la
