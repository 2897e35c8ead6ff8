"""Shared test setup: the repository root on sys.path, the ``gpu`` marker,
and in-tree builds of the native library and the oracle when missing."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


def _ensure_built():
    from cudacaml_amd import _lib, build

    if not os.path.exists(_lib.LIB_PATH):
        build.build()
    import oracle

    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()


_ensure_built()


@pytest.fixture(scope="session")
def device():
    """Fails (never skips) without a device: a GPU test must not pass
    silently on a machine that cannot run it."""
    from cudacaml_amd.runtime import Device

    if not Device.available():
        pytest.fail("no HIP device available for a gpu-marked test")
    Device.init()
    return Device.info()
