"""Shared fixtures.  GPU tests are marked `gpu` and call the HIP library
through its C ABI; CPU tests cover the oracle, host logic and the ABI's
exports."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def ora():
    import oracle as _oracle

    _oracle.lib()
    return _oracle


@pytest.fixture(scope="session")
def rt():
    """One HIP context for the whole GPU session (fails loudly when absent)."""
    from atlas_amd import HipRuntime

    runtime = HipRuntime(0)
    yield runtime
    runtime.close()
