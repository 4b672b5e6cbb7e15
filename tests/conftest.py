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
    """One HIP context for the bit-exact parity tests: the sequential
    reduction, so every op reproduces the CPU operators' bits (fails loudly
    when no GPU or library is present)."""
    from atlas_amd import ATLAS_REDUCTION_SEQUENTIAL, HipRuntime

    runtime = HipRuntime(0, ATLAS_REDUCTION_SEQUENTIAL)
    yield runtime
    runtime.close()


@pytest.fixture(scope="session")
def rt_auto():
    """A context with the library's default reduction (ATLAS_REDUCTION_AUTO):
    the tree engines for plain scaled rows, the sequential fold elsewhere."""
    from atlas_amd import ATLAS_REDUCTION_AUTO, HipRuntime

    runtime = HipRuntime(0, ATLAS_REDUCTION_AUTO)
    yield runtime
    runtime.close()
