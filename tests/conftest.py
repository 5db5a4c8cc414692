import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "faie2-flashnext_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through libfaie2fn.so)")


@pytest.fixture(scope="session")
def fnlib():
    """The product library (no fallback: a missing library or GPU is an error, not a skip)."""
    import fn

    return fn.FN()
