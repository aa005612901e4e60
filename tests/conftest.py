import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "sparse-matrix-multiplication_amd")
for p in (PKG_DIR, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libspmm_amd.so on cuda:0)")


@pytest.fixture(scope="session")
def S():
    """The engine's Python binding (loads libspmm_amd.so; raises if not built)."""
    import spmm_amd
    spmm_amd.lib()
    return spmm_amd


@pytest.fixture(scope="session")
def O():
    """The CPU oracle (tests only)."""
    import oracle_lib
    oracle_lib.lib()
    return oracle_lib
