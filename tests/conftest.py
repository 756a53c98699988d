"""Shared test setup.

Tests marked ``gpu`` need an MI355X and call the HIP library through its C
ABI; everything else runs on the CPU (oracle pinning, host logic, ABI
exports).  The oracle is the checker here and is never a compute path of the
product.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import __graft_entry__ as entry  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def pkg():
    return entry.load_package()


@pytest.fixture(scope="session")
def ora():
    return entry.load_oracle()


@pytest.fixture(scope="session")
def backend(pkg):
    be = pkg.hip.Backend(0)
    yield be
    be.close()
