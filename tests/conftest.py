"""Shared pytest setup: the `gpu` marker and import paths.

`-m gpu` tests run the HIP engine on a real MI355X and compare it with the
CPU restatement in oracle/ (test infrastructure) on the same seeded inputs.
`-m "not gpu"` tests pin the oracle itself and check the C ABI surface
without a GPU.
"""

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT,):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def engine():
    import mlxvs_amd

    return mlxvs_amd


@pytest.fixture(scope="session")
def oracle():
    import oracle as o

    o.lib()
    return o


def pytest_runtest_logstart(nodeid, location):
    # name the case before any GPU work starts, so a crash log says which
    if os.environ.get("MLXVS_TEST_ECHO"):
        print(f"\n[start] {nodeid}", flush=True)
