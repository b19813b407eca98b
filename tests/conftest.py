"""pytest configuration: the `gpu` marker and import paths for the oracle and the package."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
for p in (ROOT, ORACLE_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_oracle():
    lib = os.path.join(ORACLE_DIR, "liboracle.so")
    if not os.path.exists(lib):
        subprocess.run(["make", "-C", ORACLE_DIR, "all"], check=True,
                       stdout=subprocess.DEVNULL)


_ensure_oracle()


@pytest.fixture(scope="session")
def oracle():
    import hy_oracle
    hy_oracle.lib()
    return hy_oracle


@pytest.fixture(scope="session")
def refimpl(oracle):
    if not oracle.ref_available():
        pytest.skip("oracle/_ref/libhy_ref.so not built (needs the reference tree)")
    return oracle.ref()
