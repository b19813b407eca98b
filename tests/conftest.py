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


PKG_DIR = os.path.join(ROOT, "hunyuan-image-3-80b.cpp_amd")


def load_pkg():
    """Import the package directory (its name is not a Python identifier)."""
    import importlib.util
    if "hy3moe" in sys.modules:
        return sys.modules["hy3moe"]
    spec = importlib.util.spec_from_file_location("hy3moe", os.path.join(PKG_DIR, "__init__.py"),
                                                  submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["hy3moe"] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def hy():
    """The ctypes binding of libhy_moe.so (built in-tree by build.py)."""
    return load_pkg().hy_moe


@pytest.fixture(scope="session")
def gpu(hy):
    if hy.device_count() < 1:
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    return hy
