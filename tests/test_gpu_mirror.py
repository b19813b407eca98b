"""The reference's C++ API (include/hunyuan_moe_full.h) as served by the GPU
library: tests/cxx/test_mirror (built by build.py) calls it like the reference's
callers do and checks every result against the oracle."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cxx", "test_mirror")


def test_cxx_mirror_api(gpu):
    assert os.path.exists(EXE), "tests/cxx/test_mirror is not built (python hunyuan-image-3-80b.cpp_amd/build.py)"
    r = subprocess.run([EXE], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    print(r.stdout)
    lines = [l for l in r.stdout.splitlines() if l.startswith(("PASS", "FAIL"))]
    assert len(lines) >= 15, r.stdout
    assert r.returncode == 0, "\n".join(l for l in lines if l.startswith("FAIL"))
