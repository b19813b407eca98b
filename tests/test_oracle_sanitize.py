"""The oracle's C code (oracle/hy_oracle.c, oracle/hy_oracle_attn.c) built with
AddressSanitizer and UndefinedBehaviorSanitizer: the oracle's own test files run
against that build in a child process, so an out-of-bounds access, an overflow or a
misaligned load in the checker fails here instead of silently bending a parity result."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")


def test_oracle_under_sanitizers(tmp_path):
    gcc = shutil.which("gcc")
    if not gcc:
        pytest.skip("gcc not found")
    so = str(tmp_path / "liboracle_san.so")
    cmd = [gcc, "-std=c11", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-fopenmp", "-shared",
           "-o", so, os.path.join(ORACLE, "hy_oracle.c"), os.path.join(ORACLE, "hy_oracle_attn.c"), "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        if "sanitize" in r.stderr and ("unrecognized" in r.stderr or "cannot find" in r.stderr):
            pytest.skip("gcc without sanitizer runtimes")
        raise AssertionError(r.stderr[-3000:])
    rt = []
    for name in ("libasan.so", "libubsan.so"):
        p = subprocess.run([gcc, "-print-file-name=" + name], capture_output=True, text=True).stdout.strip()
        if not os.path.isabs(p) or not os.path.exists(p):
            pytest.skip(f"{name} not found")
        rt.append(p)
    env = dict(os.environ, HY_ORACLE_LIB=so, LD_PRELOAD=" ".join(rt),
               ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    probe = ("import sys; sys.path.insert(0, %r); import hy_oracle as O; O.lib(); "
             "print('loaded', open('/proc/self/maps').read().count(%r) > 0)" % (ORACLE, so))
    r = subprocess.run([sys.executable, "-c", probe], capture_output=True, text=True, env=env, timeout=120)
    assert r.returncode == 0 and "loaded True" in r.stdout, r.stdout + r.stderr[-2000:]
    files = [os.path.join(ROOT, "tests", f) for f in ("test_oracle_kat.py", "test_oracle_ref.py",
                                                      "test_oracle_attn.py")]
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu"]
                       + files, capture_output=True, text=True, env=env, cwd=ROOT, timeout=600)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
    assert " passed" in r.stdout, r.stdout[-2000:]
