"""Build recipe for libhy_moe.so (gfx950 HIP kernels + C ABI + the C++ mirror of the
reference API), compiled in-tree with hipcc.

    python hunyuan-image-3-80b.cpp_amd/build.py          # build
    python hunyuan-image-3-80b.cpp_amd/build.py --asm    # also keep gfx950 assembly in _build/

Every HIP translation unit is compiled with
  -ffp-contract=off   : no implicit mul+add fusion, so the bit-exact paths (router
                        order, quantizers) do only the roundings written in the source;
  -Xclang -target-feature -Xclang -packed-fp32-ops : no packed FP32 instructions.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libhy_moe.so")
PROBE = os.path.join(HERE, "probe")
PROBE_LIB = os.path.join(HERE, "libhy_probe.so")   # bench.py's measurement probes only
ARCH = "gfx950"

COMMON = ["-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wno-unused-command-line-argument"]


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def sources():
    hips = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    cpps = sorted(os.path.join(HOST, f) for f in os.listdir(HOST) if f.endswith(".cpp")) if os.path.isdir(HOST) else []
    return hips, cpps


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the device-only target feature: drop that warning
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l and l.strip()
                    and "warning generated" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}")
    return out


def build_oracle(with_ref=None):
    """The CPU oracle (test infrastructure) and, when the reference tree is present,
    oracle/_ref from the reference's own source."""
    oracle = os.path.join(ROOT, "oracle")
    subprocess.run(["make", "-s", "-C", oracle, "all"], check=True)
    if with_ref is None:
        with_ref = os.path.isdir("/root/reference/src")
    if with_ref:
        subprocess.run(["make", "-s", "-C", oracle, "ref"], check=True)


def build_cxx_tests():
    """tests/cxx/test_mirror: the C++ API mirror checked against the oracle."""
    src = os.path.join(ROOT, "tests", "cxx", "test_mirror.cpp")
    out = os.path.join(ROOT, "tests", "cxx", "test_mirror")
    cmd = ["g++", "-std=c++17", "-O2", src, f"-I{os.path.join(ROOT, 'include')}", f"-I{os.path.join(ROOT, 'oracle')}",
           f"-L{HERE}", "-lhy_moe", f"-L{os.path.join(ROOT, 'oracle')}", "-loracle",
           "-Wl,-rpath,$ORIGIN/../../hunyuan-image-3-80b.cpp_amd", "-Wl,-rpath,$ORIGIN/../../oracle",
           "-Wl,--allow-shlib-undefined", "-o", out + ".tmp"]
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


def build_all(asm=False, jobs=8, verbose=False):
    build_oracle()
    lib = build(asm=asm, jobs=jobs, verbose=verbose)
    build_probe()
    build_cxx_tests()
    return lib


def build_probe():
    """libhy_probe.so: the measurement probes bench.py reports ceilings from.  A separate
    library, so that nothing of it is linked into or exported by libhy_moe.so."""
    os.makedirs(BUILD, exist_ok=True)
    cc = hipcc()
    objs = []
    for f in sorted(os.listdir(PROBE)):
        if f.endswith(".hip"):
            obj = os.path.join(BUILD, "probe_" + f + ".o")
            _run([cc] + COMMON + DEVICE + [f"-I{PROBE}", "-c", os.path.join(PROBE, f), "-o", obj])
            objs.append(obj)
    tmp = PROBE_LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build(asm=False, jobs=8, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    hips, cpps = sources()
    cc = hipcc()
    cmds = []
    objs = []
    for src in hips + cpps:
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        objs.append(obj)
        flags = COMMON + DEVICE if src.endswith(".hip") else COMMON + ["-x", "c++"]
        cmds.append([cc] + flags + ["-c", src, "-o", obj])
        if asm and src.endswith(".hip"):
            cmds.append([cc] + COMMON + DEVICE + ["--cuda-device-only", "-S", src, "-o",
                                                  os.path.join(BUILD, os.path.basename(src) + f".{ARCH}.s")])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for out in ex.map(_run, cmds):
            if out and verbose:
                print(out)
    tmp = LIB + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--asm", action="store_true")
    ap.add_argument("-j", type=int, default=8)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build_all(asm=a.asm, jobs=a.j, verbose=a.v))
    sys.exit(0)
