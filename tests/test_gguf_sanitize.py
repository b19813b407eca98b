"""The GGUF reader (host/hy_gguf.cpp) parses files it cannot trust.  Built on its own
with AddressSanitizer and UndefinedBehaviorSanitizer (host code, g++), it must open a
valid file and survive truncated and corrupted ones: every open either succeeds or
returns an error code, and nothing it then reads goes out of bounds."""
import os
import random
import shutil
import struct
import subprocess

import numpy as np
import pytest

import gguf_io as G

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "hunyuan-image-3-80b.cpp_amd", "host")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not found")
    out = str(tmp_path_factory.mktemp("san") / "gguf_san")
    cmd = [gxx, "-std=c++17", "-g", "-O1", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-I" + os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "cxx", "gguf_sanitize.cpp"), os.path.join(HOST, "hy_gguf.cpp"), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        if "sanitize" in r.stderr and ("unrecognized" in r.stderr or "cannot find" in r.stderr):
            pytest.skip("g++ without sanitizer runtimes")
        raise AssertionError(r.stderr[-3000:])
    return out


def _valid_file():
    rng = np.random.default_rng(3)
    a = rng.standard_normal((4, 64)).astype(np.float32)
    tensors = [("blk.0.t_f32", G.GGML_F32, (64, 4), a.tobytes())]
    for name, gt in (("blk.0.t_f16", G.GGML_F16), ("blk.0.t_bf16", G.GGML_BF16), ("blk.0.t_q8_0", G.GGML_Q8_0),
                     ("blk.0.t_q4_0", G.GGML_Q4_0)):
        t, _ = G.typed_tensor(a, gt)
        tensors.append((name, gt, (64, 4), t))
    kvs = [("general.architecture", G.T_STR, "hunyuan"), ("hunyuan.hidden_size", G.T_U32, 64),
           ("hunyuan.rms_norm_eps", G.T_F32, 1e-5), ("tokenizer.list", G.T_ARR, (G.T_STR, ["a", "bc", "def"])),
           ("nested", G.T_ARR, (G.T_U64, [1, 2, 3]))]
    return G.gguf_bytes(kvs, tensors, alignment=32)


def _hostile_headers():
    """Well-formed prefixes with hostile counts, lengths, dimensions and offsets."""
    out = []
    hdr = b"GGUF" + struct.pack("<I", 3)
    out.append(hdr + struct.pack("<QQ", 1 << 62, 0))                       # n_tensors huge
    out.append(hdr + struct.pack("<QQ", 0, 1 << 62))                       # n_kv huge
    out.append(hdr + struct.pack("<QQ", 0, 1) + struct.pack("<Q", 1 << 61) + b"k")   # key length huge
    kv = struct.pack("<Q", 1) + b"k"
    out.append(hdr + struct.pack("<QQ", 0, 1) + kv + struct.pack("<I", 99))          # unknown value type
    out.append(hdr + struct.pack("<QQ", 0, 1) + kv + struct.pack("<IIQ", G.T_ARR, G.T_ARR, 1 << 40))  # nested array
    out.append(hdr + struct.pack("<QQ", 0, 1) + kv + struct.pack("<IIQ", G.T_ARR, G.T_STR, 1 << 40))  # many strings
    out.append(hdr + struct.pack("<QQ", 0, 1) + kv + struct.pack("<IQ", G.T_STR, 1 << 50))  # string value huge
    tname = struct.pack("<Q", 1) + b"t"
    for nd, ne, gt, off in ((9, [4], G.GGML_F32, 0), (2, [1 << 40, 1 << 40], G.GGML_F32, 0),
                            (1, [64], 12345, 0), (1, [64], G.GGML_F32, 1 << 60), (1, [33], G.GGML_Q8_0, 0),
                            (4, [0, 5, 7, 1], G.GGML_F32, 0), (1, [64], G.GGML_F32, (1 << 64) - 8)):
        t = tname + struct.pack("<I", nd) + b"".join(struct.pack("<Q", n) for n in ne[:min(nd, 4)])
        t += struct.pack("<IQ", gt, off)
        out.append(hdr + struct.pack("<QQ", 1, 0) + t + b"\0" * 64)
    # alignment values: 0, not a power of two, huge
    for al in (0, 3, 1 << 31):
        kvs = struct.pack("<Q", len(b"general.alignment")) + b"general.alignment" + struct.pack("<II", G.T_U32, al)
        out.append(hdr + struct.pack("<QQ", 1, 1) + kvs + tname + struct.pack("<IQIQ", 1, 8, G.GGML_F32, 0) + b"\0" * 96)
    return out


def test_reader_under_sanitizers(driver, tmp_path):
    good = _valid_file()
    files = []

    def put(b):
        p = tmp_path / f"f{len(files):04d}.gguf"
        p.write_bytes(bytes(b))
        files.append(str(p))

    put(good)
    for cut in list(range(0, 160)) + list(range(160, len(good), 37)):
        put(good[:cut])                                      # every header prefix, then the data
    rnd = random.Random(7)
    for _ in range(300):                                     # byte flips, mostly in the header
        b = bytearray(good)
        for _ in range(rnd.randint(1, 4)):
            pos = rnd.randrange(min(len(b), 400)) if rnd.random() < 0.8 else rnd.randrange(len(b))
            b[pos] = rnd.randrange(256)
        put(b)
    for b in _hostile_headers():
        put(b)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([driver] + files, capture_output=True, text=True, env=env, timeout=300)
    assert r.returncode == 0, (r.stdout[-2000:] + r.stderr[-6000:])
    opened = int(r.stdout.split("opened ")[1].split()[0])
    assert opened >= 1, r.stdout            # the valid file opens
    assert opened < len(files), r.stdout    # and the damaged ones are not all accepted
