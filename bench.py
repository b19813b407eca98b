#!/usr/bin/env python3
"""Benchmark of the MI355X MoE feed-forward block (HunyuanImage-3 shape).

Default workload (what the one JSON line reports): the 32-layer stack of the MoE block
with GGUF Q8_0 weights, all resident in HBM (about 84 GB): per layer RMSNorm (eps 1e-5)
-> MoE (hidden 4096, 64 routed + 1 shared experts of width 3072, top-8) -> residual
add, T=4096 tokens per step, inputs resident in HBM.  A step is the whole stack;
tokens/s = T / step time.  Weights are random-init N(0, 0.02) seeded by layer index
(synthetic, generated on the device), activations N(0, 1).  The same line carries the
decode (Q4_0, T=1, 2, 4 and 8) and the Zipf-skewed image-token (Q4_0, T=4096) layers as
`extras`, each timed in its own region, with the T=512 Q8_0 layer and the F32 T=16
layer, so that every configuration has a number in the one line.

Other workloads (--config): c1 F32 T=16, c2 Q8_0 T=512, c3 Q4_0 decode (--tokens
1/2/4/8), c4 Q4_0 T=4096 Zipf-skewed routing, c5 the stack (default).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c5] [--no-cpu] [--no-extras]
    python bench.py --mfma-probe          # the grouped GEMM's per-block instruction mix alone
    python bench.py --stream-probe 864    # HBM read rate of the decode GEMV's streams
    python bench.py --l2-probe            # global->LDS copy rate from L2 / Infinity Cache / HBM windows
    python bench.py --copy-probe 1024     # plain 1 GiB device copy (counter yardstick)
    python bench.py --gguf-load /tmp/l.gguf [--config c2]   # layer load from a GGUF file
    python bench.py --attn [--tokens 4096]   # attention half of a decoder layer (fp32)
    python bench.py --model [--tokens 512]   # resident backbone: embedding, 32 layers, lm_head

roofline.traffic (HBM bytes per launch of the dominant kernel) is read from
profiles/hbm_traffic.md, the table made from rocprofv3 FETCH_SIZE / WRITE_SIZE
counter runs of this script, calibrated against the copy probe; it is null for a
workload/kernel the table does not list.
"""
import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

H, I, E, K = 4096, 3072, 64, 8
PEAK_HBM = 8.0e12          # B/s, MI355X HBM3E
PEAK_INT8 = 5.0e15         # ops/s, dense int8 MFMA
PEAK_FP32_MFMA = 157.3e12  # FLOP/s, dense fp32 MFMA
# The grouped int8 GEMM keeps ggml's per-block fp32 rescale: every 32-MAC block partial
# costs an int->float conversion and an fma on the vector ALUs, and a rank-1 MFMA forms
# the scale products.  Its ceiling is measured in the same run by a compute-only probe
# of exactly that per-block instruction mix (hyp_block_mix in libhy_probe.so, probe_block_mix below)
PROBE_WGS, PROBE_ITERS = 512, 4000
ATTN = dict(H=4096, nh=32, nkv=8, hd=128)   # HunyuanImage-3 attention shape
PARAMS_PER_EXPERT = 3 * H * I
BYTES = {0: 4.0, 8: 34.0 / 32.0, 2: 18.0 / 32.0}   # bytes per weight element


def load_pkg():
    import importlib.util
    pkg = os.path.join(ROOT, "hunyuan-image-3-80b.cpp_amd")
    spec = importlib.util.spec_from_file_location("hy3moe", os.path.join(pkg, "__init__.py"),
                                                  submodule_search_locations=[pkg])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["hy3moe"] = mod
    spec.loader.exec_module(mod)
    return mod.hy_moe


WORKLOADS = {
    "c1": dict(name="moe_layer_f32_t16", wtype=0, T=16, layers=1, rot=1),
    "c2": dict(name="moe_layer_q8_0_t512", wtype=8, T=512, layers=1, rot=2),
    "c3": dict(name="moe_layer_q4_0_decode", wtype=2, T=1, layers=1, rot=8),
    "c4": dict(name="moe_layer_q4_0_t4096_zipf", wtype=2, T=4096, layers=1, rot=1, zipf=True),
    "c5": dict(name="moe_stack32_q8_0_t4096", wtype=8, T=4096, layers=32, rot=1, stack=True),
}


# beta of the Zipf(1.1) router bias, calibrated on this workload's own inputs (seed 42,
# T=4096, N(0, 0.02) router, N(0, 1) activations, feature 0 set to 1) so that the eight
# most popular experts take 63 % of the 32,768 (token, expert) pairs, the top-8 mass of
# Zipf(1.1) over 64 experts.  At this beta the hottest expert serves 3,977 of 4,096
# tokens (12.1 % of pairs: one pair per token is the most any expert can take).
ZIPF_BETA = 1.27


def zipf_bias(seed=42, s=1.1, beta=ZIPF_BETA):
    """Per-expert additive router bias b_e = beta * ln p_e, p_e ~ rank^-s under a seeded
    rank permutation (folded into input feature 0, which is set to 1)."""
    rng = np.random.default_rng(seed)
    ranks = rng.permutation(E) + 1
    p = ranks.astype(np.float64) ** -s
    p /= p.sum()
    return (beta * np.log(p)).astype(np.float32)


def expert_bytes(wtype):
    return PARAMS_PER_EXPERT * BYTES[wtype]


def kernel_traffic(kname, wtype, T, D, shared=True):
    """Algorithmic HBM bytes of one launch of a kernel of the layer forward."""
    wb = BYTES[wtype]
    n_exp = D + (1 if shared else 0)
    act_b = 1.0 + 8.0 / 32.0 if wtype != 0 else 4.0   # int8 + scale + sum per element
    if kname == "ffn_up":
        return n_exp * 2 * I * H * wb + T * H * act_b + (T * K + T) * I * act_b
    if kname == "ffn_down":
        return n_exp * H * I * wb + (T * K + T) * I * act_b + (T * K + T) * H * 4
    if kname == "combine":
        return T * (K + 1) * H * 4 + T * H * 4 * 2
    return 0.0


def kernel_ops(kname, T):
    if kname == "ffn_up":
        return 2.0 * T * (K + 1) * 2 * I * H
    if kname == "ffn_down":
        return 2.0 * T * (K + 1) * H * I
    return 0.0


TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "hbm_traffic.md")


def measured_traffic(workload, kname, path=TRAFFIC_TABLE):
    """HBM bytes per launch for (workload, kernel) from the committed counter table:
    rows '| workload | kernel | ... | bytes |' whose last cell is the calibrated
    FETCH+WRITE bytes per dispatch."""
    try:
        with open(path) as f:
            for line in f:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 3 and cells[0] == workload and cells[1] == kname:
                    return float(cells[-1])
    except (OSError, ValueError):
        return None
    return None


PROBE_LIB = os.path.join(ROOT, "hunyuan-image-3-80b.cpp_amd", "libhy_probe.so")
_probe = None


def probe_lib():
    """libhy_probe.so: the measurement probes (hunyuan-image-3-80b.cpp_amd/probe/), a
    library of their own beside the product library."""
    global _probe
    if _probe is None:
        import ctypes as C
        if not os.path.exists(PROBE_LIB):
            raise RuntimeError(f"{PROBE_LIB} is not built: run python hunyuan-image-3-80b.cpp_amd/build.py")
        L = C.CDLL(PROBE_LIB)
        L.hyp_last_error.restype = C.c_char_p
        L.hyp_block_mix.restype = C.c_int
        L.hyp_block_mix.argtypes = [C.c_int32, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]
        L.hyp_stream.restype = C.c_int
        L.hyp_stream.argtypes = [C.c_int32, C.c_void_p, C.c_uint64, C.c_uint32, C.c_void_p, C.c_void_p]
        L.hyp_l2_window.restype = C.c_int
        L.hyp_l2_window.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p]
        _probe = L
    return _probe


def probe_check(rc):
    if rc != 0:
        raise RuntimeError(f"probe error: {probe_lib().hyp_last_error().decode()}")


def probe_block_mix(hy, variant=0, reps=3):
    """Rate (block-dot int8 ops/s) of the grouped GEMM's per-block instruction mix with
    no memory traffic: the best of `reps` launches of hyp_block_mix (variant 0: the
    whole mix; 1: its four MFMAs only; 2: its 64 vector ops only; 3: the f16 block-dot
    alternative, without the operand unpack it would also need; 4: the same with the
    int8 A operand unpacked to f16)."""
    out = hy.Buf.empty((PROBE_WGS * 512,))
    st = hy.Stream()
    ev0, ev1 = hy.C.c_void_p(), hy.C.c_void_p()
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev0)))
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev1)))
    probe_check(probe_lib().hyp_block_mix(variant, PROBE_WGS, 100, out.ptr, st.h))
    best = None
    for _ in range(reps):
        hy.check(hy.lib().hy_event_record(ev0, st.h))
        probe_check(probe_lib().hyp_block_mix(variant, PROBE_WGS, PROBE_ITERS, out.ptr, st.h))
        hy.check(hy.lib().hy_event_record(ev1, st.h))
        st.synchronize()
        ms = hy.C.c_float()
        hy.check(hy.lib().hy_event_elapsed_ms(ev0, ev1, hy.C.byref(ms)))
        best = ms.value if best is None else min(best, ms.value)
    for e in (ev0, ev1):
        hy.lib().hy_event_destroy(e)
    st.close()
    ops = PROBE_WGS * 8.0 * PROBE_ITERS * 2 * 32 * 32 * 32 * 2
    return ops / (best / 1e3)


def stream_probe(hy, waves=864, kb_per_wave=144, sets=8, launches=40):
    """HBM read rate of the decode GEMV's access pattern: `waves` single-wave streams of
    kb_per_wave KB each (864 x 144 KB is the Q4_0 T=1 gate/up launch: 9 experts x 96
    row groups of 64 rows x 4096 columns), rotating over `sets` separate buffers so the
    256 MB Infinity Cache cannot serve a repeat; variant 2 streams with non-temporal
    copies (as the decode GEMV does), variant 1 reads the same bytes with a grid-stride
    vector loop."""
    per = waves * kb_per_wave * 1024
    buf = hy.Buf(per * sets, np.uint8)
    hy.check(hy.lib().hy_memset(buf.ptr, 1, per * sets))
    out = hy.Buf.empty((waves * 64,))
    st = hy.Stream()
    ev0, ev1 = hy.C.c_void_p(), hy.C.c_void_p()
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev0)))
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev1)))
    res = {}
    for variant, name in ((0, "dma_streams"), (2, "dma_streams_nontemporal"), (1, "vector_grid_stride")):
        for i in range(sets):
            probe_check(probe_lib().hyp_stream(variant, buf.ptr + i * per, per, waves, out.ptr, st.h))
        hy.check(hy.lib().hy_event_record(ev0, st.h))
        for i in range(launches):
            probe_check(probe_lib().hyp_stream(variant, buf.ptr + (i % sets) * per, per, waves, out.ptr, st.h))
        hy.check(hy.lib().hy_event_record(ev1, st.h))
        st.synchronize()
        ms = hy.C.c_float()
        hy.check(hy.lib().hy_event_elapsed_ms(ev0, ev1, hy.C.byref(ms)))
        t = ms.value / launches / 1e3
        res[name] = {"us_per_launch": t * 1e6, "GBps": per / t / 1e9, "frac_of_8TBps": per / t / PEAK_HBM}
    for e in (ev0, ev1):
        hy.lib().hy_event_destroy(e)
    st.close()
    print(json.dumps({"probe": "stream_read", "waves": waves, "bytes_per_wave": kb_per_wave * 1024,
                      "bytes_per_launch": per, "rotating_sets": sets, "launches": launches, **res}), flush=True)


def l2_probe(hy, windows_kb=(1024, 65536, 1048576), wgs_per_cu=4, launches=5):
    """Copy rate of 1 KB global->LDS copies (the grouped GEMM's operand copies) from a
    window of each size: 1 MiB stays in every XCD's 4 MB L2, 64 MiB in the 256 MB
    Infinity Cache, 1 GiB comes from HBM."""
    wgs = 256 * wgs_per_cu
    out = hy.Buf.empty((wgs * 256,))
    st = hy.Stream()
    ev0, ev1 = hy.C.c_void_p(), hy.C.c_void_p()
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev0)))
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev1)))
    res = {}
    for kb in windows_kb:
        buf = hy.Buf(kb * 1024, np.uint8)
        hy.check(hy.lib().hy_memset(buf.ptr, 1, kb * 1024))
        iters = max(4, int(2e9 / (wgs * 4 * 8 * 1024)))  # ~2 GB copied per launch
        probe_check(probe_lib().hyp_l2_window(buf.ptr, kb * 1024, wgs, iters, out.ptr, st.h))
        hy.check(hy.lib().hy_event_record(ev0, st.h))
        for _ in range(launches):
            probe_check(probe_lib().hyp_l2_window(buf.ptr, kb * 1024, wgs, iters, out.ptr, st.h))
        hy.check(hy.lib().hy_event_record(ev1, st.h))
        st.synchronize()
        ms = hy.C.c_float()
        hy.check(hy.lib().hy_event_elapsed_ms(ev0, ev1, hy.C.byref(ms)))
        t = ms.value / launches / 1e3
        nbytes = wgs * 4 * 8 * 1024 * iters
        res[f"window_{kb // 1024}MiB"] = {"us_per_launch": t * 1e6, "TBps": nbytes / t / 1e12}
        buf.free()
    for e in (ev0, ev1):
        hy.lib().hy_event_destroy(e)
    st.close()
    print(json.dumps({"probe": "l2_window_copies", "work_groups": wgs, "copies_per_batch": 8, **res}), flush=True)


def copy_probe(hy, mib, steps):
    """A plain device copy of `mib` MiB, `steps` times: the yardstick whose FETCH_SIZE
    and WRITE_SIZE per dispatch must each read `mib` MiB."""
    n = mib << 20
    a, b = hy.Buf(n, np.uint8), hy.Buf(n, np.uint8)
    hy.check(hy.lib().hy_memset(a.ptr, 1, n))
    ev0, ev1 = hy.C.c_void_p(), hy.C.c_void_p()
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev0)))
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev1)))
    hy.check(hy.lib().hy_copy_d2d(b.ptr, a.ptr, n, None))
    hy.sync()
    hy.check(hy.lib().hy_event_record(ev0, None))
    for _ in range(steps):
        hy.check(hy.lib().hy_copy_d2d(b.ptr, a.ptr, n, None))
    hy.check(hy.lib().hy_event_record(ev1, None))
    hy.sync()
    ms = hy.C.c_float()
    hy.check(hy.lib().hy_event_elapsed_ms(ev0, ev1, hy.C.byref(ms)))
    t = ms.value / steps / 1e3
    print(json.dumps({"probe": "copy_d2d", "bytes": n, "steps": steps, "ms_per_copy": t * 1e3,
                      "GBps_read_plus_write": 2 * n / t / 1e9}), flush=True)


def gguf_load(hy, wtype, path, seed=42):
    """Write one real-shape layer (H=4096, I=3072, 64 + 1 experts) as a GGUF file with
    the reference converter's tensor names, then time hy_gguf_open + the upload into
    the resident tables (page-cache reads, host->device copies, on-device repack)."""
    import hy_oracle as O
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gguf_io as G
    layer = O.synth_layer(H, I, E, K, wtype, seed=seed, std=0.02)
    blob_ts = G.layer_tensors(layer, 0)
    with open(path, "wb") as f:
        f.write(G.gguf_bytes(G.layer_meta(layer), blob_ts))
    size = os.path.getsize(path)
    m = hy.Moe(H, I, E, K, wtype, num_layers=1, max_tokens=8)
    t0 = time.perf_counter()
    g = hy.Gguf(path)
    m.upload_gguf(0, g, 0)
    hy.sync()
    dt = time.perf_counter() - t0
    # one forward checked against the oracle on the loaded weights
    x = O.synth(seed + 1, 0, O.T_X, 0, (2, H), 1.0)
    same = bool(np.array_equal(m.run(0, x).view(np.uint32), O.moe_forward_q(layer, x).view(np.uint32)))
    g.close()
    m.close()
    os.remove(path)
    print(json.dumps({"probe": "gguf_load", "weights": {0: "F32", 2: "Q4_0", 8: "Q8_0"}[wtype], "file_bytes": size,
                      "seconds": dt, "GBps": size / dt / 1e9, "forward_bit_exact": same}), flush=True)


def attn_flops(kname, T):
    """Algorithmic FLOPs of one attention kernel launch at T tokens (causal)."""
    Hh, nh, nkv, hd = ATTN["H"], ATTN["nh"], ATTN["nkv"], ATTN["hd"]
    if kname == "qkv_proj":
        return 2.0 * T * (nh + 2 * nkv) * hd * Hh
    if kname == "o_proj":
        return 2.0 * T * Hh * nh * hd
    if kname == "attention":
        return 4.0 * hd * nh * T * (T + 1) / 2      # QK^T and PV over the causal triangle
    return 0.0


def attn_decode_bytes(kname, T, L):
    """Algorithmic HBM bytes of one launch of the cached (decode) attention at T new
    tokens against L cached positions: the weights each projection streams, the keys
    and values the attention reads, q / k / v / out rows."""
    Hh, nh, nkv, hd = ATTN["H"], ATTN["nh"], ATTN["nkv"], ATTN["hd"]
    nqkv = (nh + 2 * nkv) * hd
    if kname == "qkv_proj":
        return 4.0 * (nqkv * Hh + T * Hh + T * nqkv)
    if kname == "o_proj":
        return 4.0 * (Hh * nh * hd + T * nh * hd + 2 * T * Hh)
    if kname == "attention":
        return 4.0 * (2 * (L + T) * nkv * hd + 2 * T * nh * hd)
    if kname == "rope_qknorm":
        return 4.0 * 2 * T * nqkv
    return 0.0


def attn_decode_main(a, hy):
    """The KV-cache branch at decode: T new tokens (default 1) against a cache of
    a.cache positions, fp32, weights N(0, 0.02) resident.  Each timed step appends its
    T tokens, so the cache grows by T per step (50 steps: +1 % at 4096)."""
    import hy_oracle_attn as A
    T, L = a.tokens or 1, a.cache
    steps_all = a.warmup + 2 * a.steps
    w = A.synth_weights(ATTN["H"], ATTN["nh"], ATTN["nkv"], ATTN["hd"], seed=a.seed, std=0.02)
    m = hy.Attn(ATTN["H"], ATTN["nh"], ATTN["nkv"], ATTN["hd"], max(T, min(L, 4096)),
                max_cache=L + T * steps_all)
    m.upload(w.qkv_w, w.o_w, w.q_norm, w.k_norm)
    st = hy.Stream()
    rng = np.random.default_rng(a.seed)
    chunk = min(L, 4096)
    xf = hy.Buf.from_array(rng.standard_normal((chunk, ATTN["H"])).astype(np.float32))
    of = hy.Buf.empty((chunk, ATTN["H"]))
    filled = 0
    while filled < L:  # fill the cache in prompt chunks
        n = min(chunk, L - filled)
        m.forward_cached(xf, n, of, stream=st.h)
        filled += n
    x = hy.Buf.from_array(rng.standard_normal((T, ATTN["H"])).astype(np.float32))
    out = hy.Buf.empty((T, ATTN["H"]))
    for _ in range(a.warmup):
        m.forward_cached(x, T, out, stream=st.h)
    st.synchronize()
    ev0, ev1 = hy.C.c_void_p(), hy.C.c_void_p()
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev0)))
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev1)))
    L0 = m.cache_len()
    t0 = time.perf_counter()
    hy.check(hy.lib().hy_event_record(ev0, st.h))
    for _ in range(a.steps):
        m.forward_cached(x, T, out, stream=st.h)
    hy.check(hy.lib().hy_event_record(ev1, st.h))
    st.synchronize()
    wall = time.perf_counter() - t0
    ms = hy.C.c_float()
    hy.check(hy.lib().hy_event_elapsed_ms(ev0, ev1, hy.C.byref(ms)))
    ms_per_step = ms.value / a.steps
    Lmid = L0 + T * a.steps // 2  # mean cache length over the timed steps
    m.prof_enable(True)
    for _ in range(a.steps):
        m.forward_cached(x, T, out, stream=st.h)
    st.synchronize()
    prof = {k: v for k, v in m.prof_read().items() if v[0] > 0}
    m.prof_enable(False)
    Lp = L0 + T * a.steps + T * a.steps // 2
    dom = max(prof, key=lambda k: prof[k][1])
    avg_s = prof[dom][1] / prof[dom][0] / 1e3
    by = attn_decode_bytes(dom, T, Lp)
    workload = f"attention_decode_f32_t{T}_cache{L}"
    traffic = measured_traffic(workload, dom)
    if traffic is not None and dom == "attention":  # the decode kernel and its merge
        merge = measured_traffic(workload, "attention (merge)")
        traffic = traffic + merge if merge is not None else None
    res = {
        "metric": "attention decode tokens/sec (fp32 KV cache), 1 MI355X", "value": T / (ms_per_step / 1e3),
        "unit": "tokens/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": workload, "hidden": ATTN["H"], "heads": ATTN["nh"],
                   "kv_heads": ATTN["nkv"], "head_dim": ATTN["hd"], "tokens": T, "cache_len_mean": Lmid},
        "step_hbm_gbs": sum(attn_decode_bytes(k, T, Lmid) for k in prof) / (ms_per_step / 1e3) / 1e9,
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": by / avg_s / 1e9, "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": by / avg_s / PEAK_HBM, "traffic": traffic,
                     "algorithmic_bytes_per_launch": by, "avg_launch_ms": avg_s * 1e3},
        "kernels_ms": {k: round(t / n, 5) for k, (n, t) in prof.items()},
        "wall_s": wall,
    }
    if not a.no_cpu:
        res["cpu_baseline"] = attn_decode_cpu_baseline(w, L, T)
    print(json.dumps(res), flush=True)
    m.close()


def attn_cpu_baseline(w, T_sample=192):
    """attention_forward_cpu restated (the oracle, one thread, the reference's scalar
    fp32 loops) on a T_sample-token sequence of the same shape."""
    import hy_oracle_attn as A
    x = np.random.default_rng(7).standard_normal((T_sample, ATTN["H"])).astype(np.float32)
    t0 = time.perf_counter()
    A.attention_forward(w, x)
    dt = time.perf_counter() - t0
    return {"value": T_sample / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"one {T_sample}-token causal sequence through the oracle's attention_forward_cpu "
                      f"restatement (scalar fp32, 1 thread), {dt:.1f} s"}


def attn_decode_cpu_baseline(w, L, T, n_steps=150):
    """The KV-cache branch restated (the oracle, one thread): n_steps calls of T new
    tokens against a cache of L positions.  The cache rows are filled with N(0, 1)
    values directly, since prefilling L positions through the oracle would take
    minutes; the work per decode call (projections, attention over the whole cache,
    o_proj) is the same."""
    import hy_oracle_attn as A
    rng = np.random.default_rng(7)
    cache = A.KVCache(ATTN["nkv"], ATTN["hd"], max_len=L + T * n_steps)
    cache.k[:, :L] = rng.standard_normal((ATTN["nkv"], L, ATTN["hd"])).astype(np.float32)
    cache.v[:, :L] = rng.standard_normal((ATTN["nkv"], L, ATTN["hd"])).astype(np.float32)
    cache.c.cur_len = L
    x = rng.standard_normal((T, ATTN["H"])).astype(np.float32)
    t0 = time.perf_counter()
    for _ in range(n_steps):
        A.attention_cached(w, x, cache)
    dt = time.perf_counter() - t0
    return {"value": n_steps * T / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{n_steps} calls of {T} new token(s) against {L} cached positions (random cache rows) "
                      f"through the oracle's KV-cache branch (scalar fp32, 1 thread), {dt:.1f} s"}


def attn_main(a, hy):
    """Attention half of a decoder layer: x [T][4096] -> QKV projection -> RoPE ->
    QK-norm -> causal GQA attention -> o_proj, fp32, weights N(0, 0.02) resident."""
    import hy_oracle_attn as A
    T = a.tokens or 4096
    w = A.synth_weights(ATTN["H"], ATTN["nh"], ATTN["nkv"], ATTN["hd"], seed=a.seed, std=0.02)
    m = hy.Attn(ATTN["H"], ATTN["nh"], ATTN["nkv"], ATTN["hd"], T)
    m.upload(w.qkv_w, w.o_w, w.q_norm, w.k_norm)
    x = hy.Buf.from_array(np.random.default_rng(a.seed).standard_normal((T, ATTN["H"])).astype(np.float32))
    out = hy.Buf.empty((T, ATTN["H"]))
    st = hy.Stream()
    for _ in range(a.warmup):
        m.forward(x, T, out, stream=st.h)
    hy.sync()
    ev0, ev1 = hy.C.c_void_p(), hy.C.c_void_p()
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev0)))
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev1)))
    t0 = time.perf_counter()
    hy.check(hy.lib().hy_event_record(ev0, st.h))
    for _ in range(a.steps):
        m.forward(x, T, out, stream=st.h)
    hy.check(hy.lib().hy_event_record(ev1, st.h))
    hy.sync()
    wall = time.perf_counter() - t0
    ms = hy.C.c_float()
    hy.check(hy.lib().hy_event_elapsed_ms(ev0, ev1, hy.C.byref(ms)))
    ms_per_step = ms.value / a.steps
    m.prof_enable(True)
    for _ in range(a.steps):
        m.forward(x, T, out, stream=st.h)
    hy.sync()
    prof = {k: v for k, v in m.prof_read().items() if v[0] > 0}
    m.prof_enable(False)
    dom = max(prof, key=lambda k: prof[k][1])
    avg_s = prof[dom][1] / prof[dom][0] / 1e3
    fl = attn_flops(dom, T)
    total = sum(attn_flops(k, T) for k in prof)
    res = {
        "metric": "attention tokens/sec (fp32, causal GQA), 1 MI355X", "value": T / (ms_per_step / 1e3),
        "unit": "tokens/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"attention_f32_t{T}", "hidden": ATTN["H"], "heads": ATTN["nh"],
                   "kv_heads": ATTN["nkv"], "head_dim": ATTN["hd"], "tokens": T, "causal": True},
        "step_tflops": total / (ms_per_step / 1e3) / 1e12,
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": fl / avg_s / 1e12, "peak": PEAK_FP32_MFMA / 1e12,
                     "unit": "TFLOP/s", "frac": fl / avg_s / PEAK_FP32_MFMA, "traffic": None,
                     "algorithmic_flops_per_launch": fl, "avg_launch_ms": avg_s * 1e3},
        "kernels_ms": {k: round(t / n, 5) for k, (n, t) in prof.items()},
        "wall_s": wall,
    }
    if not a.no_cpu:
        res["cpu_baseline"] = attn_cpu_baseline(w)
    print(json.dumps(res), flush=True)
    m.close()


VOCAB = 133120


def model_main(a, hy):
    """The resident backbone (HunyuanFullModel::forward): token ids -> embedding ->
    32 decoder layers (fp32 attention + Q8_0 MoE) -> final norm -> lm_head logits,
    every weight synthetic and resident (~94 GB)."""
    T = a.tokens or 512
    nl = 32
    m = hy.Model(H, I, E, K, 8, ATTN["nh"], ATTN["nkv"], ATTN["hd"], VOCAB, nl, T)
    t0 = time.perf_counter()
    m.synth_globals(seed=a.seed, std=0.02)
    for l in range(nl):
        m.attn.synth(l, seed=a.seed, std=0.02)
        m.moe.synth(l, seed=a.seed, std=0.02)
        if l % 8 == 7:
            print(f"backbone: {l + 1}/{nl} layers synthesized", file=sys.stderr, flush=True)
    setup_s = time.perf_counter() - t0
    ids = hy.Buf.from_array(np.random.default_rng(a.seed).integers(0, VOCAB, size=T).astype(np.int32))
    logits = hy.Buf.empty((T, VOCAB))
    st = hy.Stream()
    for _ in range(a.warmup):
        m.forward(ids, T, logits, stream=st.h)
    hy.sync()
    ev0, ev1 = hy.C.c_void_p(), hy.C.c_void_p()
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev0)))
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev1)))
    t1 = time.perf_counter()
    hy.check(hy.lib().hy_event_record(ev0, st.h))
    for _ in range(a.steps):
        m.forward(ids, T, logits, stream=st.h)
    hy.check(hy.lib().hy_event_record(ev1, st.h))
    hy.sync()
    wall = time.perf_counter() - t1
    ms = hy.C.c_float()
    hy.check(hy.lib().hy_event_elapsed_ms(ev0, ev1, hy.C.byref(ms)))
    ms_per_step = ms.value / a.steps
    # per-kernel times of the two layer contexts (profiled pass)
    m.moe.prof_enable(True)
    m.attn.prof_enable(True)
    m.forward(ids, T, logits, stream=st.h)
    hy.sync()
    prof = {k: v for k, v in {**m.moe.prof_read(), **m.attn.prof_read()}.items() if v[0] > 0}
    m.moe.prof_enable(False)
    m.attn.prof_enable(False)
    dom = max(prof, key=lambda k: prof[k][1])
    n_l, t_l = prof[dom]
    avg_s = t_l / n_l / 1e3
    if dom in ("qkv_proj", "o_proj", "attention"):
        fl = attn_flops(dom, T)
        roof = {"bound": "mfma", "kernel": dom, "achieved": fl / avg_s / 1e12, "peak": PEAK_FP32_MFMA / 1e12,
                "unit": "TFLOP/s", "frac": fl / avg_s / PEAK_FP32_MFMA, "traffic": None, "avg_launch_ms": avg_s * 1e3}
    else:
        tr = kernel_traffic(dom, 8, T, E)
        roof = {"bound": "hbm", "kernel": dom, "achieved": tr / avg_s / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                "frac": tr / avg_s / PEAK_HBM, "traffic": None, "avg_launch_ms": avg_s * 1e3}
    per_forward = {k: round(t, 4) for k, (n, t) in prof.items()}
    res = {
        "metric": "backbone tokens/sec (HunyuanFullModel forward, 32 layers + lm_head), 1 MI355X",
        "value": T / (ms_per_step / 1e3), "unit": "tokens/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": ms_per_step, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 attention / int8 MoE", "data": "synthetic",
        "config": {"workload": f"backbone32_q8_0_t{T}", "hidden": H, "layers": nl, "vocab": VOCAB, "tokens": T,
                   "moe_weights": "Q8_0", "attention_weights": "F32"},
        "roofline": roof,
        "kernel_ms_per_forward": per_forward,
        "lm_head_and_rest_ms": ms_per_step - sum(t for _, t in prof.values()),
        "setup_s": setup_s, "wall_s": wall,
    }
    print(json.dumps(res), flush=True)
    m.close()


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def ref_cpu_baseline(wl, seed, budget_s=10.0):
    """The reference's own arithmetic: moe_forward_full restated operation for operation
    (scalar fp32, one thread, one sequential accumulator per dot product,
    src/hunyuan_moe_full.cpp:405-516), on layer 0's weights dequantized to F32 as the
    reference's loader does (src/hunyuan_gguf_loader.cpp:212-216), over a token sample."""
    import ctypes as C
    import hy_oracle as O
    wtype, T = wl["wtype"], wl["T"]
    layer = O.synth_layer(H, I, E, K, wtype, seed=seed, layer=0, std=0.02)

    def f32(q, rows, cols):
        return q if wtype == 0 else O.dequantize(q, wtype, cols).reshape(rows, cols)

    gu = np.empty((E, 2 * I, H), np.float32)
    dn = np.empty((E, H, I), np.float32)
    for e in range(E):
        gu[e] = f32(layer.gu[e], 2 * I, H)
        dn[e] = f32(layer.dn[e], H, I)
    sgu, sdn = f32(layer.shared_gu, 2 * I, H), f32(layer.shared_dn, H, I)
    router = layer.router
    del layer
    x = O.synth(seed + 1000, 0, O.T_X, 0, (min(T, 64), H), 1.0)
    cfg = O.default_cfg(E, K)

    def run(n):
        out = np.empty((n, H), np.float32)
        t0 = time.perf_counter()
        rc = O.lib().hyo_moe_forward_full(O.fp(x[:n].copy()), n, H, O.fp(router), O.fp(sgu), O.fp(sdn),
                                          O.fp(gu), O.fp(dn), E, I, C.byref(cfg), O.fp(out))
        assert rc == 0
        return time.perf_counter() - t0

    dt = run(1)
    n = int(max(1, min(16, min(T, 64), budget_s / max(dt, 1e-3))))
    if n > 1:
        dt = run(n)
    per_layer = n / dt
    nl = wl["layers"]
    return {"value": per_layer / nl, "unit": "tokens/s", "cores": 1, "kind": "port",
            "extrapolated": T > n or nl > 1,
            "sample": f"{n} of the {T} tokens through one layer of reference arithmetic (moe_forward_full "
                      f"restated: scalar fp32, 1 thread, weights dequantized to F32), {dt:.1f} s"
                      + (f"; the per-layer rate divided by {nl} layers" if nl > 1 else "")}


def cpu_baseline(wl, seed, budget_s=15.0):
    """The oracle's q-semantics layer (the int8 block dots of ggml's CPU vec_dot, OpenMP
    over all host threads; ggml itself is not in the reference tree) on a bounded token
    sample of the same workload, plus the reference-arithmetic leg."""
    import hy_oracle as O
    nthreads = os.cpu_count() or 1
    wtype = wl["wtype"]
    layer = O.synth_layer(H, I, E, K, wtype, seed=seed, layer=0, std=0.02)
    T = wl["T"]
    x = O.synth(seed + 1000, 0, O.T_X, 0, (T, H), 1.0)
    n = min(T, max(8, nthreads))
    rows = np.arange(n) % T
    t0 = time.perf_counter()
    O.moe_forward_q_rows(layer, x, rows, nthreads=nthreads)
    dt = time.perf_counter() - t0
    n2 = int(min(T * 4, max(n, n * budget_s / max(dt, 1e-6))))
    rows = np.arange(n2) % T
    t0 = time.perf_counter()
    O.moe_forward_q_rows(layer, x, rows, nthreads=nthreads)
    dt = time.perf_counter() - t0
    del layer
    nl = wl["layers"]
    res = {"value": n2 / dt / nl, "unit": "tokens/s", "cores": nthreads, "kind": "port",
           "extrapolated": nl > 1 or n2 < T, "cpu_model": cpu_model(),
           "sample": f"{n2} tokens of the {wl['name']} workload through one layer of the oracle's int8 "
                     f"(ggml-semantics) path, {nthreads} OpenMP threads, {dt:.1f} s"
                     + (f"; the per-layer rate divided by {nl} layers" if nl > 1 else "")}
    if wtype != 0:
        res["reference_arithmetic"] = ref_cpu_baseline(wl, seed)
    return res


def run_moe(hy, wl, steps, warmup, seed, graph=False, tokens=None, mix_ceiling=None):
    """Times `steps` steps of one MoE workload (after `warmup`) and profiles the
    kernels in a second pass; returns the result fields of its JSON line."""
    wl = dict(wl)
    if tokens:
        wl["T"] = tokens
    T, wtype, nl = wl["T"], wl["wtype"], wl["layers"]
    rot = wl["rot"] if not wl.get("stack") else 1
    n_layers = nl * rot
    bias = zipf_bias(seed) if wl.get("zipf") else None

    m = hy.Moe(H, I, E, K, wtype, num_layers=n_layers, max_tokens=T)
    for l in range(n_layers):
        m.synth(l, seed=seed, std=0.02, router_bias=bias)
    x = hy.Buf.empty((T, H))
    hy.check(hy.lib().hy_synth_fill(x.ptr, T * H, seed + 1000, 0, 0, 0, 1.0, None))
    if bias is not None:   # feature 0 carries the per-expert bias
        xh = x.numpy()
        xh[:, 0] = 1.0
        x = hy.Buf.from_array(xh)
    out = hy.Buf.empty((T, H))
    st = hy.Stream()
    stream = st.h

    def eager_step(i):
        if wl.get("stack"):
            m.stack_forward(0, nl, x, T, 1e-5, out, stream)
        else:
            m.forward(i % rot, x, T, out, stream)

    for i in range(warmup):
        eager_step(i)
    hy.sync()
    # kernels are launched from the host on a created stream (measured faster than the
    # null stream); --graph replays the layer forward captured once per resident weight
    # set instead (hipGraph; on this stack no faster than the eager launches)
    graphs = [hy.Graph(st, lambda l=l: eager_step(l)) for l in range(rot)] if graph else []

    def step(i):
        if graphs:
            graphs[i % rot].launch()
        else:
            eager_step(i)

    for i in range(warmup):
        step(i)
    hy.sync()
    ev0, ev1 = hy.C.c_void_p(), hy.C.c_void_p()
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev0)))
    hy.check(hy.lib().hy_event_create(hy.C.byref(ev1)))
    hy.sync()
    t0 = time.perf_counter()
    hy.check(hy.lib().hy_event_record(ev0, stream))
    for i in range(steps):
        step(i)
    hy.check(hy.lib().hy_event_record(ev1, stream))
    hy.sync()
    wall = time.perf_counter() - t0
    ms = hy.C.c_float()
    hy.check(hy.lib().hy_event_elapsed_ms(ev0, ev1, hy.C.byref(ms)))
    ms_per_step = ms.value / steps
    tokens_per_s = T / (ms_per_step / 1e3)

    D, counts = m.last_routing()
    # per-kernel durations on the launch stream (separate, profiled pass, eager launches)
    m.prof_enable(True)
    for i in range(steps):
        eager_step(i)
    hy.sync()
    prof = m.prof_read()
    m.prof_enable(False)
    kern = {k: (n, t) for k, (n, t) in prof.items() if n > 0}
    dom = max(kern, key=lambda k: kern[k][1])
    n_l, t_l = kern[dom]
    avg_s = t_l / n_l / 1e3
    n_layer_launch = nl if wl.get("stack") else 1
    traffic = kernel_traffic(dom, wtype, T, D)
    hbm_measured = measured_traffic(wl["name"] if not tokens else f"{wl['name']}_t{T}", dom)
    ops = kernel_ops(dom, T)
    layer_bytes = (D + 1) * expert_bytes(wtype) + E * H * 4 + 2 * T * H * 4
    layer_ops = 2.0 * T * (K + 1) * PARAMS_PER_EXPERT
    t_layer = ms_per_step / 1e3 / n_layer_launch
    # bound: HBM when the layer's bytes take longer at peak than its ops at int8 peak
    bound = "hbm" if layer_bytes / PEAK_HBM >= layer_ops / PEAK_INT8 else "mfma"
    if bound == "hbm":
        roof = {"bound": "hbm", "kernel": dom, "achieved": traffic / avg_s / 1e9, "peak": PEAK_HBM / 1e9,
                "unit": "GB/s", "frac": traffic / avg_s / PEAK_HBM, "traffic": hbm_measured,
                "algorithmic_bytes_per_launch": traffic, "avg_launch_ms": avg_s * 1e3}
    else:
        roof = {"bound": "mfma", "kernel": dom, "achieved": ops / avg_s / 1e12, "peak": PEAK_INT8 / 1e12,
                "unit": "TFLOP/s", "frac": ops / avg_s / PEAK_INT8, "traffic": hbm_measured,
                "algorithmic_ops_per_launch": ops, "avg_launch_ms": avg_s * 1e3}
        if mix_ceiling:
            roof["rescale_ceiling"] = {"peak": mix_ceiling / 1e12, "unit": "TOP/s",
                                       "frac": ops / avg_s / mix_ceiling,
                                       "source": "hyp_block_mix, the per-block mix alone, same run"}
    top8 = float(np.sort(counts)[::-1][:8].sum() / max(1, counts.sum()))
    res = {
        "value": tokens_per_s, "ms_per_step": ms_per_step,
        "config": {"workload": wl["name"], "hidden": H, "intermediate": I, "experts": E, "shared_experts": 1,
                   "topk": K, "tokens": T, "weights": {0: "F32", 2: "Q4_0", 8: "Q8_0"}[wtype],
                   "layers": nl, "resident_weight_sets": n_layers, "distinct_experts_last_step": int(D)},
        "layer_hbm_gbps": layer_bytes / t_layer / 1e9,
        "layer_hbm_frac": layer_bytes / t_layer / PEAK_HBM,
        "layer_int8_util": layer_ops / t_layer / PEAK_INT8,
        "roofline": roof,
        "kernels_ms": {k: round(t / n, 5) for k, (n, t) in kern.items()},
        "launch": "hip_graph" if graph else "eager",
        "wall_s": wall,
    }
    if wl.get("zipf"):
        res["routing"] = {"zipf_s": 1.1, "zipf_beta": ZIPF_BETA, "top8_pair_share": top8,
                          "hottest_expert_tokens": int(counts.max()), "pairs_per_expert_sorted":
                          [int(c) for c in np.sort(counts)[::-1]]}
    for g in graphs:
        g.close()
    st.close()
    m.close()
    return res


# extra workloads timed after the headline in the same run, so that every configuration
# has a number in the one JSON line: the decode batches, the skewed image-token layer,
# the T=512 prefill layer and the F32 layer (name, workload, tokens, steps multiplier)
EXTRAS = (("decode_t1", "c3", 1, 10), ("decode_t2", "c3", 2, 10), ("decode_t4", "c3", 4, 10),
          ("decode_t8", "c3", 8, 10), ("zipf_t4096", "c4", None, 1), ("prefill_t512", "c2", None, 5),
          ("f32_t16", "c1", None, 5))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c5", choices=sorted(WORKLOADS))
    ap.add_argument("--tokens", type=int, default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="time only the --config workload")
    ap.add_argument("--graph", action="store_true", help="replay the step as a captured hipGraph")
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB")
    ap.add_argument("--stream-probe", type=int, default=0, metavar="WAVES",
                    help="HBM read rate of WAVES single-wave 144 KB streams (864: the decode T=1 gate/up shape)")
    ap.add_argument("--l2-probe", action="store_true",
                    help="global->LDS copy rate of 1 KB copies from 1 MiB / 64 MiB / 1 GiB windows")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="rate of the grouped GEMM's per-block instruction mix alone (and of its halves)")
    ap.add_argument("--attn", action="store_true", help="time the attention half instead of the MoE layer")
    ap.add_argument("--cache", type=int, default=0, metavar="L",
                    help="with --attn: decode T (--tokens, default 1) new tokens against L cached positions")
    ap.add_argument("--model", action="store_true", help="time the resident 32-layer backbone with lm_head")
    ap.add_argument("--gguf-load", default=None, metavar="PATH",
                    help="time loading one real-shape layer from a GGUF file written at PATH")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {a.gpus}): this build has no multi-GPU path; "
              f"expert-parallel sharding is a design note, not code.", file=sys.stderr)
        sys.exit(2)

    hy = load_pkg()
    if hy.device_count() < 1:
        sys.exit("no HIP device visible")
    if a.copy_probe:
        copy_probe(hy, a.copy_probe, a.steps)
        return
    if a.gguf_load:
        gguf_load(hy, WORKLOADS[a.config]["wtype"], a.gguf_load, a.seed)
        return
    if a.attn:
        (attn_decode_main if a.cache else attn_main)(a, hy)
        return
    if a.model:
        model_main(a, hy)
        return
    if a.stream_probe:
        stream_probe(hy, waves=a.stream_probe)
        return
    if a.l2_probe:
        l2_probe(hy)
        return
    if a.mfma_probe:
        rates = {name: probe_block_mix(hy, v) for v, name in ((0, "mix"), (1, "mfma_only"), (2, "valu_only"),
                                                           (3, "f16_block_dots"),
                                                           (4, "f16_block_dots_a_unpacked"))}
        print(json.dumps({"probe": "block_mix", "work_groups": PROBE_WGS, "iters_per_wave": PROBE_ITERS,
                          "block_dot_ops_per_s": rates, "frac_of_dense_int8": rates["mix"] / PEAK_INT8}),
              flush=True)
        return
    wl = WORKLOADS[a.config]
    mix = probe_block_mix(hy) if wl["wtype"] != 0 and wl["T"] > 16 else None
    r = run_moe(hy, wl, a.steps, a.warmup, a.seed, graph=a.graph, tokens=a.tokens, mix_ceiling=mix)
    print(f"bench: {r['config']['workload']} {r['ms_per_step']:.3f} ms/step", file=sys.stderr, flush=True)
    res = {"metric": "MoE-layer tokens/sec + achieved HBM GB/s / int8 MFMA util, 1 MI355X",
           "value": r.pop("value"), "unit": "tokens/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
           "ms_per_step": r.pop("ms_per_step"), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8" if wl["wtype"] != 0 else "f32", "data": "synthetic"}
    res.update(r)
    if not a.no_extras and a.config == "c5" and not a.tokens:
        extras = {}
        for name, cfg, toks, mult in EXTRAS:
            e = run_moe(hy, WORKLOADS[cfg], a.steps * mult, a.warmup, a.seed, graph=a.graph, tokens=toks,
                        mix_ceiling=mix)
            print(f"bench: {name} {e['ms_per_step']:.4f} ms/step", file=sys.stderr, flush=True)
            extras[name] = {"workload": e["config"]["workload"], "tokens": e["config"]["tokens"],
                            "value": e["value"], "unit": "tokens/s", "ms_per_step": e["ms_per_step"],
                            "steps": a.steps * mult, "layer_hbm_frac": e["layer_hbm_frac"],
                            "layer_int8_util": e["layer_int8_util"], "roofline": e["roofline"],
                            "kernels_ms": e["kernels_ms"],
                            "distinct_experts_last_step": e["config"]["distinct_experts_last_step"]}
            if "routing" in e:
                extras[name]["routing"] = e["routing"]
        res["extras"] = extras
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(wl if not a.tokens else dict(wl, T=a.tokens), a.seed)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
