"""bench.py's accounting on the CPU: the algorithmic byte and op counts behind
`roofline.achieved`, checked against independent facts (the byte sizes of the
oracle's own arrays, the published per-expert sizes of the workloads), and the
lookup of `roofline.traffic` in the committed counter table."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
import hy_oracle as O  # noqa: E402
import hy_oracle_attn as A  # noqa: E402


def test_moe_weight_bytes_match_published_expert_sizes():
    # bytes per expert: F32 150,994,944; Q8_0 40,108,032; Q4_0 21,233,664 (gate_up + down)
    for wt, per_expert in ((0, 150_994_944), (8, 40_108_032), (2, 21_233_664)):
        T, D = 1, 8
        up = bench.kernel_traffic("ffn_up", wt, T, D) - T * bench.H * (4.0 if wt == 0 else 1.25) \
            - (T * bench.K + T) * bench.I * (4.0 if wt == 0 else 1.25)
        down_w = bench.kernel_traffic("ffn_down", wt, T, D) - (T * bench.K + T) * bench.I * (4.0 if wt == 0 else 1.25) \
            - (T * bench.K + T) * bench.H * 4
        assert up + down_w == (D + 1) * per_expert


def test_moe_ops_are_two_per_mac():
    # T tokens x (K routed + 1 shared) experts x 37,748,736 parameters x 2
    T = 512
    assert bench.kernel_ops("ffn_up", T) + bench.kernel_ops("ffn_down", T) == 2.0 * T * 9 * 37_748_736


def test_decode_attention_bytes_match_cache_and_weight_arrays():
    a = bench.ATTN
    T, L = 1, 4096
    cache = A.KVCache(a["nkv"], a["hd"], max_len=L + T)
    kv = cache.k.nbytes + cache.v.nbytes          # every cached row plus the new one
    qo = 2 * T * a["nh"] * a["hd"] * 4            # q in, merged rows out
    assert bench.attn_decode_bytes("attention", T, L) == kv + qo
    w = A.synth_weights(256, a["nh"], a["nkv"], a["hd"], seed=0)   # hidden 256: same row count
    qkv_rows = w.qkv_w.shape[0]
    assert bench.attn_decode_bytes("qkv_proj", T, L) == 4.0 * (qkv_rows * a["H"] + T * a["H"] + T * qkv_rows)
    assert bench.attn_decode_bytes("o_proj", T, L) >= a["H"] * a["nh"] * a["hd"] * 4


def test_traffic_table_lookup():
    path = os.path.join(ROOT, "profiles", "hbm_traffic.md")
    got = bench.measured_traffic("moe_layer_q8_0_t512", "ffn_up", path)
    assert got is not None and got > 1.7e9            # at least the unique weights
    dec = bench.measured_traffic("attention_decode_f32_t1_cache4096", "attention", path)
    assert dec is not None and abs(dec - 33.6e6) / 33.6e6 < 0.1
    assert bench.measured_traffic("no_such_workload", "ffn_up", path) is None
    assert bench.measured_traffic("x", "y", path=os.path.join(ROOT, "no_such_file.md")) is None
    assert np.isfinite(got)


def zipf_routing_counts(T=4096, seed=42):
    """Pairs per expert of the skewed T=4096 workload, routed by the oracle's router
    (the GPU's logits order, so the GPU routes these inputs identically)."""
    x = O.synth(seed + 1000, 0, O.T_X, 0, (T, bench.H), 1.0)
    x[:, 0] = 1.0
    wr = O.synth(seed, 0, O.T_ROUTER, 0, (bench.E, bench.H), 0.02)
    wr[:, 0] = bench.zipf_bias(seed)
    _, idx = O.route_topk(O.router_logits_blocked(x, wr), bench.K)
    return np.bincount(idx.ravel(), minlength=bench.E)


def test_zipf_workload_is_calibrated():
    """The Zipf(1.1) bias puts 63 % of the pairs on the eight most popular experts (the
    top-8 mass of Zipf(1.1) over 64 experts) and one expert on nearly every token."""
    p = np.arange(1, 65, dtype=np.float64) ** -1.1
    assert abs(p[:8].sum() / p.sum() - 0.63) < 0.005
    cnt = np.sort(zipf_routing_counts())[::-1]
    assert cnt.sum() == 4096 * bench.K
    share8 = cnt[:8].sum() / cnt.sum()
    assert 0.625 <= share8 <= 0.635, share8
    assert cnt[0] > 3900 and cnt[-1] < 100
