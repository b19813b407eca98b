"""Index agreement between the reference's router arithmetic and the q semantics, on
the benchmark workloads' own inputs (hidden 4096, 64 experts, top-8, router weights
N(0, 0.02) seeded by layer index, activations N(0, 1) from seed 1042).

For every token both selections are computed (tests/index_agreement.py): the
reference's sequential logits + softmax + top-k on probabilities (bit-exact against
the reference build), and the GPU's blocked logits + top-k on logits.  Every logit
must lie within the rounding bound of the other method's, and every token whose
selected set or order differs must have its disagreeing experts within the bound of
each other.  The counts are printed (pytest -s).

The 32-layer stack's layers past the first take the GPU's own activations as input:
tests/test_gpu_index_agreement.py.
"""
import numpy as np
import pytest

import bench
import hy_oracle as O
from index_agreement import compare, rms_norm_blocked, rms_norm_seq

H, E, K, SEED = 4096, 64, 8, 42


def router(layer, bias=None):
    wr = O.synth(SEED, layer, O.T_ROUTER, 0, (E, H), 0.02)
    if bias is not None:
        wr[:, 0] = bias
    return wr


def bench_x(T):
    return O.synth(SEED + 1000, 0, O.T_X, 0, (T, H), 1.0)


def report(name, r):
    print(f"\n{name}: {r}")
    assert r["max_logit_diff_over_uA"] < r["bound_coeff"]


@pytest.mark.parametrize("layer", [0, 1])
def test_q8_0_t512(layer):
    x = bench_x(512)
    report(f"Q8_0 T=512 layer {layer}", compare(x, x, router(layer), K))


def test_f32_t16():
    x = bench_x(16)
    report("F32 T=16", compare(x, x, router(0), K))


def test_decode_t8_every_weight_set():
    """The decode workload rotates over 8 resident layers (Infinity-Cache defeat)."""
    x = bench_x(8)
    for layer in range(8):
        r = compare(x, x, router(layer), K)
        report(f"decode T=8 layer {layer}", r)


def test_q4_0_t4096_zipf():
    x = bench_x(4096)
    x[:, 0] = 1.0
    report("Q4_0 T=4096 Zipf", compare(x, x, router(0, bench.zipf_bias(SEED)), K))


def test_stack_layer0_t4096():
    """Layer 0 of the stack: the router reads RMSNorm(x), the reference's sequential
    norm on one side and the blocked norm on the other."""
    x = bench_x(4096)
    report("stack T=4096 layer 0", compare(rms_norm_seq(x), rms_norm_blocked(x), router(0), K, with_norm=True))


def test_bound_is_tight_enough_to_fail():
    """The elementwise bound must reject plausible mistakes: the reference side reading
    the router with its rows shifted by one expert, or dropping the last 32-element
    block of every dot (a loop bound one block short)."""
    x = bench_x(64)
    wr = router(0)
    with pytest.raises(AssertionError, match="rounding bound"):
        compare_sides(x, wr, np.ascontiguousarray(np.roll(wr, 1, axis=0)))
    short = wr.copy()
    short[:, H - 32:] = 0.0
    with pytest.raises(AssertionError, match="rounding bound"):
        compare_sides(x, wr, short)


def compare_sides(x, wr_q, wr_ref):
    """compare()'s elementwise check with the two sides reading different routers."""
    import index_agreement as IA
    l_r = IA.logits_seq(x, wr_ref)
    l_q = IA.logits_blocked(x, wr_q)
    A = np.abs(x.astype(np.float64)) @ np.abs(wr_q.astype(np.float64)).T
    eps = IA.bound_coeff(H, False) * IA.U * A
    assert (np.abs(l_r.astype(np.float64) - l_q) <= eps).all(), "logit difference beyond the rounding bound"
