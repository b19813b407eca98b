"""Index agreement with the reference's router arithmetic at every layer of the
32-layer Q8_0 stack (T=4096, the benchmark's inputs).

The stack runs on the GPU one layer at a time; layer l's input h_l (the GPU's own
activations, which test_gpu_workloads.py pins against the oracle) is copied back and
its routing computed both ways on the host: the reference's sequential RMSNorm,
sequential router dot, softmax and top-k on probabilities, against the blocked RMSNorm
and router and the top-k on logits that the GPU uses (tests/index_agreement.py states
the bound each disagreement must meet).  Layer 0 is also covered by the CPU test
test_index_agreement.py; the counts are printed (pytest -s).
"""
import numpy as np
import pytest

import hy_oracle as O
from index_agreement import compare, rms_norm_blocked, rms_norm_seq

pytestmark = pytest.mark.gpu

H, I, E, K, SEED, NL, T = 4096, 3072, 64, 8, 42, 32, 4096


@pytest.fixture(scope="module")
def layer_inputs(gpu):
    m = gpu.Moe(H, I, E, K, O.Q8_0, num_layers=NL, max_tokens=T)
    try:
        for l in range(NL):
            m.synth(l, seed=SEED, std=0.02)
        x = O.synth(SEED + 1000, 0, O.T_X, 0, (T, H), 1.0)
        bufs = [gpu.Buf.from_array(x), gpu.Buf.empty((T, H))]
        hs = [x]
        for l in range(NL - 1):
            m.stack_forward(l, 1, bufs[l % 2], T, 1e-5, bufs[(l + 1) % 2])
            hs.append(bufs[(l + 1) % 2].numpy())
        print(f"stack inputs of {NL} layers collected", flush=True)
        return hs
    finally:
        m.close()


@pytest.mark.parametrize("first", [0, 8, 16, 24])
def test_stack_layers(layer_inputs, first):
    tot = {"set_differs": 0, "order_differs": 0, "near_ties_8_9_64uA": 0, "selected_prob_ties_with_distinct_logits": 0,
           "boundary_prob_ties_with_distinct_logits": 0}
    for l in range(first, first + 8):
        h = layer_inputs[l]
        wr = O.synth(SEED, l, O.T_ROUTER, 0, (E, H), 0.02)
        r = compare(rms_norm_seq(h), rms_norm_blocked(h), wr, K, with_norm=True)
        print(f"stack T=4096 layer {l}: set_differs {r['set_differs']} {r['set_differs_tokens']} order_differs "
              f"{r['order_differs']} near_ties(64uA) {r['near_ties_8_9_64uA']} prob_ties "
              f"{r['selected_prob_ties_with_distinct_logits']}/{r['boundary_prob_ties_with_distinct_logits']} "
              f"min_gap {r['min_gap_8_9']:.3e} max|dl|/uA {r['max_logit_diff_over_uA']:.1f} "
              f"worst/bound {r['worst_disagreement_over_bound']:.2e}", flush=True)
        for k in tot:
            tot[k] += r[k]
    print(f"stack T=4096 layers {first}-{first + 7} total: {tot}", flush=True)
