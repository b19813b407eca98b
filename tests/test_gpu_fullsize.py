"""GPU parity at the real layer shape (hidden 4096, 64 + 1 experts of width 3072,
top-8).  Decode batches are compared whole; large batches on a sample of tokens
(each token's output depends only on its own row: no capacity or drops in the
default routing), which the oracle finishes in seconds."""
import numpy as np
import pytest

import hy_oracle as O
from test_gpu_parity import assert_exact

pytestmark = pytest.mark.gpu

H, I, E, K = 4096, 3072, 64, 8


@pytest.fixture(scope="module")
def full_layers():
    return {wt: O.synth_layer(H, I, E, K, wt, seed=42, std=0.02) for wt in (O.Q4_0, O.Q8_0)}


@pytest.fixture(scope="module")
def ctxs(gpu, full_layers):
    out = {}
    for wt, layer in full_layers.items():
        m = gpu.Moe(H, I, E, K, wt, max_tokens=4096)
        m.upload(0, layer)          # host GGUF blocks -> resident layout
        out[wt] = m
    yield out
    for m in out.values():
        m.close()


@pytest.mark.parametrize("wt,T", [(O.Q4_0, 1), (O.Q4_0, 2), (O.Q4_0, 3), (O.Q4_0, 4), (O.Q4_0, 6), (O.Q4_0, 8),
                                   (O.Q4_0, 16), (O.Q8_0, 2), (O.Q8_0, 4), (O.Q8_0, 8)])
def test_decode_full_shape(gpu, full_layers, ctxs, wt, T):
    """Bit-exact decode at every ring-step size the launcher picks from the launch's
    wave bound (row groups x tile bound; 64 + 1 experts, top-8, 4-token tiles).
    Q4_0: T=1 864 gate/up waves on 8-block steps (the one-token routed launch); T=2
    1,632 on 8-block steps; T=3 2,400 gate/up on 4-block steps, 1,600 down on 8; T=4
    3,168 / 2,112 on 4-block steps; T=6 4,800 gate/up on 2-block steps, 3,200 down on 4;
    T=8 6,336 / 4,224 on 2-block steps; T=16 8,064 gate/up on 8-block steps (more waves
    than any step size keeps resident), 5,376 down on 2-block steps.  Q8_0: T=2 1,632 /
    1,088 on 4-block steps; T=4 3,168 / 2,112 on 2-block steps; T=8 6,336 gate/up on
    8-block steps, 4,224 down on 2-block steps."""
    x = O.synth(100 + T, 0, O.T_X, 0, (T, H), 1.0)
    out, lg, w, idx = ctxs[wt].run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(full_layers[wt], x, debug=True, nthreads=16)
    np.testing.assert_array_equal(lg.view(np.uint32), rlg.view(np.uint32))
    np.testing.assert_array_equal(idx, ridx)
    assert_exact(out, ref, f"decode wt={wt} T={T}")


@pytest.mark.parametrize("wt,T", [(O.Q8_0, 512), (O.Q4_0, 4096), (O.Q8_0, 100)])
def test_prefill_full_shape_sampled(gpu, full_layers, ctxs, wt, T):
    x = O.synth(200 + T, 0, O.T_X, 0, (T, H), 1.0)
    out, lg, w, idx = ctxs[wt].run(0, x, debug=True)
    rows = np.unique(np.concatenate([[0, T - 1], np.random.default_rng(T).integers(0, T, 14)]))
    ref = O.moe_forward_q_rows(full_layers[wt], x, rows, nthreads=16)
    rlg = O.router_logits_blocked(x[rows], full_layers[wt].router)
    np.testing.assert_array_equal(lg[rows].view(np.uint32), rlg.view(np.uint32))
    _, ridx = O.route_topk(rlg, K)
    np.testing.assert_array_equal(idx[rows], ridx)
    assert_exact(out[rows], ref, f"prefill wt={wt} T={T}")


def test_device_generated_layer_matches_host(gpu, full_layers, ctxs):
    """The on-device generator reproduces the host layer: same outputs bit for bit."""
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=64)
    m.synth(0, seed=42, std=0.02)
    x = O.synth(300, 0, O.T_X, 0, (64, H), 1.0)
    a = m.run(0, x)
    b = ctxs[O.Q8_0].run(0, x)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    m.close()
