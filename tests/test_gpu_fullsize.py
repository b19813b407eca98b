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


@pytest.mark.parametrize("T", [1, 2, 4, 8])
def test_decode_q4_0_full_shape(gpu, full_layers, ctxs, T):
    """Bit-exact decode; T=1 runs the up GEMV with the 3-step ring (864 waves), T >= 2
    with the 2-step ring (more waves than the 3-step ring keeps resident)."""
    x = O.synth(100 + T, 0, O.T_X, 0, (T, H), 1.0)
    out, lg, w, idx = ctxs[O.Q4_0].run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(full_layers[O.Q4_0], x, debug=True, nthreads=16)
    np.testing.assert_array_equal(lg.view(np.uint32), rlg.view(np.uint32))
    np.testing.assert_array_equal(idx, ridx)
    assert_exact(out, ref, f"decode T={T}")


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
