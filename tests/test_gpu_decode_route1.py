"""One-token batches whose routing runs inside the gate/up launch (T = 1, Q8_0 / Q4_0,
hidden sizes the ring GEMV takes): the logits launch computes the router logits and the
Q8_0 of x, each gate/up wave selects the top-k itself, and one wave writes every
routing product the down GEMV, the combine and the caller read.  Outputs, logits,
weights and indices must equal the oracle bit for bit; the dispatch lists must be the
ones the separate selection pass writes (gate statistics and T = 1 -> T > 1 -> T = 1
sequences through one work arena), and a captured graph must replay it."""
import numpy as np
import pytest

import hy_oracle as O
from test_gpu_parity import assert_exact

pytestmark = pytest.mark.gpu

H, I = 1024, 768   # 32 blocks per row: the ring GEMV (and so the one-token path) takes it


def _run_check(gpu, m, layer, x, what):
    out, lg, w, idx = m.run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
    np.testing.assert_array_equal(lg.view(np.uint32), rlg.view(np.uint32), err_msg=what)
    np.testing.assert_array_equal(idx, ridx, err_msg=what)
    np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32), err_msg=what)
    assert_exact(out, ref, what)
    # gate statistics: distinct experts and per-expert pair counts of this call
    d, counts = m.last_routing()
    ref_counts = np.bincount(ridx.ravel(), minlength=layer.E).astype(np.int32)
    np.testing.assert_array_equal(counts, ref_counts, err_msg=what)
    assert d == int((ref_counts > 0).sum()), what
    return out


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("E,K,shared,norm,scale", [(16, 4, True, True, 1.0), (64, 8, True, True, 1.0),
                                                    (16, 1, True, True, 2.5), (16, 1, False, False, 2.5),
                                                    (16, 16, False, True, 1.0), (64, 64, True, True, 1.0),
                                                    (32, 6, True, False, 0.75)])
def test_one_token_layer(gpu, wtype, E, K, shared, norm, scale):
    layer = O.synth_layer(H, I, E, K, wtype, seed=E * 7 + K, std=0.05, shared=shared)
    layer.norm_topk_prob, layer.routed_scaling_factor = norm, scale
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=16, has_shared=shared, norm_topk_prob=norm,
                routed_scaling_factor=scale)
    m.set_path(gpu.PATH_VALU)
    m.upload(0, layer)
    for seed in (3, 4):
        x = O.synth(100 + seed, 0, O.T_X, 0, (1, H), 1.0)
        _run_check(gpu, m, layer, x, f"T=1 wtype={wtype} E={E} K={K} shared={shared} norm={norm} seed={seed}")
    m.close()


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
def test_one_token_between_batches(gpu, wtype):
    """The one-token path and the selection pass write the same work arena: alternate
    them (and the grouped GEMM) so stale lists from either would show."""
    E, K = 16, 4
    layer = O.synth_layer(H, I, E, K, wtype, seed=91, std=0.05)
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=256)
    m.upload(0, layer)
    for i, T in enumerate((1, 7, 1, 200, 1, 2, 1)):
        x = O.synth(200 + i, 0, O.T_X, 0, (T, H), 1.0)
        _run_check(gpu, m, layer, x, f"sequence step {i} T={T} wtype={wtype}")
    m.close()


def test_one_token_graph_replay(gpu):
    """A captured one-token forward replays bit for bit what the eager call computes,
    with other work through the same arena between the replays."""
    E, K = 64, 8
    m = gpu.Moe(H, I, E, K, O.Q4_0, max_tokens=64)
    m.synth(0, seed=17, std=0.05)
    st = gpu.Stream()
    x = gpu.Buf.from_array(O.synth(300, 0, O.T_X, 0, (1, H), 1.0))
    out = gpu.Buf.empty((1, H))
    other_x, other_out = gpu.Buf.from_array(O.synth(301, 0, O.T_X, 0, (64, H), 1.0)), gpu.Buf.empty((64, H))
    g = gpu.Graph(st, lambda: m.forward(0, x, 1, out, st.h))
    try:
        for rep in range(3):
            m.forward(0, other_x, 64 if rep % 2 == 0 else 3, other_out, st.h)
            st.synchronize()
            g.launch()
            st.synchronize()
            got = out.numpy()
            ref = gpu.Buf.empty((1, H))
            m.forward(0, x, 1, ref, st.h)
            st.synchronize()
            np.testing.assert_array_equal(got.view(np.uint32), ref.numpy().view(np.uint32), err_msg=f"replay {rep}")
    finally:
        g.close()
        st.close()
        m.close()
