"""GPU parity at the limits the C ABI accepts: the largest batch (max_tokens = 16384),
large top-k (16, 32 and the bound 64, topk_f32's best[64]), top-k equal to the number of
experts, and a single expert.

Each token's output depends only on its own row (default routing: no capacity, no
drops), so the oracle runs on sampled rows and row-permutation invariance covers the
rest (every output element is computed in a fixed order whatever tile a token lands
in)."""
import numpy as np
import pytest

import hy_oracle as O
from test_gpu_parity import assert_exact
from test_gpu_workloads import assert_permutes, sample_rows

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
def test_layer_at_max_tokens_and_topk(gpu, wtype):
    """T = 16384 (the largest batch a context takes) at K = 16 over 64 experts: T*K =
    262,144 pairs, the most the dispatch scratch is sized for, all dispatched; the
    routing of every row and sampled output rows against the oracle, every row through
    permutation invariance.  (Larger K up to 64 is covered at smaller T below.)"""
    H, I, E, K, T = 256, 128, 64, 16, 16384
    layer = O.synth_layer(H, I, E, K, wtype, seed=71, std=0.05)
    x = O.synth(72, 0, O.T_X, 0, (T, H), 1.0)
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=T)
    m.upload(0, layer)
    out, lg, w, idx = m.run(0, x, debug=True)
    rows = sample_rows(T, n=40)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x[rows], debug=True)
    np.testing.assert_array_equal(lg[rows].view(np.uint32), rlg.view(np.uint32))
    np.testing.assert_array_equal(idx[rows], ridx)
    np.testing.assert_array_equal(w[rows].view(np.uint32), rw.view(np.uint32))
    assert_exact(out[rows], ref, f"T={T} K={K} wtype={wtype}")
    # every row selects 16 distinct experts; the dispatch placed all of them
    assert np.all(np.sort(idx, axis=1)[:, 1:] != np.sort(idx, axis=1)[:, :-1])
    D, counts = m.last_routing()
    assert counts.sum() == T * K and D == E
    assert_permutes(lambda v: m.run(0, v), x, f"T={T} K={K}")
    m.close()


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0, O.F32])
@pytest.mark.parametrize("T", [1, 5, 40])
def test_topk_equals_experts(gpu, wtype, T):
    """K = E: every token routes to every expert (decode GEMV for T <= 16, grouped GEMM
    above for the quantized types)."""
    H, I, E = 256, 128, 8
    layer = O.synth_layer(H, I, E, E, wtype, seed=80 + T, std=0.05)
    x = O.synth(81 + T, 0, O.T_X, 0, (T, H), 1.0)
    m = gpu.Moe(H, I, E, E, wtype, max_tokens=64)
    m.upload(0, layer)
    out, lg, w, idx = m.run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
    np.testing.assert_array_equal(idx, ridx)
    assert np.all(np.sort(idx, axis=1) == np.arange(E))
    assert_exact(out, ref, f"K=E={E} wtype={wtype} T={T}")
    m.close()


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("shared", [True, False])
def test_single_expert(gpu, wtype, shared):
    """E = 1, K = 1: routing is trivial (weight p * routed_scaling_factor, as the
    reference's K = 1 rule gives); with and without the shared expert."""
    H, I = 256, 128
    layer = O.synth_layer(H, I, 1, 1, wtype, seed=90, std=0.05, shared=shared)
    m = gpu.Moe(H, I, 1, 1, wtype, max_tokens=64, has_shared=shared)
    m.upload(0, layer)
    for T in (1, 3, 33):
        x = O.synth(91 + T, 0, O.T_X, 0, (T, H), 1.0)
        out, lg, w, idx = m.run(0, x, debug=True)
        ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
        assert np.all(idx == 0)
        np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
        assert_exact(out, ref, f"E=1 wtype={wtype} shared={shared} T={T}")
    m.close()


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0, O.F32])
def test_topk_64_every_expert(gpu, wtype):
    """K = E = 64, the top-k bound: the one-launch decode routing while T*K <= 256 (T = 1,
    4), the general routing above (T = 5), the grouped GEMM for batches (T = 100); the
    combine sums 64 pairs per token in four chunks."""
    H, I, E, K = 256, 128, 64, 64
    layer = O.synth_layer(H, I, E, K, wtype, seed=190, std=0.05)
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=100)
    m.upload(0, layer)
    for T in ((1, 4, 5) if wtype == O.F32 else (1, 4, 5, 100)):
        x = O.synth(191 + T, 0, O.T_X, 0, (T, H), 1.0)
        out, lg, w, idx = m.run(0, x, debug=True)
        ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
        np.testing.assert_array_equal(idx, ridx)
        np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
        assert np.all(np.sort(idx, axis=1) == np.arange(E))
        assert_exact(out, ref, f"K=E=64 wtype={wtype} T={T}")
    m.close()


def test_topk_32_large_batch(gpu):
    """K = 32 of 64 experts at T = 8192 (262,144 routed pairs): sampled rows against the
    oracle, every row through permutation invariance; the combine takes two chunks."""
    H, I, E, K, T = 256, 128, 64, 32, 8192
    layer = O.synth_layer(H, I, E, K, O.Q8_0, seed=200, std=0.05)
    x = O.synth(201, 0, O.T_X, 0, (T, H), 1.0)
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=T)
    m.upload(0, layer)
    out, lg, w, idx = m.run(0, x, debug=True)
    rows = sample_rows(T, n=24)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x[rows], debug=True)
    np.testing.assert_array_equal(idx[rows], ridx)
    np.testing.assert_array_equal(w[rows].view(np.uint32), rw.view(np.uint32))
    assert_exact(out[rows], ref, f"K={K} T={T}")
    D, counts = m.last_routing()
    assert counts.sum() == T * K
    assert_permutes(lambda v: m.run(0, v), x, f"K={K} T={T}")
    m.close()


def test_router_topk_64(gpu):
    """The stateless router and gating entry points at K = 64."""
    rng = np.random.default_rng(210)
    x = rng.standard_normal((9, 256)).astype(np.float32)
    wr = (rng.standard_normal((64, 256)) * 0.1).astype(np.float32)
    lg, w, idx = gpu.router_topk(x, wr, 64)
    np.testing.assert_array_equal(lg.view(np.uint32), O.router_logits_blocked(x, wr).view(np.uint32))
    rw, ridx = O.route_topk(lg, 64)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
