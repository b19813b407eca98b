"""GPU parity at the benchmark workloads' own sizes (hidden 4096, 64 routed + 1 shared
experts of width 3072, top-8):

  F32 T=16             every row against the oracle's q semantics, plus the error
                       against the reference's scalar moe_forward_full (reported)
  Q8_0 T=512           every row through row-permutation invariance
  Q4_0 T=4096 Zipf     the whole routing (logits, indices, weights) of all 4096 rows,
                       sampled rows of the layer output, permutation invariance
  32-layer Q8_0 stack  the stacked call equals 32 chained one-layer calls bit for bit;
                       the first and last layer's rows against the oracle; permutation

Row-permutation invariance is exact and covers every row: with the default routing
(no capacity, no drops) each token's output depends only on its own row, and every
output element is computed in a fixed order whatever tile the token lands in.  So
permuting the input rows must permute the output rows bit for bit.  The decode
workload (Q4_0, T = 1..8) is compared whole in test_gpu_fullsize.py.
"""
import ctypes as C

import numpy as np
import pytest

import bench
import hy_oracle as O
from test_gpu_parity import assert_exact, rel_err

pytestmark = pytest.mark.gpu

H, I, E, K = 4096, 3072, 64, 8
SEED = 42


def assert_permutes(run, x, what):
    """run(x) on a row permutation of x returns the same rows, permuted, bit for bit."""
    T = x.shape[0]
    perm = np.random.default_rng(T).permutation(T)
    a = run(x)
    b = run(np.ascontiguousarray(x[perm]))
    diff = b.view(np.uint32) != a[perm].view(np.uint32)
    assert not diff.any(), f"{what}: {int(diff.any(axis=1).sum())} of {T} rows change under a row permutation"
    return a


def sample_rows(T, extra=(), n=14):
    rng = np.random.default_rng(T + 7)
    return np.unique(np.concatenate([[0, T - 1], rng.integers(0, T, n), np.asarray(extra, np.int64)]))


def test_f32_t16_full_layer(gpu):
    """F32 weights, T=16 activations after a unit-weight RMSNorm: every output row
    bit-exact against the q semantics; the reference-semantics error is reported."""
    T = 16
    layer = O.synth_layer(H, I, E, K, O.F32, seed=SEED, std=0.02)
    raw = O.synth(SEED + 1, 0, O.T_X, 0, (T, H), 1.0)
    x = np.empty_like(raw)
    O.lib().hyo_rms_norm_f32(O.fp(raw), O.fp(np.ones(H, np.float32)), O.fp(x), T, H, np.float32(1e-5))
    m = gpu.Moe(H, I, E, K, O.F32, max_tokens=T)
    m.upload(0, layer)
    out, lg, w, idx = m.run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True, nthreads=16)
    np.testing.assert_array_equal(lg.view(np.uint32), rlg.view(np.uint32))
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert_exact(out, ref, "F32 T=16")
    # the reference's own arithmetic (sequential fp32 sums, capacity-slot dispatch):
    # its capacity stride is right while no expert takes more than 8 of the 16 tokens
    assert np.bincount(idx.ravel(), minlength=E).max() <= 8
    rs = np.zeros((T, H), np.float32)
    cfg = O.default_cfg(E, K)
    assert O.lib().hyo_moe_forward_full(O.fp(x), T, H, O.fp(layer.router), O.fp(layer.shared_gu),
                                        O.fp(layer.shared_dn), O.fp(layer.gu), O.fp(layer.dn), E, I,
                                        C.byref(cfg), O.fp(rs)) == 0
    e = rel_err(out, rs)
    print(f"F32 T=16 vs reference semantics: normwise rel err {e:.3e}")
    assert e < 1e-4
    assert_permutes(lambda v: m.run(0, v), x, "F32 T=16")
    m.close()


def test_q8_0_t512_every_row(gpu):
    T = 512
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=T)
    m.synth(0, seed=SEED, std=0.02)
    x = O.synth(SEED + 1000, 0, O.T_X, 0, (T, H), 1.0)
    assert_permutes(lambda v: m.run(0, v), x, "Q8_0 T=512")
    m.close()


def test_q4_0_t4096_zipf(gpu):
    """The skewed image-token workload: all 4096 rows' routing bit-exact, the skew as
    calibrated, sampled rows (hot, cold and unrouted-hot tokens) of the output exact."""
    T = 4096
    bias = bench.zipf_bias(SEED)
    layer = O.synth_layer(H, I, E, K, O.Q4_0, seed=SEED, std=0.02, router_bias=bias)
    x = O.synth(SEED + 1000, 0, O.T_X, 0, (T, H), 1.0)
    x[:, 0] = 1.0
    m = gpu.Moe(H, I, E, K, O.Q4_0, max_tokens=T)
    m.upload(0, layer)
    out, lg, w, idx = m.run(0, x, debug=True)
    rlg = O.router_logits_blocked(x, layer.router)
    np.testing.assert_array_equal(lg.view(np.uint32), rlg.view(np.uint32))
    rw, ridx = O.route_topk(rlg, K)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
    cnt = np.bincount(idx.ravel(), minlength=E)
    order = np.argsort(-cnt, kind="stable")
    assert cnt[order[:8]].sum() / (T * K) >= 0.62 and cnt[order[0]] > 3900
    hot, cold = order[0], order[np.flatnonzero(cnt[order] > 0)[-1]]
    no_hot = np.flatnonzero(~(idx == hot).any(axis=1))[:3]
    with_cold = np.flatnonzero((idx == cold).any(axis=1))[:3]
    rows = sample_rows(T, extra=np.concatenate([no_hot, with_cold]))
    ref = O.moe_forward_q_rows(layer, x, rows, nthreads=16)
    assert_exact(out[rows], ref, "Q4_0 T=4096 Zipf")
    assert_permutes(lambda v: m.run(0, v), x, "Q4_0 T=4096 Zipf")
    m.close()


def test_q8_0_stack32_t4096(gpu):
    """32 resident Q8_0 layers (h <- h + MoE(RMSNorm(h)), weights seeded by layer
    index): the stacked call equals 32 chained one-layer calls bit for bit, layers 0
    and 31 match the oracle on sampled rows, and the stack permutes rows exactly."""
    T, nl, eps = 4096, 32, 1e-5
    m = gpu.Moe(H, I, E, K, O.Q8_0, num_layers=nl, max_tokens=T)
    for l in range(nl):
        m.synth(l, seed=SEED, std=0.02)
    x = O.synth(SEED + 1000, 0, O.T_X, 0, (T, H), 1.0)
    xb = gpu.Buf.from_array(x)
    out = gpu.Buf.empty((T, H))
    m.stack_forward(0, nl, xb, T, eps, out)
    stacked = out.numpy()
    bufs = [gpu.Buf.from_array(x), gpu.Buf.empty((T, H))]
    h1 = h31 = None
    for l in range(nl):
        m.stack_forward(l, 1, bufs[l % 2], T, eps, bufs[(l + 1) % 2])
        if l == 0:
            h1 = bufs[1].numpy()
        if l == nl - 2:
            h31 = bufs[(l + 1) % 2].numpy()
    chained = bufs[nl % 2].numpy()
    np.testing.assert_array_equal(chained.view(np.uint32), stacked.view(np.uint32))
    rows = sample_rows(T)
    L0 = O.synth_layer(H, I, E, K, O.Q8_0, seed=SEED, layer=0, std=0.02)
    assert_exact(h1[rows], O.moe_stack_q([L0], x[rows], eps, nthreads=16), "stack layer 0")
    del L0
    L31 = O.synth_layer(H, I, E, K, O.Q8_0, seed=SEED, layer=nl - 1, std=0.02)
    assert_exact(stacked[rows], O.moe_stack_q([L31], h31[rows], eps, nthreads=16), "stack layer 31")
    del L31

    def run(v):
        vb = gpu.Buf.from_array(v)
        m.stack_forward(0, nl, vb, T, eps, out)
        return out.numpy()

    assert_permutes(run, x, "32-layer stack T=4096")
    m.close()
