"""Pins the q-semantics oracle's routing options beyond the default: group-limited
greedy, the load-balancing aux loss and capacity-limited token dropping
(src/hunyuan_moe_full.cpp:135-214, 245-304).

Anchors: the reference-semantics gating (hyo_topkgating_full, itself bit-exact against
the reference's own code and its fixtures in test_oracle_ref.py), closed forms, and
float64 arithmetic on the dequantized operands for the layer with dropped pairs.
"""
import numpy as np
import pytest

import hy_oracle as O
from test_oracle_ref import oracle_gating_full

GROUP_CASES = [
    # T, E, K, n_group, topk_group
    (40, 16, 4, 4, 2),      # the fixture case's shape
    (50, 64, 8, 8, 3),
    (30, 64, 6, 3, 2),      # 64 % 3: experts 63.. belong to no group and are never masked
    (20, 16, 6, 4, 1),      # K > the 4 allowed experts: masked zeros fill, lowest index first
    (20, 16, 4, 20, 3),     # E / n_group == 0: no expert is in a group
    (20, 16, 4, 4, 9),      # topk_group > n_group: every group kept
    (25, 8, 1, 2, 1),       # K = 1: p * scale
]


def _selected(g, T, E):
    """Selected experts and their weights per token from the dense reference outputs."""
    sel = [set(np.nonzero(g["mask"][t].any(axis=1))[0].tolist()) for t in range(T)]
    w = g["cw"].sum(axis=2)
    return sel, w


@pytest.mark.parametrize("T,E,K,ng,tg", GROUP_CASES)
def test_group_routing_matches_reference_semantics(oracle, T, E, K, ng, tg):
    rng = np.random.default_rng(1000 + 7 * E + ng)
    lg = (rng.standard_normal((T, E)) * 1.5).astype(np.float32)
    for norm, scale in ((1, 1.0), (0, 2.5)):
        g = oracle_gating_full(lg, O.default_cfg(E, K, group_limited_greedy=1, n_group=ng, topk_group=tg,
                                                 norm_topk_prob=norm, routed_scaling_factor=scale))
        sel, wref = _selected(g, T, E)
        w, idx, probs = O.route_topk_groups(lg, K, norm=norm, scale=scale, n_group=ng, topk_group=tg)
        for t in range(T):
            assert set(idx[t].tolist()) == sel[t], (t, idx[t], sel[t])
            # q probabilities (hyo_expf, tree sum) against the reference's softmax
            np.testing.assert_allclose(w[t], wref[t, idx[t]], rtol=3e-6, atol=1e-12)
        # ranks: descending masked probability, equal values by index
        for t in range(T):
            key = [(-probs[t, e], e) for e in idx[t]]
            assert key == sorted(key)


def test_group_routing_fixture_case(oracle):
    """The reference-built fixture case group_t9_e16_k4 (tests/golden/ref_routing.npz)."""
    import os
    data = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_routing.npz"))
    for kind in ("gauss", "ties"):
        lg = data[f"group_t9_e16_k4_{kind}/logits"]
        mask, cw = data[f"group_t9_e16_k4_{kind}/full_mask"], data[f"group_t9_e16_k4_{kind}/full_cw"]
        w, idx, _ = O.route_topk_groups(lg, 4, n_group=4, topk_group=2)
        for t in range(lg.shape[0]):
            assert set(idx[t].tolist()) == set(np.nonzero(mask[t].any(axis=1))[0].tolist())
            np.testing.assert_allclose(w[t], cw[t].sum(axis=1)[idx[t]], rtol=3e-6, atol=1e-12)


def test_group_routing_without_groups_is_default(oracle):
    """n_group = 0 or topk_group = 0 leaves the default rule (the reference's condition,
    src/hunyuan_moe_full.cpp:135): bit-identical to hyo_route_topk."""
    rng = np.random.default_rng(5)
    lg = rng.standard_normal((33, 64)).astype(np.float32)
    w0, i0 = O.route_topk(lg, 8)
    for ng, tg in ((0, 3), (8, 0)):
        w, idx, _ = O.route_topk_groups(lg, 8, n_group=ng, topk_group=tg)
        np.testing.assert_array_equal(idx, i0)
        np.testing.assert_array_equal(w.view(np.uint32), w0.view(np.uint32))


def test_group_masking_closed_form(oracle):
    """Two groups of 4, the best group holds the single largest logit: every selected
    expert comes from it, and with K = 6 the two fillers are the masked group's experts
    0 and 1 with weight exactly 0."""
    lg = np.array([[0.0, 0.1, 0.2, 0.3, 5.0, -1.0, -2.0, -3.0]], np.float32)
    w, idx, probs = O.route_topk_groups(lg, 6, n_group=2, topk_group=1)
    assert idx[0].tolist() == [4, 5, 6, 7, 0, 1]
    assert np.all(w[0, 4:] == 0.0) and np.all(probs[0, :4] == 0.0)
    np.testing.assert_allclose(w[0, :4].sum(), 1.0, rtol=1e-6)


@pytest.mark.parametrize("T,E,K,ng,tg", [(12, 8, 3, 0, 0), (40, 16, 4, 4, 2), (64, 64, 8, 8, 3)])
def test_aux_loss_matches_reference_semantics(oracle, T, E, K, ng, tg):
    rng = np.random.default_rng(77 + T)
    lg = (rng.standard_normal((T, E)) * 1.5).astype(np.float32)
    kw = dict(compute_aux_loss=1)
    if ng:
        kw.update(group_limited_greedy=1, n_group=ng, topk_group=tg)
    g = oracle_gating_full(lg, O.default_cfg(E, K, **kw))
    w, idx, probs = O.route_topk_groups(lg, K, n_group=ng, topk_group=tg)
    aux = O.aux_loss_q(probs, idx)
    np.testing.assert_allclose(aux, g["aux"], rtol=2e-5)


def test_aux_loss_closed_form(oracle):
    """Equal logits: p = 1/E for every expert (E a power of two: exact), every token picks
    experts 0..K-1 (lower index on ties), so tokens_per_expert is 1 for those K and 0 for
    the rest, router_prob_per_expert is 1/E, and the loss is K * (1/E) * E^2 = K * E."""
    for T, E, K in ((10, 8, 2), (33, 64, 8), (5, 16, 16)):
        lg = np.zeros((T, E), np.float32)
        w, idx, probs = O.route_topk_groups(lg, K)
        assert np.all(idx == np.arange(K))
        assert O.aux_loss_q(probs, idx) == np.float32(K * E)


@pytest.mark.parametrize("T,E,K,cf,mc", [(40, 16, 4, 1.0, 2), (200, 64, 8, 1.0, 0), (200, 64, 8, 0.5, 0),
                                         (97, 16, 4, 1.25, 3), (30, 8, 2, 0.3, 9), (16, 64, 8, 1.0, 0)])
def test_capacity_and_drops_match_reference_semantics(oracle, T, E, K, cf, mc):
    rng = np.random.default_rng(300 + T + K)
    # skewed logits so that some experts overflow
    lg = (rng.standard_normal((T, E)) * 1.5 + np.linspace(2.0, -2.0, E)[None]).astype(np.float32)
    g = oracle_gating_full(lg, O.default_cfg(E, K, drop_tokens=1, capacity_factor=cf, min_capacity=mc))
    cap = O.drop_capacity(T, E, K, cf, mc)
    assert cap == int(g["capacity"])
    w, idx = O.route_topk(lg, K)
    keep = O.capacity_keep(idx, E, cap)
    kept_ref = g["mask"].any(axis=2)  # [T, E]
    for t in range(T):
        assert set(idx[t][keep[t]].tolist()) == set(np.nonzero(kept_ref[t])[0].tolist())
    # the kept share is the reference's exp_capacity_rate
    assert np.float32(keep.sum()) / np.float32(T * K) == g["rate"]
    counts = np.bincount(idx.ravel(), minlength=E)
    assert np.array_equal(np.bincount(idx[keep], minlength=E), np.minimum(counts, cap))


@pytest.mark.parametrize("wtype", [O.Q8_0, O.F32])
def test_q_layer_with_drops_vs_float64(wtype):
    """Dropped pairs contribute nothing: the layer equals float64 arithmetic over the kept
    pairs only, and a token whose pairs are all dropped gets the shared expert alone."""
    T, H, I, E, K = 24, 64, 32, 4, 2
    layer = O.synth_layer(H, I, E, K, wtype, seed=19, std=0.05)
    x = O.synth(19, 0, O.T_X, 0, (T, H), 1.0)
    layer.capacity = 5  # 48 pairs over 4 experts: most experts overflow
    out, lg, w, idx = O.moe_forward_q(layer, x, debug=True)
    keep = O.capacity_keep(idx, E, 5)
    assert 0 < keep.sum() < T * K
    gu, dn, sgu, sdn = layer.dequant()

    def act(v):
        v = O.f32(v)
        return v.astype(np.float64) if wtype == O.F32 else O.dequantize(O.quantize(v, O.Q8_0), O.Q8_0,
                                                                        v.shape[-1]).astype(np.float64)

    def ffn(xt, g_u, d):
        t = g_u.astype(np.float64) @ act(xt[None])[0]
        g, u = t[:I], t[I:]
        h = (g / (1 + np.exp(-g)) * u).astype(np.float32)
        return d.astype(np.float64) @ act(h[None])[0]

    ref = np.zeros((T, H))
    for t in range(T):
        for k in np.argsort(idx[t]):
            if keep[t, k]:
                ref[t] += w[t, k] * ffn(x[t], gu[idx[t, k]], dn[idx[t, k]])
        ref[t] += ffn(x[t], sgu, sdn)
    err = np.abs(out - ref).max() / np.abs(ref).max()
    assert err < 2e-4, err
    # every pair of the last tokens is dropped: shared expert only, bit for bit equal to a
    # layer whose routed weights are all 0 (zero weights are skipped)
    gone = np.nonzero(~keep.any(axis=1))[0]
    assert gone.size > 0
    zero = O.Layer(H, I, E, K, wtype, layer.router, layer.shared_gu, layer.shared_dn, layer.gu, layer.dn,
                   norm_topk_prob=False, routed_scaling_factor=0.0)
    np.testing.assert_array_equal(out[gone], O.moe_forward_q(zero, x[gone]))
    # sampled rows equal the full batch (the batch is routed first)
    rows = np.array([0, 7, T - 1])
    np.testing.assert_array_equal(O.moe_forward_q_rows(layer, x, rows), out[rows])
    # a capacity no expert reaches drops nothing
    layer.capacity = T * K
    np.testing.assert_array_equal(O.moe_forward_q(layer, x), O.moe_forward_q(
        O.Layer(H, I, E, K, wtype, layer.router, layer.shared_gu, layer.shared_dn, layer.gu, layer.dn), x))


def test_route_q_batch_matches_per_token(oracle):
    H, I, E, K, T = 64, 32, 16, 4, 30
    layer = O.synth_layer(H, I, E, K, O.Q8_0, seed=23, std=0.05)
    layer.n_group, layer.topk_group = 4, 2
    x = O.synth(23, 0, O.T_X, 0, (T, H), 1.0)
    lg, w, idx, probs, keep = O.moe_route_q(layer, x)
    w2, i2, p2 = O.route_topk_groups(lg, K, n_group=4, topk_group=2)
    np.testing.assert_array_equal(idx, i2)
    np.testing.assert_array_equal(w.view(np.uint32), w2.view(np.uint32))
    np.testing.assert_array_equal(probs.view(np.uint32), p2.view(np.uint32))
    assert keep.all()
    _, lg3, w3, i3 = O.moe_forward_q(layer, x, debug=True)
    np.testing.assert_array_equal(i3, idx)
    np.testing.assert_array_equal(lg3.view(np.uint32), lg.view(np.uint32))


def random_routing_configs(n, seed):
    """Seeded random routing configurations: shapes, groups (including E / n_group = 0
    and topk_group >= n_group), dropping with small and large capacity factors, the aux
    loss, both weight rules."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        E = int(rng.choice([1, 2, 3, 7, 8, 16, 33, 64]))
        K = int(rng.integers(1, E + 1))
        T = int(rng.integers(1, 120))
        kw = dict(norm_topk_prob=int(rng.integers(0, 2)), routed_scaling_factor=float(rng.choice([1.0, 2.5])))
        if rng.random() < 0.5:
            kw.update(group_limited_greedy=1, n_group=int(rng.integers(1, 2 * E + 2)),
                      topk_group=int(rng.integers(1, 9)))
        if rng.random() < 0.5:
            kw.update(drop_tokens=1, capacity_factor=float(rng.choice([0.25, 0.5, 1.0, 2.0])),
                      min_capacity=int(rng.integers(0, 6)))
        if rng.random() < 0.5:
            kw.update(compute_aux_loss=1)
        out.append((T, E, K, kw))
    return out


def test_random_configs_vs_reference_semantics(oracle):
    """200 random configurations: the q-semantics pieces (selection, weights, kept pairs,
    capacity, capacity rate, aux loss) against the reference-semantics gating."""
    rng = np.random.default_rng(12)
    for T, E, K, kw in random_routing_configs(200, 11):
        lg = (rng.standard_normal((T, E)) * 1.5).astype(np.float32)
        g = oracle_gating_full(lg, O.default_cfg(E, K, **kw))
        groups = kw.get("group_limited_greedy", 0)
        ng, tg = (kw["n_group"], kw["topk_group"]) if groups else (0, 0)
        w, idx, probs = O.route_topk_groups(lg, K, norm=kw["norm_topk_prob"], scale=kw["routed_scaling_factor"],
                                            n_group=ng, topk_group=tg)
        what = f"T={T} E={E} K={K} {kw}"
        counts = np.bincount(idx.ravel(), minlength=E)
        np.testing.assert_array_equal(counts, g["counts"], err_msg=what)
        if kw.get("drop_tokens"):
            cap = O.drop_capacity(T, E, K, kw["capacity_factor"], kw["min_capacity"])
        else:
            cap = max(int(counts.max()), kw.get("min_capacity", 8))
        assert cap == int(g["capacity"]), what
        keep = O.capacity_keep(idx, E, cap)
        assert np.float32(keep.sum()) / np.float32(T * K) == g["rate"], what
        kept_ref = g["mask"].any(axis=2)
        wref = g["cw"].sum(axis=2)
        for t in range(T):
            assert set(idx[t][keep[t]].tolist()) == set(np.nonzero(kept_ref[t])[0].tolist()), (what, t)
            np.testing.assert_allclose(w[t][keep[t]], wref[t, idx[t][keep[t]]], rtol=3e-6, atol=1e-12,
                                       err_msg=what)
        if kw.get("compute_aux_loss"):
            np.testing.assert_allclose(O.aux_loss_q(probs, idx), g["aux"], rtol=2e-5, err_msg=what)


# ------------------------------------------------------------------ NaN logits

def select_q(x, k):
    x = O.f32(x)
    v = np.empty(k, np.float32)
    i = np.empty(k, np.int32)
    O.lib().hyo_select_q(O.fp(x), x.size, k, O.fp(v), O.ip(i))
    return v, i


def test_select_q_is_topk_f32_without_nan(oracle):
    """Rows without NaN (with ties and infinities): the q selection equals the
    reference's insertion top-k (src/hunyuan_moe_full.cpp:56-82) exactly."""
    rng = np.random.default_rng(11)
    for trial in range(400):
        n = int(rng.integers(1, 65))
        k = int(rng.integers(1, n + 1))
        x = rng.integers(-4, 5, n).astype(np.float32)          # many ties
        if trial % 3 == 0:
            x[rng.integers(0, n, 2)] = -np.inf
        if trial % 5 == 0:
            x[rng.integers(0, n)] = np.inf
        v, i = select_q(x, k)
        rv = np.empty(k, np.float32)
        ri = np.empty(k, np.int32)
        O.lib().hyo_topk_f32(O.fp(x), n, k, O.fp(rv), O.ip(ri))
        np.testing.assert_array_equal(i, ri)
        np.testing.assert_array_equal(v, rv)


def test_select_q_nan_rows(oracle):
    """An all-NaN row selects 0..k-1 (the reference's insertion order for NaN); in a
    mixed row every number ranks above every NaN and NaNs follow in index order."""
    v, i = select_q(np.full(64, np.nan, np.float32), 8)
    np.testing.assert_array_equal(i, np.arange(8))
    assert np.isnan(v).all()
    rv = np.empty(8, np.float32)
    ri = np.empty(8, np.int32)
    O.lib().hyo_topk_f32(O.fp(np.full(64, np.nan, np.float32)), 64, 8, O.fp(rv), O.ip(ri))
    np.testing.assert_array_equal(ri, np.arange(8))
    x = np.array([np.nan, 5, np.nan, 3, -np.inf, np.nan, 5], np.float32)
    v, i = select_q(x, 6)
    np.testing.assert_array_equal(i, [1, 6, 3, 4, 0, 2])
    np.testing.assert_array_equal(v[:4], [5, 5, 3, -np.inf])
    assert np.isnan(v[4:]).all()


def test_route_q_nan_row(oracle):
    """The q routing of a token whose logits are all NaN: experts 0..K-1, NaN weights;
    the other tokens of the batch are unaffected."""
    rng = np.random.default_rng(3)
    lg = rng.standard_normal((4, 16)).astype(np.float32)
    ref_w, ref_i = O.route_topk(lg, 4)
    lg[2] = np.nan
    w, i = O.route_topk(lg, 4)
    np.testing.assert_array_equal(i[2], np.arange(4))
    assert np.isnan(w[2]).all()
    keep = [0, 1, 3]
    np.testing.assert_array_equal(i[keep], ref_i[keep])
    np.testing.assert_array_equal(w[keep], ref_w[keep])
