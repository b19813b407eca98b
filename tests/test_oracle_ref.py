"""Pins the oracle's reference-semantics functions to the reference's own code.

Two sources: the committed fixtures in tests/golden/ (written by
tests/golden/make_golden.py from the reference's hunyuan_moe_full.cpp), and, where
it is built, that same reference code run live on fresh seeded inputs.  All
comparisons are bit-exact: the oracle restates the reference operation for
operation.
"""
import ctypes as C
import os

import numpy as np
import pytest

import hy_oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def oracle_gating_full(logits, cfg):
    T, E = logits.shape
    g = O.GateFull()
    rc = O.lib().hyo_topkgating_full(O.fp(logits), T, C.byref(cfg), C.byref(g))
    assert rc == 0
    cap = g.capacity
    n = T * E * cap
    out = dict(
        mask=np.ctypeslib.as_array(g.dispatch_mask, (n,)).copy().reshape(T, E, cap),
        cw=np.ctypeslib.as_array(g.combine_weights, (n,)).copy().reshape(T, E, cap),
        counts=np.ctypeslib.as_array(g.exp_counts, (E,)).copy(),
        probs=np.ctypeslib.as_array(g.router_probs, (T * E,)).copy().reshape(T, E),
        capacity=np.uint32(cap), aux=np.float32(g.aux_loss), rate=np.float32(g.exp_capacity_rate))
    O.lib().hyo_gate_full_free(C.byref(g))
    return out


def oracle_easy(logits, K):
    T, E = logits.shape
    w = np.zeros((T, K), dtype=np.float32)
    idx = np.zeros((T, K), dtype=np.int32)
    O.lib().hyo_topkgating_easy(O.fp(logits), T, E, K, O.fp(w), O.ip(idx))
    return w, idx


def _cases():
    import sys
    sys.path.insert(0, GOLD)
    import make_golden
    return make_golden


def test_golden_routing(oracle):
    mg = _cases()
    data = np.load(os.path.join(GOLD, "ref_routing.npz"))
    n_checked = 0
    for name, T, E, K, kw in mg.GATING_CASES:
        for kind in ("gauss", "ties"):
            key = f"{name}_{kind}"
            lg = data[f"{key}/logits"]
            w, idx = oracle_easy(lg, K)
            np.testing.assert_array_equal(idx, data[f"{key}/easy_idx"])
            np.testing.assert_array_equal(w.view(np.uint32), data[f"{key}/easy_w"].view(np.uint32))
            g = oracle_gating_full(lg, O.default_cfg(E, K, **kw))
            for k in ("mask", "counts", "capacity"):
                np.testing.assert_array_equal(g[k], data[f"{key}/full_{k}"], err_msg=f"{key}:{k}")
            for k in ("cw", "probs", "aux", "rate"):
                np.testing.assert_array_equal(np.asarray(g[k]).view(np.uint32),
                                              np.asarray(data[f"{key}/full_{k}"]).view(np.uint32),
                                              err_msg=f"{key}:{k}")
            sm = lg[0].copy()
            O.lib().hyo_softmax_f32(O.fp(sm), E)
            np.testing.assert_array_equal(sm.view(np.uint32), data[f"{key}/softmax0"].view(np.uint32))
            n_checked += 1
    assert n_checked == 2 * len(mg.GATING_CASES)


def test_golden_single_expert_q_semantics(oracle):
    """K = 1 fixtures: the q-semantics router (the GPU's rule) selects the reference's
    expert and, under rule 1, gives the reference topkgating_full's weight p * scale
    to float rounding (the reference sums the softmax sequentially, the q-semantics
    router in a 64-lane tree); topkgating_easy's weight is exactly 1 under rule 2."""
    mg = _cases()
    data = np.load(os.path.join(GOLD, "ref_routing.npz"))
    cases = [c for c in mg.GATING_CASES if c[3] == 1]
    assert len(cases) >= 3
    for name, T, E, K, kw in cases:
        cfg = O.default_cfg(E, K, **kw)
        for kind in ("gauss", "ties"):
            key = f"{name}_{kind}"
            lg = data[f"{key}/logits"]
            norm = 1 if cfg.norm_topk_prob else 0
            w, idx = O.route_topk(lg, 1, norm=norm, scale=cfg.routed_scaling_factor)
            mask, cw = data[f"{key}/full_mask"], data[f"{key}/full_cw"]
            e_ref = mask.any(axis=2).argmax(axis=1)
            np.testing.assert_array_equal(idx[:, 0], e_ref, err_msg=key)
            w_ref = cw.sum(axis=2)[np.arange(T), e_ref]
            np.testing.assert_allclose(w[:, 0], w_ref, rtol=2e-6, err_msg=key)
            w2, _ = O.route_topk(lg, 1, norm=2)
            np.testing.assert_array_equal(w2.view(np.uint32), data[f"{key}/easy_w"].view(np.uint32))
            np.testing.assert_array_equal(data[f"{key}/easy_idx"][:, 0], e_ref)


def test_golden_test_components(oracle):
    """The reference's own component-test inputs (src/test_components.cpp:88-115)."""
    d = np.load(os.path.join(GOLD, "ref_test_components.npz"))
    lg = d["logits"]
    w, idx = oracle_easy(lg, 8)
    np.testing.assert_array_equal(idx, d["easy_idx"])
    np.testing.assert_array_equal(w.view(np.uint32), d["easy_w"].view(np.uint32))
    g = oracle_gating_full(lg, O.default_cfg(64, 8))
    assert int(g["capacity"]) == int(d["full_capacity"]) == 8
    np.testing.assert_array_equal(g["mask"], d["full_mask"])
    np.testing.assert_array_equal(g["cw"].view(np.uint32), d["full_cw"].view(np.uint32))
    assert float(g["rate"]) == float(d["full_rate"]) == 1.0


def test_golden_einsum(oracle):
    d = np.load(os.path.join(GOLD, "ref_einsum.npz"))
    x, mask = d["x"], d["mask"]
    T, H = x.shape
    E, Cc = mask.shape[1], mask.shape[2]
    disp = np.zeros((E, Cc, H), dtype=np.float32)
    O.lib().hyo_einsum_dispatch(O.fp(x), T, H, O.vp(mask), E, Cc, O.fp(disp))
    np.testing.assert_array_equal(disp.view(np.uint32), d["disp"].view(np.uint32))
    comb = np.zeros((T, H), dtype=np.float32)
    O.lib().hyo_einsum_combine(O.fp(d["cw"]), O.fp(d["eo"]), T, H, E, Cc, O.fp(comb))
    np.testing.assert_array_equal(comb.view(np.uint32), d["comb"].view(np.uint32))


def oracle_moe_full(x, wr, gu, dn, E, I, K, sgu=None, sdn=None):
    T, H = x.shape
    out = np.zeros((T, H), dtype=np.float32)
    cfg = O.default_cfg(E, K)
    rc = O.lib().hyo_moe_forward_full(O.fp(x), T, H, O.fp(wr),
                                      O.fp(sgu) if sgu is not None else None,
                                      O.fp(sdn) if sdn is not None else None,
                                      O.fp(gu), O.fp(dn), E, I, C.byref(cfg), O.fp(out))
    assert rc == 0
    return out


def test_golden_moe_forward_full(oracle):
    mg = _cases()
    d = np.load(os.path.join(GOLD, "ref_moe_full.npz"))
    for name, T, H, I, E, K, seed in mg.MOE_CASES:
        assert list(d[f"{name}/dims"]) == [T, H, I, E, K, seed]
        x, wr, gu, dn = mg.moe_case_inputs(T, H, I, E, seed)
        out = oracle_moe_full(x, wr, gu, dn, E, I, K)
        np.testing.assert_array_equal(out.view(np.uint32), d[f"{name}/out"].view(np.uint32))


# ------------------------------------------------------------------ live reference

@pytest.mark.parametrize("seed", [1, 2, 3])
def test_live_routing_vs_reference(refimpl, seed):
    mg = _cases()
    rng = np.random.default_rng(1000 + seed)
    for name, T, E, K, kw in mg.GATING_CASES:
        for kind in ("gauss", "ties"):
            lg = (rng.standard_normal((T, E)).astype(np.float32) * 2.0 if kind == "gauss"
                  else mg.logits_with_ties(rng, T, E))
            w_r = np.zeros((T, K), dtype=np.float32)
            i_r = np.zeros((T, K), dtype=np.int32)
            refimpl.ref_topkgating_easy(O.fp(lg), T, E, K, O.fp(w_r), O.ip(i_r))
            w, idx = oracle_easy(lg, K)
            np.testing.assert_array_equal(idx, i_r)
            np.testing.assert_array_equal(w.view(np.uint32), w_r.view(np.uint32))
            cfg = O.default_cfg(E, K, **kw)
            g_r = mg.ref_gating_full(refimpl, lg, cfg)
            g = oracle_gating_full(lg, cfg)
            for k in g:
                a, b = np.asarray(g[k]), np.asarray(g_r[k])
                if a.dtype == np.float32:
                    a, b = a.view(np.uint32), b.view(np.uint32)
                np.testing.assert_array_equal(a, b, err_msg=f"{name}/{kind}:{k}")


def test_live_topk_all_k(refimpl):
    rng = np.random.default_rng(5)
    for E in (8, 16, 64):
        for K in sorted({1, 2, E // 2, E}):
            for _ in range(20):
                x = (rng.integers(-3, 4, size=E) * 0.25).astype(np.float32)
                v_r = np.zeros(K, dtype=np.float32)
                i_r = np.zeros(K, dtype=np.int32)
                refimpl.ref_topk_f32(O.fp(x), E, K, O.fp(v_r), O.ip(i_r))
                v = np.zeros(K, dtype=np.float32)
                i = np.zeros(K, dtype=np.int32)
                O.lib().hyo_topk_f32(O.fp(x), E, K, O.fp(v), O.ip(i))
                np.testing.assert_array_equal(i, i_r)
                np.testing.assert_array_equal(v, v_r)


@pytest.mark.parametrize("dims", [(3, 64, 32, 8, 2), (16, 96, 64, 16, 4), (12, 64, 32, 64, 8), (7, 64, 32, 16, 1)])
def test_live_moe_forward_full_vs_reference(refimpl, dims):
    T, H, I, E, K = dims
    seed = 11 + T
    x = O.synth(seed, 0, O.T_X, 0, (T, H), 1.0)
    wr = O.synth(seed, 0, O.T_ROUTER, 0, (E, H), 0.2)
    gu = O.synth(seed, 0, O.T_GU, 0, (E, 2 * I, H), 0.05)
    dn = O.synth(seed, 0, O.T_DN, 0, (E, H, I), 0.05)
    out_r = np.zeros((T, H), dtype=np.float32)
    cfg = O.default_cfg(E, K)
    refimpl.ref_moe_forward_full_noshared(O.fp(x), T, H, O.fp(wr), O.fp(gu), O.fp(dn), E, I,
                                          C.byref(cfg), O.fp(out_r))
    out = oracle_moe_full(x, wr, gu, dn, E, I, K)
    np.testing.assert_array_equal(out.view(np.uint32), out_r.view(np.uint32))


@pytest.mark.parametrize("kw", [
    dict(drop_tokens=1, capacity_factor=1.0, min_capacity=2),
    dict(drop_tokens=1, capacity_factor=0.5, min_capacity=0, group_limited_greedy=1, n_group=4, topk_group=2),
    dict(drop_tokens=1, capacity_factor=0.75, min_capacity=0, compute_aux_loss=1, norm_topk_prob=0,
         routed_scaling_factor=2.0),
])
def test_live_moe_forward_full_options_vs_reference(refimpl, kw):
    """moe_forward_full with token dropping (alone, with group-limited greedy, with the aux
    loss and scaling): with drop_tokens the reference sizes its buffers with the same
    capacity topkgating_full writes, so these configurations run it as written."""
    T, H, I, E, K = 40, 64, 32, 16, 4
    seed = 77
    x = O.synth(seed, 0, O.T_X, 0, (T, H), 1.0)
    wr = O.synth(seed, 0, O.T_ROUTER, 0, (E, H), 0.3)
    gu = O.synth(seed, 0, O.T_GU, 0, (E, 2 * I, H), 0.05)
    dn = O.synth(seed, 0, O.T_DN, 0, (E, H, I), 0.05)
    cfg = O.default_cfg(E, K, **kw)
    out_r = np.zeros((T, H), dtype=np.float32)
    refimpl.ref_moe_forward_full_noshared(O.fp(x), T, H, O.fp(wr), O.fp(gu), O.fp(dn), E, I,
                                          C.byref(cfg), O.fp(out_r))
    out = np.zeros((T, H), dtype=np.float32)
    assert O.lib().hyo_moe_forward_full(O.fp(x), T, H, O.fp(wr), None, None, O.fp(gu), O.fp(dn), E, I,
                                        C.byref(cfg), O.fp(out)) == 0
    np.testing.assert_array_equal(out.view(np.uint32), out_r.view(np.uint32))
    # the configuration does drop pairs
    lg = np.zeros((T, E), dtype=np.float32)
    O.lib().hyo_router_logits_seq(O.fp(x), O.fp(wr), T, H, E, O.fp(lg))
    assert oracle_gating_full(lg, cfg)["rate"] < 1.0
