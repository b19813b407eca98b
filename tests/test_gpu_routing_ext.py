"""GPU parity of the routing options of topkgating_full beyond the default
(src/hunyuan_moe_full.cpp:135-214, 245-304): group-limited greedy, capacity-limited
token dropping and the load-balancing aux loss, through the C ABI, against the
q-semantics oracle, bit for bit.  Decode batches (T <= 16) take the general routing
path when an option is on, so every T regime is covered."""
import numpy as np
import pytest

import hy_oracle as O
from test_gpu_parity import assert_exact

pytestmark = pytest.mark.gpu

H, I = 256, 128


def skewed_input(seed, T, E):
    """x with x[:, 0] = 1 so the router bias column (router_bias) skews the logits."""
    x = O.synth(seed, 0, O.T_X, 0, (T, H), 1.0)
    x[:, 0] = 1.0
    return x


def bias(E, span=2.0):
    return np.linspace(span, -span, E).astype(np.float32)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0, O.F32])
def test_group_limited_greedy_layer(gpu, wtype):
    E, K, ng, tg = 64, 8, 8, 3
    layer = O.synth_layer(H, I, E, K, wtype, seed=120, std=0.05)
    layer.n_group, layer.topk_group = ng, tg
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=300, group_limited_greedy=1, n_group=ng, topk_group=tg)
    m.upload(0, layer)
    paths = [gpu.PATH_AUTO] if wtype == O.F32 else [gpu.PATH_AUTO, gpu.PATH_VALU, gpu.PATH_MFMA]
    for T in (1, 7, 40, 300):
        x = O.synth(121 + T, 0, O.T_X, 0, (T, H), 1.0)
        ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
        for path in paths if T == 40 else [gpu.PATH_AUTO]:
            m.set_path(path)
            out, lg, w, idx = m.run(0, x, debug=True)
            np.testing.assert_array_equal(lg.view(np.uint32), rlg.view(np.uint32))
            np.testing.assert_array_equal(idx, ridx)
            np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
            assert_exact(out, ref, f"groups wtype={wtype} T={T} path={path}")
        # every selected expert lies in one of the topk_group kept groups
        assert all(len(set((idx[t] // (E // ng)).tolist())) <= tg for t in range(T))
    m.set_path(gpu.PATH_AUTO)
    m.close()


def test_group_limited_greedy_fillers(gpu):
    """K larger than the kept groups' experts: masked experts fill with weight 0, which
    the combine skips."""
    E, K, ng, tg = 16, 6, 4, 1
    layer = O.synth_layer(H, I, E, K, O.Q8_0, seed=130, std=0.05)
    layer.n_group, layer.topk_group = ng, tg
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=64, group_limited_greedy=1, n_group=ng, topk_group=tg)
    m.upload(0, layer)
    for T in (3, 33):
        x = O.synth(131 + T, 0, O.T_X, 0, (T, H), 1.0)
        out, lg, w, idx = m.run(0, x, debug=True)
        ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
        np.testing.assert_array_equal(idx, ridx)
        np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
        assert np.all(w[:, 4:] == 0.0)
        assert_exact(out, ref, f"fillers T={T}")
    m.close()


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0, O.F32])
@pytest.mark.parametrize("cf,mc", [(0.5, 0), (1.0, 3)])
def test_token_dropping_layer(gpu, wtype, cf, mc):
    E, K = 16, 4
    layer = O.synth_layer(H, I, E, K, wtype, seed=140, std=0.05, router_bias=bias(E))
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=700, drop_tokens=1, capacity_factor=cf, min_capacity=mc)
    m.upload(0, layer)
    n_dropped = 0
    for T in (5, 16, 40, 700):
        x = skewed_input(141 + T, T, E)
        cap = O.drop_capacity(T, E, K, cf, mc)
        layer.capacity = cap
        out, lg, w, idx = m.run(0, x, debug=True)
        ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
        np.testing.assert_array_equal(idx, ridx)
        np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
        assert_exact(out, ref, f"drop wtype={wtype} cf={cf} T={T} cap={cap}")
        keep = O.capacity_keep(ridx, E, cap)
        n_dropped += int((~keep).sum())
        aux, gcap, rate = m.last_gate()
        assert gcap == cap and aux == 0.0
        assert rate == np.float32(keep.sum()) / np.float32(T * K)
        D, counts = m.last_routing()
        np.testing.assert_array_equal(counts, np.bincount(ridx.ravel(), minlength=E))
    assert n_dropped > 0
    m.close()


@pytest.mark.parametrize("groups", [False, True])
def test_aux_loss(gpu, groups):
    E, K = 64, 8
    kw = dict(group_limited_greedy=1, n_group=8, topk_group=4) if groups else {}
    layer = O.synth_layer(H, I, E, K, O.Q8_0, seed=150, std=0.05)
    if groups:
        layer.n_group, layer.topk_group = 8, 4
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=2000, compute_aux_loss=1, **kw)
    m.upload(0, layer)
    for T in (1, 16, 40, 2000):
        x = O.synth(151 + T, 0, O.T_X, 0, (T, H), 1.0)
        out = m.run(0, x)
        lg, w, idx, probs, keep = O.moe_route_q(layer, x, nthreads=8)
        aux, cap, rate = m.last_gate()
        assert aux == O.aux_loss_q(probs, idx), (T, aux, O.aux_loss_q(probs, idx))
        counts = np.bincount(idx.ravel(), minlength=E)
        assert cap == max(int(counts.max()), 0) and rate == np.float32(1.0)
        if T <= 40:
            assert_exact(out, O.moe_forward_q(layer, x), f"aux T={T}")
    m.close()


def test_all_options_stack(gpu):
    """Two stacked layers with groups, dropping and the aux loss on, decode and batch."""
    E, K, L = 16, 4, 2
    layers = [O.synth_layer(H, I, E, K, O.Q8_0, seed=160, layer=l, std=0.05) for l in range(L)]
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=100, num_layers=L, group_limited_greedy=1, n_group=4, topk_group=2,
                drop_tokens=1, capacity_factor=0.75, min_capacity=0, compute_aux_loss=1)
    for l in range(L):
        m.synth(l, seed=160, std=0.05)
    for T in (6, 100):
        cap = O.drop_capacity(T, E, K, 0.75, 0)
        for lyr in layers:
            lyr.n_group, lyr.topk_group, lyr.capacity = 4, 2, cap
        x = O.synth(161 + T, 0, O.T_X, 0, (T, H), 1.0)
        xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((T, H))
        m.stack_forward(0, L, xb, T, 1e-5, ob)
        assert_exact(ob.numpy(), O.moe_stack_q(layers, x, eps=1e-5), f"options stack T={T}")
    m.close()


def test_route_logits_groups_and_aux_entry_points(gpu):
    """hy_route_logits_groups and hy_aux_loss, the calls the C++ topkgating_full uses."""
    rng = np.random.default_rng(170)
    for T, E, K, ng, tg in ((37, 64, 8, 8, 3), (5, 16, 6, 4, 1), (300, 16, 4, 0, 0), (9, 64, 8, 3, 2),
                            (20, 16, 4, 20, 3), (20, 16, 4, 4, 9), (25, 8, 1, 2, 1), (11, 64, 16, 64, 64)):
        lg = (rng.standard_normal((T, E)) * 1.5).astype(np.float32)
        for norm, scale in ((1, 1.0), (0, 2.5)):
            w, idx, probs = gpu.route_logits_groups(lg, K, norm=norm, scale=scale, n_group=ng, topk_group=tg)
            rw, ridx, rprobs = O.route_topk_groups(lg, K, norm=norm, scale=scale, n_group=ng, topk_group=tg)
            np.testing.assert_array_equal(idx, ridx)
            np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
            np.testing.assert_array_equal(probs.view(np.uint32), rprobs.view(np.uint32))
            counts = np.bincount(idx.ravel(), minlength=E).astype(np.int32)
            assert gpu.aux_loss(probs, counts) == O.aux_loss_q(rprobs, ridx)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
def test_options_without_shared_expert_and_single_topk(gpu, wtype):
    """No shared expert (a token whose pairs are all dropped gets exactly 0) and K = 1
    (weight p * scale under topkgating_full's rule), with groups and dropping."""
    E, K = 8, 1
    layer = O.synth_layer(H, I, E, K, wtype, seed=180, std=0.05, router_bias=bias(E, 3.0), shared=False)
    layer.n_group, layer.topk_group = 2, 1
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=64, has_shared=False, routed_scaling_factor=1.5,
                group_limited_greedy=1, n_group=2, topk_group=1, drop_tokens=1, capacity_factor=1.0, min_capacity=0)
    layer.routed_scaling_factor = 1.5
    m.upload(0, layer)
    for T in (3, 16, 64):
        x = skewed_input(181 + T, T, E)
        cap = O.drop_capacity(T, E, K, 1.0, 0)
        layer.capacity = cap
        out, lg, w, idx = m.run(0, x, debug=True)
        ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
        np.testing.assert_array_equal(idx, ridx)
        np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
        assert_exact(out, ref, f"no shared, K=1, T={T}")
        keep = O.capacity_keep(ridx, E, cap)
        if (~keep).any():
            assert np.all(out[~keep[:, 0]] == 0.0)
    m.close()


def test_random_configs_layer(gpu):
    """24 seeded random configurations (E from 1 to 64, K up to E, groups including
    n_group > E and topk_group >= n_group, dropping with small and large capacity
    factors, the aux loss, both weight rules, with and without the shared expert, all
    three weight types) through the layer: bit for bit against the q-semantics oracle,
    with the gate statistics."""
    from test_oracle_routing_ext import random_routing_configs
    H2, I2 = 128, 128
    for i, (T, E, K, kw) in enumerate(random_routing_configs(24, 21)):
        wtype = (O.Q8_0, O.Q4_0, O.F32)[i % 3]
        shared = i % 2 == 0
        layer = O.synth_layer(H2, I2, E, K, wtype, seed=300 + i, std=0.05, shared=shared)
        layer.norm_topk_prob = kw["norm_topk_prob"]
        layer.routed_scaling_factor = kw["routed_scaling_factor"]
        if kw.get("group_limited_greedy"):
            layer.n_group, layer.topk_group = kw["n_group"], kw["topk_group"]
        cap = O.drop_capacity(T, E, K, kw["capacity_factor"], kw["min_capacity"]) if kw.get("drop_tokens") else 0
        layer.capacity = cap
        m = gpu.Moe(H2, I2, E, K, wtype, max_tokens=T, has_shared=shared, **kw)
        m.upload(0, layer)
        x = O.synth(400 + i, 0, O.T_X, 0, (T, H2), 1.0)
        what = f"case {i}: T={T} E={E} K={K} wtype={wtype} shared={shared} {kw}"
        out, lg, w, idx = m.run(0, x, debug=True)
        ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
        np.testing.assert_array_equal(idx, ridx, err_msg=what)
        np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32), err_msg=what)
        assert_exact(out, ref, what)
        aux, gcap, rate = m.last_gate()
        _, _, ridx2, probs, keep = O.moe_route_q(layer, x)
        counts = np.bincount(ridx.ravel(), minlength=E)
        assert gcap == (cap if cap else max(int(counts.max()), kw.get("min_capacity", 0))), what
        assert rate == np.float32(keep.sum()) / np.float32(T * K), what
        assert aux == (O.aux_loss_q(probs, ridx) if kw.get("compute_aux_loss") else 0.0), what
        m.close()


# ------------------------------------------------------------------ NaN logits

def assert_weights(w, rw):
    """Weights equal bit for bit where the oracle's are numbers, NaN where its are."""
    np.testing.assert_array_equal(np.isnan(w), np.isnan(rw))
    ok = ~np.isnan(rw)
    np.testing.assert_array_equal(w[ok].view(np.uint32), rw[ok].view(np.uint32))


@pytest.mark.parametrize("E,K", [(64, 8), (16, 4), (64, 64)])
def test_nan_and_infinite_logits(gpu, E, K):
    """Selection with NaN and infinite logits: an all-NaN row selects experts 0..K-1
    (the reference's insertion order for NaN), numbers rank above NaN, -inf ties go to
    the lower index; every index stays in [0, E) and distinct.  Default and grouped
    selection against the oracle."""
    rng = np.random.default_rng(E + K)
    T = 6
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[1] = np.nan
    lg[3, ::3] = np.nan
    lg[4] = -np.inf
    lg[4, 5] = 0.0
    lg[5, 2] = np.inf
    w, idx, _ = gpu.route_logits_groups(lg, K)
    rw, ridx = O.route_topk(lg, K)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(idx[1], np.arange(K))
    assert all(len(set(r)) == K for r in idx.tolist()) and idx.min() >= 0 and idx.max() < E
    assert_weights(w, rw)
    if E % 4 == 0:
        w, idx, p = gpu.route_logits_groups(lg, K, n_group=4, topk_group=2)
        rw, ridx, rp = O.route_topk_groups(lg, K, n_group=4, topk_group=2)
        np.testing.assert_array_equal(idx, ridx)
        assert_weights(w, rw)
        assert_weights(p, rp)
    vals, ti = gpu.topk_rows(lg, K)
    np.testing.assert_array_equal(ti[1], np.arange(K))
    assert np.isnan(vals[1]).all()


@pytest.mark.parametrize("T", [1, 5, 40])
def test_nan_token_in_layer(gpu, T):
    """A token whose activations are NaN routes to experts 0..K-1 and gets a NaN
    output row; the other tokens are bit-exact against the oracle (one-token routing
    inside the gate/up launch, the decode routing pass, the grouped GEMM)."""
    E, K = 64, 8
    layer = O.synth_layer(H, I, E, K, O.Q8_0, seed=130, std=0.05)
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=64)
    m.upload(0, layer)
    x = O.synth(131, 0, O.T_X, 0, (T, H), 1.0)
    bad = T // 2
    xn = x.copy()
    xn[bad] = np.nan
    out, lg, w, idx = m.run(0, xn, debug=True)
    np.testing.assert_array_equal(idx[bad], np.arange(K))
    assert np.isnan(out[bad]).all()
    rest = [t for t in range(T) if t != bad]
    if rest:
        ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
        np.testing.assert_array_equal(idx[rest], ridx[rest])
        assert_exact(out[rest], ref[rest], f"T={T} rows beside the NaN token")
    m.close()


@pytest.mark.parametrize("E", [1, 7, 16, 64])
def test_aux_loss_kernel_shapes(gpu, E):
    """hy_aux_loss on gate rows staged in 128-row chunks: partial last chunks, expert
    counts that do not divide the stage, T = 1 .. 4096, bit-exact against the oracle's
    sequential sums.  Prints the T=4096, E=64 kernel time."""
    rng = np.random.default_rng(E)
    for T in (1, 127, 128, 129, 300, 4096):
        probs = rng.random((T, E)).astype(np.float32)
        probs /= probs.sum(axis=1, keepdims=True)
        K = min(E, 4)
        idx = np.argsort(-probs, axis=1, kind="stable")[:, :K].astype(np.int32)
        counts = np.bincount(idx.ravel(), minlength=E).astype(np.int32)
        got = gpu.aux_loss(probs, counts)
        assert got == O.aux_loss_q(probs, idx), (E, T)
    if E == 64:
        pb, cb, ob = gpu.Buf.from_array(probs), gpu.Buf.from_array(counts), gpu.Buf.empty((1,))
        st = gpu.Stream()
        ev0, ev1 = gpu.C.c_void_p(), gpu.C.c_void_p()
        gpu.check(gpu.lib().hy_event_create(gpu.C.byref(ev0)))
        gpu.check(gpu.lib().hy_event_create(gpu.C.byref(ev1)))
        gpu.check(gpu.lib().hy_aux_loss(pb.ptr, cb.ptr, 4096, E, ob.ptr, st.h))
        gpu.check(gpu.lib().hy_event_record(ev0, st.h))
        for _ in range(20):
            gpu.check(gpu.lib().hy_aux_loss(pb.ptr, cb.ptr, 4096, E, ob.ptr, st.h))
        gpu.check(gpu.lib().hy_event_record(ev1, st.h))
        st.synchronize()
        ms = gpu.C.c_float()
        gpu.check(gpu.lib().hy_event_elapsed_ms(ev0, ev1, gpu.C.byref(ms)))
        print(f"\naux_loss T=4096 E=64: {ms.value / 20 * 1e3:.1f} us per call")
        for e in (ev0, ev1):
            gpu.lib().hy_event_destroy(e)
        st.close()
