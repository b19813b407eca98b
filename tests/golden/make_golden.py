"""Writes the golden fixtures under tests/golden/ from the reference's own code.

Runs the reference's hunyuan_moe_full.cpp, compiled unmodified into
oracle/_ref/libhy_ref.so by `make -C oracle ref`, on seeded inputs and stores the
inputs and outputs as small .npz files.  The fixtures are data only; the tests
compare the oracle against them wherever the reference build is not at hand.

    make -C oracle all ref && python tests/golden/make_golden.py
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import hy_oracle as O  # noqa: E402


def ref_gating_full(R, logits, cfg):
    T, E = logits.shape
    bound = R.ref_capacity_bound(T, C.byref(cfg))
    mask = np.zeros(T * E * bound, dtype=np.uint8)
    cw = np.zeros(T * E * bound, dtype=np.float32)
    counts = np.zeros(E, dtype=np.int32)
    probs = np.zeros((T, E), dtype=np.float32)
    cap = C.c_uint32()
    aux = C.c_float()
    rate = C.c_float()
    R.ref_topkgating_full(O.fp(logits), T, C.byref(cfg), O.vp(mask), O.fp(cw), O.ip(counts), O.fp(probs),
                          C.byref(cap), C.byref(aux), C.byref(rate))
    n = T * E * cap.value
    return dict(mask=mask[:n].reshape(T, E, cap.value), cw=cw[:n].reshape(T, E, cap.value), counts=counts,
                probs=probs, capacity=np.uint32(cap.value), aux=np.float32(aux.value),
                rate=np.float32(rate.value))


MOE_CASES = [
    # name, T, H, I, E, K, seed
    ("a", 5, 64, 32, 8, 2, 7),
    ("b", 9, 128, 64, 16, 4, 8),
    # K = 1: topkgating_full keeps p * routed_scaling_factor (no renormalisation)
    ("c", 6, 64, 32, 8, 1, 9),
]


def moe_case_inputs(T, H, I, E, seed):
    """x ~ N(0,1), router ~ N(0,0.2), experts ~ N(0,0.05) from the seeded generator."""
    x = O.synth(seed, 0, O.T_X, 0, (T, H), 1.0)
    wr = O.synth(seed, 0, O.T_ROUTER, 0, (E, H), 0.2)
    gu = O.synth(seed, 0, O.T_GU, 0, (E, 2 * I, H), 0.05)
    dn = O.synth(seed, 0, O.T_DN, 0, (E, H, I), 0.05)
    return x, wr, gu, dn


GATING_CASES = [
    # name, T, E, K, cfg overrides
    ("default_t17_e16_k4", 17, 16, 4, {}),
    ("default_t33_e64_k8", 33, 64, 8, {}),
    ("drop_t40_e16_k4", 40, 16, 4, dict(drop_tokens=1, capacity_factor=1.0, min_capacity=2)),
    ("group_t9_e16_k4", 9, 16, 4, dict(group_limited_greedy=1, n_group=4, topk_group=2)),
    ("nonorm_t6_e8_k2", 6, 8, 2, dict(norm_topk_prob=0, routed_scaling_factor=2.5)),
    ("aux_t12_e8_k3", 12, 8, 3, dict(compute_aux_loss=1)),
    # K = 1: easy gating renormalises (weight 1), full gating keeps p * scale
    # (src/hunyuan_moe_full.cpp:230 `norm_topk_prob && K > 1`)
    ("default_t11_e16_k1", 11, 16, 1, {}),
    ("scaled_t7_e8_k1", 7, 8, 1, dict(routed_scaling_factor=2.5)),
    ("nonorm_t5_e64_k1", 5, 64, 1, dict(norm_topk_prob=0, routed_scaling_factor=0.75)),
]


def logits_with_ties(rng, T, E):
    # coarse values so equal logits (and equal probabilities) occur often
    return (rng.integers(-6, 7, size=(T, E)).astype(np.float32) * 0.5)


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libhy_ref.so missing: run `make -C oracle ref` first")
    R = O.ref()
    rng = np.random.default_rng(42)

    # ---- routing: softmax / topk / easy / full
    routing = {}
    for name, T, E, K, kw in GATING_CASES:
        for kind in ("gauss", "ties"):
            lg = (rng.standard_normal((T, E)).astype(np.float32) * 1.5 if kind == "gauss"
                  else logits_with_ties(rng, T, E))
            key = f"{name}_{kind}"
            routing[f"{key}/logits"] = lg
            w = np.zeros((T, K), dtype=np.float32)
            idx = np.zeros((T, K), dtype=np.int32)
            R.ref_topkgating_easy(O.fp(lg), T, E, K, O.fp(w), O.ip(idx))
            routing[f"{key}/easy_w"] = w
            routing[f"{key}/easy_idx"] = idx
            cfg = O.default_cfg(E, K, **kw)
            g = ref_gating_full(R, lg, cfg)
            for k, v in g.items():
                routing[f"{key}/full_{k}"] = v
            sm = lg[0].copy()
            R.ref_softmax_f32(O.fp(sm), E)
            routing[f"{key}/softmax0"] = sm
    np.savez_compressed(os.path.join(HERE, "ref_routing.npz"), **routing)

    # ---- src/test_components.cpp:88-115 inputs: srand(42), rand()/RAND_MAX*10-5
    libc = C.CDLL(None)
    libc.srand(42)
    RAND_MAX = 2147483647
    lg = np.array([np.float32(libc.rand()) / np.float32(RAND_MAX) for _ in range(4 * 64)], dtype=np.float32)
    lg = (lg * np.float32(10) - np.float32(5)).astype(np.float32).reshape(4, 64)
    w = np.zeros((4, 8), dtype=np.float32)
    idx = np.zeros((4, 8), dtype=np.int32)
    R.ref_topkgating_easy(O.fp(lg), 4, 64, 8, O.fp(w), O.ip(idx))
    g = ref_gating_full(R, lg, O.default_cfg(64, 8))
    np.savez_compressed(os.path.join(HERE, "ref_test_components.npz"), logits=lg, easy_w=w, easy_idx=idx,
                        **{f"full_{k}": v for k, v in g.items()})

    # ---- dispatch / combine
    T, H, E, Cc = 7, 40, 5, 3
    x = rng.standard_normal((T, H)).astype(np.float32)
    mask = (rng.random((T, E, Cc)) < 0.3).astype(np.uint8)
    disp = np.zeros((E, Cc, H), dtype=np.float32)
    R.ref_einsum_dispatch(O.fp(x), T, H, O.vp(mask), E, Cc, O.fp(disp))
    cw = (rng.standard_normal((T, E, Cc)).astype(np.float32) * mask).astype(np.float32)
    eo = rng.standard_normal((E, Cc, H)).astype(np.float32)
    comb = np.zeros((T, H), dtype=np.float32)
    R.ref_einsum_combine(O.fp(cw), O.fp(eo), T, H, E, Cc, O.fp(comb))
    np.savez_compressed(os.path.join(HERE, "ref_einsum.npz"), x=x, mask=mask, disp=disp, cw=cw, eo=eo,
                        comb=comb)

    # ---- moe_forward_full (no shared expert): inputs from the oracle's seeded
    # generator (regenerated by the test), outputs from the reference
    moe = {}
    for name, T, H, I, E, K, seed in MOE_CASES:
        x, wr, gu, dn = moe_case_inputs(T, H, I, E, seed)
        out = np.zeros((T, H), dtype=np.float32)
        cfg = O.default_cfg(E, K)
        R.ref_moe_forward_full_noshared(O.fp(x), T, H, O.fp(wr), O.fp(gu), O.fp(dn), E, I, C.byref(cfg),
                                        O.fp(out))
        moe[f"{name}/out"] = out
        moe[f"{name}/dims"] = np.array([T, H, I, E, K, seed], dtype=np.int64)
    np.savez_compressed(os.path.join(HERE, "ref_moe_full.npz"), **moe)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
