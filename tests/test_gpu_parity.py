"""GPU parity: every kernel of the MoE block through the C ABI against the oracle.

Bars: bit-exact for integer/byte/index work (quantized blocks, int dots, expert
indices, dispatch positions) and for the operations that share a defined order
with the oracle (router logits, RMSNorm, synthetic weights); layer outputs within
normwise max relative error 1e-3 and cosine >= 0.99999 of the oracle's q semantics.
"""
import numpy as np
import pytest

import hy_oracle as O

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3
COS_TOL = 0.99999


def rel_err(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def cosine(a, b):
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def assert_close(got, ref, what=""):
    e, c = rel_err(got, ref), cosine(got, ref)
    assert e <= REL_TOL and c >= COS_TOL, f"{what}: rel_err={e:.3e} cos={c:.8f}"


def assert_exact(got, ref, what=""):
    """Layer outputs: the GPU path evaluates the oracle's q semantics operation for
    operation, so the bar is bit equality (the 1e-3 / 0.99999 check runs first so a
    failure says how far off it is)."""
    assert_close(got, ref, what)
    diff = got.view(np.uint32) != ref.view(np.uint32)
    assert not diff.any(), f"{what}: {int(diff.sum())} of {diff.size} values differ (rel_err={rel_err(got, ref):.2e})"


# ------------------------------------------------------------------ data kernels

def test_synth_fill_bit_exact(gpu):
    for (seed, layer, tensor, expert, std) in [(42, 0, 2, 5, 0.02), (7, 31, 3, 64, 1.0)]:
        got = gpu.synth_fill(100_003, seed, layer, tensor, expert, std)
        ref = O.synth(seed, layer, tensor, expert, (100_003,), std)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_quantize_q8_0_bytes(gpu):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((37, 4096)) * np.exp(rng.standard_normal((37, 1)) * 3)).astype(np.float32)
    x[0, :32] = 0.0                      # all-zero block
    x[1, :32] = np.linspace(-1, 1, 32)   # exact .5 ties after scaling
    x[2, 32:64] = 1e-30                  # subnormal-range scale
    got = gpu.quantize_q8_0(x)
    ref = O.quantize(x, O.Q8_0)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
def test_dequantize_bit_exact(gpu, wtype):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((8, 1024)).astype(np.float32)
    q = O.quantize(x, wtype)
    got = gpu.dequantize(q, wtype, x.size)
    ref = O.dequantize(q, wtype, 1024).ravel()
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def brute_block_dots(wtype, w, x, rows, n):
    """int64 brute force from the raw GGUF bytes: Q8_0 int8 quants; Q4_0 element j in
    the low nibble of byte j, element j + 16 in the high nibble, value nibble - 8."""
    nb = n // 32
    xq = x.reshape(nb, 34)[:, 2:].view(np.int8).astype(np.int64)                  # [nb, 32]
    if wtype == O.Q8_0:
        wq = w.reshape(rows, nb, 34)[:, :, 2:].view(np.int8).astype(np.int64)     # [rows, nb, 32]
    else:
        nib = w.reshape(rows, nb, 18)[:, :, 2:].astype(np.int64)                  # [rows, nb, 16]
        wq = np.concatenate([nib & 0xF, nib >> 4], axis=2) - 8
    return np.einsum("rbj,bj->rb", wq, xq)


@pytest.mark.parametrize("path", [0, 1])
@pytest.mark.parametrize("wtype,rows", [(O.Q8_0, 33), (O.Q4_0, 33), (O.Q8_0, 200), (O.Q4_0, 130)])
def test_block_dots_exact(gpu, wtype, rows, path):
    """Per-block int32 dots of the decode GEMV's VALU routine (path 0) and of the grouped
    GEMM's MFMA operand path (path 1) against int64 brute force.  Extremes: Q8_0
    weights over the full int8 range including -128 and whole blocks of -128 and 127,
    an activation block of -128 and one of 127; Q4_0 blocks of nibble 0x0 (-8) and 0xF
    (7).  Row counts that are not multiples of 64 cover the MFMA path's partial row
    group."""
    rng = np.random.default_rng(2 + rows)
    n = 4096
    nb = n // 32
    w = O.quantize(rng.standard_normal((rows, n)).astype(np.float32), wtype)
    if wtype == O.Q8_0:   # full int8 range incl. -128
        wq = w.reshape(rows, nb, 34)
        wq[:, :, 2:] = rng.integers(0, 256, size=wq[:, :, 2:].shape, dtype=np.uint8)
        wq[0, 1, 2:] = np.uint8(0x80)
        wq[rows - 1, 2, 2:] = np.uint8(0x7F)
    else:
        wq = w.reshape(rows, nb, 18)
        wq[0, 0, 2:] = np.uint8(0x00)
        wq[rows - 1, 1, 2:] = np.uint8(0xFF)
        wq[rows // 2, 0:nb:2, 2:] = np.uint8(0x0F)     # low nibbles 0xF, high 0x0
    w = wq.reshape(rows, -1)
    x = O.quantize(rng.standard_normal((1, n)).astype(np.float32), O.Q8_0)
    xb = x.reshape(nb, 34)
    xb[0, 2:] = np.uint8(0x80)            # a block of -128
    xb[1, 2:] = np.uint8(0x7F)            # a block of 127
    got = gpu.block_dots(wtype, w, x, rows, n, path=path)
    ref = brute_block_dots(wtype, w, x, rows, n)
    assert np.abs(ref).max() <= 32 * 128 * 128
    np.testing.assert_array_equal(got.astype(np.int64), ref)
    if wtype == O.Q8_0:   # a block of -128 against a block of 127
        assert got[0, 1] == 32 * -128 * 127
    else:                 # nibbles 0xF (7) against a block of 127
        assert got[rows - 1, 1] == 32 * 7 * 127
    # the oracle's block dots agree too
    f = O.lib().hyo_block_dots_q8_0_q8_0 if wtype == O.Q8_0 else O.lib().hyo_block_dots_q4_0_q8_0
    for r in (0, rows // 2, rows - 1):
        o = np.zeros(nb, np.int32)
        f(O.vp(np.ascontiguousarray(w[r])), O.vp(x), n, O.ip(o))
        np.testing.assert_array_equal(got[r], o)


def test_block_dots_rejects_bad_path(gpu):
    with pytest.raises(gpu.HyError):
        gpu.block_dots(O.Q8_0, np.zeros((1, 34), np.uint8), np.zeros((1, 34), np.uint8), 1, 32, path=2)


# ------------------------------------------------------------------ routing

@pytest.mark.parametrize("T,H,E,K", [(37, 4096, 64, 8), (5, 256, 16, 4), (1, 4096, 64, 8), (64, 512, 8, 2),
                                   (2, 196, 64, 8), (4, 324, 16, 4), (100, 452, 64, 8), (33, 68, 12, 2),
                                   (512, 4096, 64, 8), (300, 768, 64, 8), (2048, 1024, 64, 8),
                                   (2050, 452, 40, 8)])
def test_router_logits_and_indices_bit_exact(gpu, T, H, E, K):
    x = O.synth(3, 0, O.T_X, 0, (T, H), 1.0)
    wr = O.synth(3, 0, O.T_ROUTER, 0, (E, H), 0.02)
    wr[E // 2] = wr[1]            # identical experts: equal logits, lower index must win
    lg, w, idx = gpu.router_topk(x, wr, K)
    ref_lg = O.router_logits_blocked(x, wr)
    np.testing.assert_array_equal(lg.view(np.uint32), ref_lg.view(np.uint32))
    ref_w, ref_idx = O.route_topk(ref_lg, K)
    np.testing.assert_array_equal(idx, ref_idx)
    np.testing.assert_array_equal(w.view(np.uint32), ref_w.view(np.uint32))


def test_router_scaling_without_norm(gpu):
    T, H, E, K = 9, 256, 16, 4
    x = O.synth(4, 0, O.T_X, 0, (T, H), 1.0)
    wr = O.synth(4, 0, O.T_ROUTER, 0, (E, H), 0.1)
    lg, w, idx = gpu.router_topk(x, wr, K, norm=False, scale=2.5)
    ref_w, ref_idx = O.route_topk(O.router_logits_blocked(x, wr), K, norm=False, scale=2.5)
    np.testing.assert_array_equal(idx, ref_idx)
    np.testing.assert_array_equal(w.view(np.uint32), ref_w.view(np.uint32))


@pytest.mark.parametrize("norm", [0, 1, 2])
def test_router_single_expert_rules(gpu, norm):
    """K = 1: rule 1 (topkgating_full's `norm_topk_prob && K > 1`) keeps p * scale,
    rule 2 (moe_forward_cpu) gives exactly 1, rule 0 scales."""
    T, H, E = 21, 256, 16
    x = O.synth(5, 0, O.T_X, 0, (T, H), 1.0)
    wr = O.synth(5, 0, O.T_ROUTER, 0, (E, H), 0.1)
    lg, w, idx = gpu.router_topk(x, wr, 1, norm=norm, scale=2.5)
    ref_w, ref_idx = O.route_topk(O.router_logits_blocked(x, wr), 1, norm=norm, scale=2.5)
    np.testing.assert_array_equal(idx, ref_idx)
    np.testing.assert_array_equal(w.view(np.uint32), ref_w.view(np.uint32))
    if norm == 2:
        assert np.all(w == 1.0)
    else:
        assert np.all(w < 2.5) and np.all(w > 0)
    ew, eidx = gpu.topkgating_easy(lg, 1)
    np.testing.assert_array_equal(eidx, ref_idx)
    assert np.all(ew == 1.0)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0, O.F32])
@pytest.mark.parametrize("T", [1, 5, 40, 300])
def test_layer_single_expert(gpu, wtype, T):
    """A layer with K = 1 routes with p * routed_scaling_factor (moe_forward_full's
    rule) on the decode and the grouped-GEMM paths."""
    H, I, E = 256, 128, 16
    layer = O.synth_layer(H, I, E, 1, wtype, seed=13, std=0.05)
    layer.routed_scaling_factor = 1.5
    m = gpu.Moe(H, I, E, 1, wtype, max_tokens=512, routed_scaling_factor=1.5)
    m.upload(0, layer)
    x = O.synth(70 + T, 0, O.T_X, 0, (T, H), 1.0)
    out, lg, w, idx = m.run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert np.all(w < 1.5)
    assert_exact(out, ref, f"K=1 wtype={wtype} T={T}")
    m.close()


def test_topkgating_easy_from_logits(gpu):
    """topkgating_easy (reference semantics: glibc expf, sequential softmax sum): the
    GPU selects on logits, so indices match exactly and weights to float rounding."""
    rng = np.random.default_rng(5)
    T, E, K = 50, 64, 8
    lg = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    w, idx = gpu.topkgating_easy(lg, K)
    rw = np.zeros((T, K), np.float32)
    ri = np.zeros((T, K), np.int32)
    O.lib().hyo_topkgating_easy(O.fp(lg), T, E, K, O.fp(rw), O.ip(ri))
    np.testing.assert_array_equal(idx, ri)
    np.testing.assert_allclose(w, rw, rtol=2e-6)


def test_softmax_rows(gpu):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((7, 64)) * 3).astype(np.float32)
    got = gpu.softmax_rows(x)
    ref = x.copy()
    for r in range(7):
        O.lib().hyo_softmax_f32(O.fp(ref[r]), 64)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-9)


def test_rms_norm_bit_exact(gpu):
    T, H = 19, 4096
    x = O.synth(8, 0, O.T_X, 0, (T, H), 1.5)
    got = gpu.rms_norm(x, 1e-5)
    ss = np.array([O.router_logits_blocked(x[t:t + 1], x[t:t + 1])[0, 0] for t in range(T)], np.float32)
    rms = np.float32(1.0) / np.sqrt(ss / np.float32(H) + np.float32(1e-5))
    ref = (x * rms[:, None]).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


# ------------------------------------------------------------------ whole layer

SMALL = dict(H=256, I=128, E=16, K=4)


@pytest.fixture(scope="module")
def small_layers():
    return {wt: O.synth_layer(SMALL["H"], SMALL["I"], SMALL["E"], SMALL["K"], wt, seed=11, std=0.05)
            for wt in (O.Q8_0, O.Q4_0, O.F32)}


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0, O.F32])
@pytest.mark.parametrize("T", [1, 3, 17, 64, 100])
def test_layer_small(gpu, small_layers, wtype, T):
    layer = small_layers[wtype]
    m = gpu.Moe(SMALL["H"], SMALL["I"], SMALL["E"], SMALL["K"], wtype, max_tokens=128)
    m.upload(0, layer)
    x = O.synth(12 + T, 0, O.T_X, 0, (T, SMALL["H"]), 1.0)
    out, lg, w, idx = m.run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
    np.testing.assert_array_equal(lg.view(np.uint32), rlg.view(np.uint32))
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert_exact(out, ref, f"wtype={wtype} T={T}")
    m.close()


# with E=16, K=4 the grouped GEMM tiles 64 pairs up to T=383 and 128 pairs from T=384
DECODE = dict(H=768, I=768, E=64, K=8)


@pytest.fixture(scope="module")
def decode_layers():
    return {wt: O.synth_layer(DECODE["H"], DECODE["I"], DECODE["E"], DECODE["K"], wt, seed=31, std=0.05)
            for wt in (O.Q8_0, O.Q4_0)}


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("T", [2, 4, 5, 8, 9, 16])
def test_decode_batch_routing(gpu, decode_layers, wtype, T):
    """Decode batches of 2-16 tokens route in one selection pass whose work group has
    4, 8 or 16 waves (one per token), then run the ring GEMV (768-wide rows: three or
    more 8-block steps): logits, indices, weights and outputs bit-exact against the
    oracle at the real expert count (64 routed experts, top-8)."""
    H, I, E, K = DECODE["H"], DECODE["I"], DECODE["E"], DECODE["K"]
    layer = decode_layers[wtype]
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=16)
    m.upload(0, layer)
    x = O.synth(300 + T, 0, O.T_X, 0, (T, H), 1.0)
    out, lg, w, idx = m.run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
    np.testing.assert_array_equal(lg.view(np.uint32), rlg.view(np.uint32))
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert_exact(out, ref, f"decode T={T} wtype={wtype}")
    m.close()


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("T", [1, 17, 64, 65, 130, 300, 383, 384, 700])
def test_layer_small_mfma_path(gpu, small_layers, wtype, T):
    layer = small_layers[wtype]
    m = gpu.Moe(SMALL["H"], SMALL["I"], SMALL["E"], SMALL["K"], wtype, max_tokens=1024)
    m.set_path(gpu.PATH_MFMA)
    m.upload(0, layer)
    x = O.synth(50 + T, 0, O.T_X, 0, (T, SMALL["H"]), 1.0)
    out, lg, w, idx = m.run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
    np.testing.assert_array_equal(idx, ridx)
    assert_exact(out, ref, f"mfma wtype={wtype} T={T}")
    # the decode GEMV computes the same operations in the same order
    m.set_path(gpu.PATH_VALU)
    assert_exact(m.run(0, x), ref, f"gemv wtype={wtype} T={T}")
    m.close()


# decode GEMV with the DMA ring: needs a multiple of 8 blocks per row and >= 3 (Q4_0) /
# 2 (Q8_0) steps of 8; the shapes cover ring depth == steps (no steady-state loop) and
# the plain-kernel fallback on one of the two matrices
@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
@pytest.mark.parametrize("H,I,shared", [(768, 768, True), (1024, 640, True), (640, 1536, True),
                                        (512, 1024, True), (1024, 768, False)])
def test_decode_gemv_ring(gpu, wtype, H, I, shared):
    E, K = 16, 4
    layer = O.synth_layer(H, I, E, K, wtype, seed=H + I, std=0.05, shared=shared)
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=16, has_shared=shared)
    m.set_path(gpu.PATH_VALU)
    m.upload(0, layer)
    for T in (1, 2, 5, 8, 16, 3):
        x = O.synth(90 + T, 0, O.T_X, 0, (T, H), 1.0)
        assert_exact(m.run(0, x), O.moe_forward_q(layer, x), f"gemv H={H} I={I} wtype={wtype} T={T}")
    m.close()


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0])
def test_mfma_narrow_hidden(gpu, wtype):
    """H = 128 fits only the 128-row tile shape: small batches must still run on it."""
    H, I, E, K = 128, 128, 8, 2
    layer = O.synth_layer(H, I, E, K, wtype, seed=21, std=0.05)
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=256)
    m.set_path(gpu.PATH_MFMA)
    m.upload(0, layer)
    for T in (5, 40, 256):
        x = O.synth(70 + T, 0, O.T_X, 0, (T, H), 1.0)
        assert_exact(m.run(0, x), O.moe_forward_q(layer, x), f"H=128 wtype={wtype} T={T}")
    m.close()


def test_mfma_path_rejected_for_f32(gpu, small_layers):
    m = gpu.Moe(SMALL["H"], SMALL["I"], SMALL["E"], SMALL["K"], O.F32, max_tokens=8)
    with pytest.raises(gpu.HyError):
        m.set_path(gpu.PATH_MFMA)
    m.close()


def test_skewed_routing_single_hot_expert(gpu, small_layers):
    """All tokens to one expert (capped at T per expert): many tiles of one expert."""
    base = small_layers[O.Q4_0]
    router = base.router.copy()
    router[:, 0] = -50.0
    router[5, 0] = 50.0       # x[:, 0] = 1 -> expert 5 dominates every token
    layer = O.Layer(base.H, base.I, base.E, base.K, O.Q4_0, router, base.shared_gu, base.shared_dn, base.gu, base.dn)
    T = 400
    x = O.synth(60, 0, O.T_X, 0, (T, SMALL["H"]), 1.0)
    x[:, 0] = 1.0
    m = gpu.Moe(SMALL["H"], SMALL["I"], SMALL["E"], SMALL["K"], O.Q4_0, max_tokens=T)
    m.upload(0, layer)
    out, lg, w, idx = m.run(0, x, debug=True)
    ref, rlg, rw, ridx = O.moe_forward_q(layer, x, debug=True)
    assert np.all(idx[:, 0] == 5)
    np.testing.assert_array_equal(idx, ridx)
    assert_exact(out, ref, "hot expert")
    D, counts = m.last_routing()
    assert counts[5] == T and counts.sum() == T * SMALL["K"]
    m.close()


def test_layer_without_shared_expert(gpu, small_layers):
    base = small_layers[O.Q8_0]
    layer = O.Layer(base.H, base.I, base.E, base.K, O.Q8_0, base.router, None, None, base.gu, base.dn)
    m = gpu.Moe(SMALL["H"], SMALL["I"], SMALL["E"], SMALL["K"], O.Q8_0, max_tokens=32, has_shared=False)
    m.upload(0, layer)
    x = O.synth(30, 0, O.T_X, 0, (20, SMALL["H"]), 1.0)
    assert_exact(m.run(0, x), O.moe_forward_q(layer, x), "no shared")
    m.close()


def test_device_synth_equals_host_upload(gpu):
    H, I, E, K = 256, 128, 16, 4
    for wt in (O.Q8_0, O.Q4_0):
        host = O.synth_layer(H, I, E, K, wt, seed=77, layer=3, std=0.02)
        a = gpu.Moe(H, I, E, K, wt, max_tokens=16, num_layers=4)
        a.upload(3, host)
        a.synth(2, seed=77, std=0.02)   # wrong layer index on purpose: different weights
        b = gpu.Moe(H, I, E, K, wt, max_tokens=16, num_layers=4)
        b.synth(3, seed=77, std=0.02)
        x = O.synth(5, 0, O.T_X, 0, (16, H), 1.0)
        ya, yb = a.run(3, x), b.run(3, x)
        np.testing.assert_array_equal(ya.view(np.uint32), yb.view(np.uint32))
        assert not np.array_equal(a.run(2, x), ya)
        a.close()
        b.close()


def test_forward_is_deterministic(gpu, small_layers):
    m = gpu.Moe(SMALL["H"], SMALL["I"], SMALL["E"], SMALL["K"], O.Q4_0, max_tokens=128)
    m.upload(0, small_layers[O.Q4_0])
    x = O.synth(40, 0, O.T_X, 0, (100, SMALL["H"]), 1.0)
    a, b = m.run(0, x), m.run(0, x)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    m.close()


def test_stack_matches_oracle(gpu):
    H, I, E, K, L, T = 256, 128, 16, 4, 3, 24
    layers = [O.synth_layer(H, I, E, K, O.Q8_0, seed=5, layer=l, std=0.05) for l in range(L)]
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=T, num_layers=L)
    for l in range(L):
        m.synth(l, seed=5, std=0.05)
    x = O.synth(6, 0, O.T_X, 0, (T, H), 1.0)
    xb = gpu.Buf.from_array(x)
    ob = gpu.Buf.empty((T, H))
    m.stack_forward(0, L, xb, T, 1e-5, ob)
    got = ob.numpy()
    ref = O.moe_stack_q(layers, x, eps=1e-5)
    assert_exact(got, ref, "stack")
    m.close()


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0, O.F32])
def test_stack_with_norm_weights_matches_oracle(gpu, wtype):
    """The decoder layer's MoE half with per-layer post-attention RMSNorm weights,
    h <- h + MoE(RMSNorm(h) * w_l): quantized weights run the fused RMSNorm + Q8_0
    pass.  Every token regime: decode routing (T <= 16), fused selection (T <= 32),
    the batch path, and both expert paths."""
    H, I, E, K, L = 256, 128, 16, 4, 3
    layers = [O.synth_layer(H, I, E, K, wtype, seed=15, layer=l, std=0.05) for l in range(L)]
    rng = np.random.default_rng(15)
    ws = [rng.standard_normal(H).astype(np.float32), None, (0.5 + rng.random(H)).astype(np.float32)]
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=100, num_layers=L)
    for l in range(L):
        m.synth(l, seed=15, std=0.05)
        m.set_ffn_norm(l, ws[l])
    paths = [gpu.PATH_AUTO] + ([gpu.PATH_VALU, gpu.PATH_MFMA] if wtype != O.F32 else [])
    for T in (1, 3, 24, 100):
        x = O.synth(60 + T, 0, O.T_X, 0, (T, H), 1.0)
        ref = O.moe_stack_qw(layers, ws, x, eps=1e-5)
        xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((T, H))
        for path in paths:
            m.set_path(path)
            m.stack_forward(0, L, xb, T, 1e-5, ob)
            assert_exact(ob.numpy(), ref, f"wtype={wtype} T={T} path={path}")
    m.set_path(gpu.PATH_AUTO)
    for l in range(L):
        m.set_ffn_norm(l, None)
    x = O.synth(7, 0, O.T_X, 0, (40, H), 1.0)
    xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((40, H))
    m.stack_forward(0, L, xb, 40, 1e-5, ob)
    assert_exact(ob.numpy(), O.moe_stack_q(layers, x, eps=1e-5), "unit weight restored")
    with pytest.raises(ValueError):
        m.set_ffn_norm(0, np.ones(H + 1, np.float32))
    m.close()


def test_invalid_token_count_rejected(gpu, small_layers):
    m = gpu.Moe(SMALL["H"], SMALL["I"], SMALL["E"], SMALL["K"], O.Q8_0, max_tokens=8)
    xb = gpu.Buf.empty((16, SMALL["H"]))
    ob = gpu.Buf.empty((16, SMALL["H"]))
    with pytest.raises(gpu.HyError):
        m.forward(0, xb, 4, ob)          # layer not loaded
    m.upload(0, small_layers[O.Q8_0])
    with pytest.raises(gpu.HyError):
        m.forward(0, xb, 16, ob)         # T > max_tokens
    with pytest.raises(gpu.HyError):
        m.forward(0, xb, 0, ob)
    m.close()


@pytest.mark.parametrize("nbytes", [0, 1, 17, 4096, (1 << 20) + 5])
def test_copy_d2d(gpu, nbytes):
    rng = np.random.default_rng(nbytes)
    src = rng.integers(0, 256, size=max(nbytes, 1), dtype=np.uint8)
    a = gpu.Buf.from_array(src)
    b = gpu.Buf.from_array(np.zeros_like(src))
    gpu.check(gpu.lib().hy_copy_d2d(b.ptr, a.ptr, nbytes, None))
    got = b.numpy()
    np.testing.assert_array_equal(got[:nbytes], src[:nbytes])
    assert not got[nbytes:].any()


def _dispatch_expected(idx, E):
    """Counts, offsets and positions of the capacity-slot priority order (k-major,
    then token) by brute force."""
    T, K = idx.shape
    counts = np.bincount(idx.ravel(), minlength=E).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    pos = np.zeros((T, K), np.int32)
    nxt = offsets[:-1].copy()
    for k in range(K):
        for t in range(T):
            e = idx[t, k]
            pos[t, k] = nxt[e]
            nxt[e] += 1
    return counts, offsets, pos


@pytest.mark.parametrize("T,skew", [(1, False), (300, False), (1024, False), (1025, True), (3000, False),
                                    (5000, True)])
def test_dispatch_pairs_multiblock(gpu, T, skew):
    E, K = 64, 8
    rng = np.random.default_rng(T)
    p = np.ones(E) if not skew else 1.0 / np.arange(1, E + 1) ** 1.1
    p /= p.sum()
    idx = np.stack([rng.choice(E, size=K, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, K)).astype(np.float32)
    ib, wb = gpu.Buf.from_array(idx), gpu.Buf.from_array(w)
    cb, ob, pb = gpu.Buf.empty((E,), np.int32), gpu.Buf.empty((E + 1,), np.int32), gpu.Buf.empty((T, K), np.int32)
    gpu.check(gpu.lib().hy_dispatch_pairs(ib.ptr, wb.ptr, T, K, E, cb.ptr, ob.ptr, pb.ptr, None))
    counts, offsets, pos = _dispatch_expected(idx, E)
    np.testing.assert_array_equal(cb.numpy(), counts)
    np.testing.assert_array_equal(ob.numpy(), offsets)
    np.testing.assert_array_equal(pb.numpy(), pos)


def test_layer_mfma_multiblock_dispatch(gpu, small_layers):
    """T > 1024 tokens: the dispatch ranks pairs in several token blocks."""
    layer = small_layers[O.Q8_0]
    T = 2100
    m = gpu.Moe(SMALL["H"], SMALL["I"], SMALL["E"], SMALL["K"], O.Q8_0, max_tokens=T)
    m.upload(0, layer)
    x = O.synth(77, 0, O.T_X, 0, (T, SMALL["H"]), 1.0)
    assert_exact(m.run(0, x), O.moe_forward_q(layer, x), "T=2100")
    m.close()
