"""Known-answer, closed-form and brute-force checks that pin the oracle where no
reference code runs: fp16 conversion, GGUF block codecs, exact int dots, the
synthetic generator, the shared router reduction order, SwiGLU, RMSNorm, and the
q-semantics layer against float64 arithmetic.
"""
import ctypes as C
from fractions import Fraction

import numpy as np
import pytest

import hy_oracle as O

L = None


@pytest.fixture(autouse=True)
def _lib(oracle):
    global L
    L = oracle.lib()


# ------------------------------------------------------------------ fp16

def test_fp16_to_fp32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([L.hyo_fp16_to_fp32(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp32_to_fp16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    vals = [0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e9, np.inf, -np.inf,
            2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 6e-8, 1e-30]
    # every fp16 value, and the midpoints between neighbours (ties)
    f16 = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (f16[:-1] + f16[1:]) / 2
    cand = np.concatenate([np.array(vals), f16[::7], mids[::5], -mids[::11],
                           rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000)])
    x = cand.astype(np.float32)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    got = np.array([L.hyo_fp32_to_fp16(float(v)) for v in x], dtype=np.uint16)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, (x[bad[:5]], got[bad[:5]], ref[bad[:5]])
    assert L.hyo_fp32_to_fp16(float("nan")) & 0x7c00 == 0x7c00


def test_fp16_reference_decoder_flushes_subnormals():
    # src/hunyuan_gguf_loader.cpp:21-32: exponent field 0 -> signed zero
    assert L.hyo_fp16_to_fp32_ref(0x0001) == 0.0
    assert L.hyo_fp16_to_fp32_ref(0x83ff) == 0.0
    assert L.hyo_fp16_to_fp32_ref(0x3c00) == 1.0
    assert L.hyo_fp16_to_fp32_ref(0xc000) == -2.0
    assert L.hyo_fp16_to_fp32_ref(0x7c00) == 65536.0  # no inf: exponent 31 decodes as 2^16
    assert L.hyo_fp16_to_fp32(0x0001) == 2.0 ** -24


# ------------------------------------------------------------------ Q8_0

def test_q8_0_quantize_exact_values():
    d = np.float32(2.0 ** -7)  # exactly representable scale
    k = np.arange(-127, 128, dtype=np.int32)
    k = np.concatenate([k, k[:1]])[:256]
    x = (k.astype(np.float32) * d).astype(np.float32)
    # put 127*d in every block so amax = 127*d and the block scale is exactly d
    x = x.reshape(8, 32)
    x[:, 0] = 127 * d
    q = O.quantize(x, O.Q8_0)
    for b in range(8):
        blk = q[b]
        assert blk[:2].view(np.uint16)[0] == np.float16(d).view(np.uint16)
        np.testing.assert_array_equal(blk[2:].view(np.int8), np.round(x[b] / d).astype(np.int8))


def test_q8_0_roundtrip_bound():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 256)) * np.exp(rng.standard_normal((64, 1)))).astype(np.float32)
    q = O.quantize(x, O.Q8_0)
    y = O.dequantize(q, O.Q8_0, 256)
    amax = np.abs(x.reshape(64, 8, 32)).max(-1, keepdims=True)
    d = amax / 127.0
    err = np.abs((y - x).reshape(64, 8, 32))
    assert np.all(err <= 0.5 * d + 127 * d * 2.0 ** -11 + 1e-30)


def test_q8_0_zero_block():
    q = O.quantize(np.zeros((1, 32), np.float32), O.Q8_0)
    assert np.all(q == 0)


# ------------------------------------------------------------------ Q4_0

def test_q4_0_nibble_table_gguf_vs_reference_loader():
    blk = np.zeros(18, dtype=np.uint8)
    blk[:2] = np.array([np.float16(1.0)]).view(np.uint8)
    blk[2] = 0x80   # GGUF: elem 0 = 0-8 = -8, elem 16 = 8-8 = 0
    blk[3] = 0x0F   # GGUF: elem 1 = 15-8 = 7, elem 17 = 0-8 = -8
    gguf = O.dequantize(blk, O.Q4_0, 32)
    assert gguf[0] == -8 and gguf[16] == 0 and gguf[1] == 7 and gguf[17] == -8
    assert gguf[2] == -8 and gguf[18] == -8  # zero bytes -> -8
    ref = np.zeros(32, np.float32)
    L.hyo_dequantize_row_q4_0_ref(O.vp(blk), O.fp(ref), 32)
    # reference loader: elem i from byte i/2, low nibble for even i, 4-bit sign extension
    assert ref[0] == 0 and ref[1] == -8 and ref[2] == -1 and ref[3] == 0
    assert not np.array_equal(ref, gguf)


def test_q4_0_quantize_extremes_and_roundtrip():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((32, 128)).astype(np.float32)
    q = O.quantize(x, O.Q4_0)
    y = O.dequantize(q, O.Q4_0, 128)
    xb, yb = x.reshape(-1, 32), y.reshape(-1, 32)
    for b in range(xb.shape[0]):
        j = int(np.argmax(np.abs(xb[b])))
        d = abs(float(np.float16(xb[b, j] / -8.0)))
        # the largest-magnitude element is reproduced up to the fp16 scale rounding
        assert abs(yb[b, j] - xb[b, j]) <= 8 * d * 2.0 ** -10 + 1e-7
        assert np.all(np.abs(yb[b] - xb[b]) <= 1.01 * d + 1e-7)


# ------------------------------------------------------------------ int dots

def _blocks_q8(qs, d):
    n = qs.shape[0]
    out = np.zeros((n, 34), np.uint8)
    out[:, :2] = np.asarray(d, np.float16).reshape(n, 1).view(np.uint8)
    out[:, 2:] = qs.astype(np.int8).view(np.uint8)
    return out


def test_int_dot_known_answers():
    a = _blocks_q8(np.full((1, 32), 127), [1.0])
    dots = np.zeros(1, np.int32)
    L.hyo_block_dots_q8_0_q8_0(O.vp(a), O.vp(a), 32, O.ip(dots))
    assert dots[0] == 516128
    m = _blocks_q8(np.full((1, 32), -128), [1.0])
    L.hyo_block_dots_q8_0_q8_0(O.vp(m), O.vp(m), 32, O.ip(dots))
    assert dots[0] == 524288
    alt = _blocks_q8(np.tile([127, -127], 16)[None], [1.0])
    L.hyo_block_dots_q8_0_q8_0(O.vp(alt), O.vp(a), 32, O.ip(dots))
    assert dots[0] == 0


def test_int_dots_brute_force():
    rng = np.random.default_rng(3)
    nb = 257
    w8 = rng.integers(-128, 128, size=(nb, 32))
    x8 = rng.integers(-128, 128, size=(nb, 32))
    wb, xb = _blocks_q8(w8, np.ones(nb)), _blocks_q8(x8, np.ones(nb))
    got = np.zeros(nb, np.int32)
    L.hyo_block_dots_q8_0_q8_0(O.vp(wb), O.vp(xb), nb * 32, O.ip(got))
    np.testing.assert_array_equal(got, (w8.astype(np.int64) * x8).sum(1))
    nib = rng.integers(0, 16, size=(nb, 32))
    w4 = np.zeros((nb, 18), np.uint8)
    w4[:, :2] = np.ones((nb, 1), np.float16).view(np.uint8)
    w4[:, 2:] = (nib[:, :16] | (nib[:, 16:] << 4)).astype(np.uint8)
    L.hyo_block_dots_q4_0_q8_0(O.vp(w4), O.vp(xb), nb * 32, O.ip(got))
    np.testing.assert_array_equal(got, ((nib - 8).astype(np.int64) * x8).sum(1))


def test_vec_dot_scale_accumulation():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 4096)).astype(np.float32)
    w = (rng.standard_normal((1, 4096)) * 0.02).astype(np.float32)
    for wt in (O.Q8_0, O.Q4_0):
        wq, xq = O.quantize(w, wt), O.quantize(x, O.Q8_0)
        f = L.hyo_vec_dot_q8_0_q8_0 if wt == O.Q8_0 else L.hyo_vec_dot_q4_0_q8_0
        got = f(O.vp(wq), O.vp(xq), 4096)
        exact = float(np.dot(O.dequantize(wq, wt, 4096).astype(np.float64)[0],
                             O.dequantize(xq, O.Q8_0, 4096).astype(np.float64)[0]))
        scale = float(np.abs(O.dequantize(wq, wt, 4096)[0] * O.dequantize(xq, O.Q8_0, 4096)[0]).sum())
        assert abs(got - exact) <= 1e-6 * scale


# ------------------------------------------------------------------ synthetic generator

def _mix64(z):
    M = (1 << 64) - 1
    z = (z + 0x9E3779B97F4A7C15) & M
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return z ^ (z >> 31)


def test_synth_generator_definition_and_moments():
    seed, layer, tensor, expert = 42, 3, 2, 17
    key = _mix64(_mix64(seed) ^ ((layer << 40) | (tensor << 24) | expert))
    assert L.hyo_stream_key(seed, layer, tensor, expert) == key
    scale = np.float32(0.02) * np.float32(2.6428990e-05)
    got = O.synth(seed, layer, tensor, expert, (3000,), 0.02, idx0=12345)
    for i in range(0, 3000, 97):
        r = _mix64(key ^ (((12345 + i) * 0xD1B54A32D192ED03) & ((1 << 64) - 1)))
        s = sum((r >> (16 * j)) & 0xFFFF for j in range(4)) - 131070
        assert got[i] == np.float32(np.float32(s) * scale)
    big = O.synth(7, 0, 0, 0, (1 << 20,), 1.0)
    assert abs(big.mean()) < 5e-3 and abs(big.std() - 1.0) < 5e-3


# ------------------------------------------------------------------ shared exp

def test_expf_accuracy_and_specials():
    L.hyo_expf.restype = C.c_float
    L.hyo_expf.argtypes = [C.c_float]
    rng = np.random.default_rng(11)
    xs = np.concatenate([rng.uniform(-100, 88, 20000), rng.uniform(-1, 1, 5000), np.arange(-87, 88, 0.25)])
    xs = xs.astype(np.float32)
    got = np.array([L.hyo_expf(float(v)) for v in xs], np.float32)
    ref = np.exp(xs.astype(np.float64))
    normal = ref > 1.2e-38
    ulp = np.spacing(ref[normal].astype(np.float32)).astype(np.float64)
    err_ulp = np.abs(got[normal].astype(np.float64) - ref[normal]) / ulp
    assert err_ulp.max() <= 2.0, err_ulp.max()
    assert L.hyo_expf(0.0) == 1.0
    assert L.hyo_expf(89.0) == np.inf and L.hyo_expf(-104.0) == 0.0
    assert np.isnan(L.hyo_expf(float("nan")))
    # subnormal results stay close in absolute terms
    sub = ~normal & (ref > 0)
    assert np.all(np.abs(got[sub] - ref[sub]) <= 2 * 1.4e-45)


# ------------------------------------------------------------------ router order

def _f32_round(q: Fraction) -> np.float32:
    """Exact rational -> float32, round to nearest even (normal range only)."""
    if q == 0:
        return np.float32(0.0)
    s = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    scaled = a / Fraction(2) ** (e - 23)  # in [2^23, 2^24)
    m = scaled.numerator // scaled.denominator
    rem = scaled - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    return np.float32(s * float(Fraction(m) * Fraction(2) ** (e - 23)))


def _blocked_dot_exact(a, b):
    p = [np.float32(0.0)] * 64
    for h0 in range(0, len(a), 4):
        l = (h0 // 4) % 64
        for c in range(4):
            p[l] = _f32_round(Fraction(float(a[h0 + c])) * Fraction(float(b[h0 + c])) + Fraction(float(p[l])))
    s = 32
    while s >= 1:
        for l in range(s):
            p[l] = np.float32(p[l] + p[l + s])
        s //= 2
    return p[0]


def test_router_blocked_order_bit_exact():
    rng = np.random.default_rng(6)
    H, E, T = 512, 3, 2
    x = rng.standard_normal((T, H)).astype(np.float32)
    wr = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    got = O.router_logits_blocked(x, wr)
    for t in range(T):
        for e in range(E):
            assert got[t, e] == _blocked_dot_exact(x[t], wr[e]), (t, e)
    # and the sequential reference order differs from it somewhere (order matters)
    seq = np.zeros((T, E), np.float32)
    L.hyo_router_logits_seq(O.fp(x), O.fp(wr), T, H, E, O.fp(seq))
    np.testing.assert_allclose(seq, got, rtol=0, atol=1e-5)


def test_route_topk_known_answers():
    E, K = 64, 8
    w, idx = O.route_topk(np.zeros((1, E), np.float32), K)
    np.testing.assert_array_equal(idx[0], np.arange(K))
    np.testing.assert_allclose(w[0], 1.0 / K, rtol=1e-6)
    lg = np.zeros((1, E), np.float32)
    lg[0, :7] = 5.0
    lg[0, [20, 9, 40]] = 1.0   # three-way tie for the 8th slot
    w, idx = O.route_topk(lg, K)
    assert list(idx[0]) == [0, 1, 2, 3, 4, 5, 6, 9]
    lg = np.zeros((1, E), np.float32)
    lg[0, 37] = 100.0
    w, idx = O.route_topk(lg, K)
    assert idx[0, 0] == 37 and abs(w[0, 0] - 1.0) < 1e-6 and np.all(w[0, 1:] < 1e-40)
    # descending ramp with duplicates: stable descending sort order
    rng = np.random.default_rng(7)
    for _ in range(50):
        lg = (rng.integers(-4, 5, size=(1, E)) * 0.5).astype(np.float32)
        w, idx = O.route_topk(lg, K)
        order = np.argsort(-lg[0], kind="stable")[:K]
        np.testing.assert_array_equal(idx[0], order)
        p = np.exp(lg[0].astype(np.float64) - lg[0].max())
        np.testing.assert_allclose(w[0], p[order] / p[order].sum(), rtol=2e-6)


def test_route_topk_single_expert_rules():
    """K = 1.  Rule 1 (topkgating_full, src/hunyuan_moe_full.cpp:230: `norm_topk_prob &&
    K > 1`) keeps the softmax probability times the scale; rule 2 (moe_forward_cpu,
    src/attention.cpp:268-275) renormalises it to exactly 1; rule 0 scales.  The
    probabilities are checked against float64 softmax, the index against argmax with
    the lower index winning ties."""
    rng = np.random.default_rng(11)
    for E in (1, 8, 64):
        lg = (rng.standard_normal((40, E)) * 1.5).astype(np.float32)
        lg[:5] = np.round(lg[:5])               # ties for the top slot
        order = np.argmax(lg, axis=1)          # first (lowest) index of the maximum
        p = np.exp(lg.astype(np.float64) - lg.max(axis=1, keepdims=True))
        p = p[np.arange(40), order] / p.sum(axis=1)
        for scale in (1.0, 2.5):
            w1, i1 = O.route_topk(lg, 1, norm=1, scale=scale)
            w0, i0 = O.route_topk(lg, 1, norm=0, scale=scale)
            np.testing.assert_array_equal(i1[:, 0], order)
            np.testing.assert_array_equal(i0, i1)
            np.testing.assert_array_equal(w1.view(np.uint32), w0.view(np.uint32))
            np.testing.assert_allclose(w1[:, 0], scale * p, rtol=2e-6)
        w2, i2 = O.route_topk(lg, 1, norm=2, scale=2.5)
        np.testing.assert_array_equal(i2[:, 0], order)
        assert np.all(w2 == 1.0)
    # K > 1: rules 1 and 2 agree
    lg = (rng.standard_normal((20, 16)) * 1.5).astype(np.float32)
    a = O.route_topk(lg, 4, norm=1)
    b = O.route_topk(lg, 4, norm=2)
    np.testing.assert_array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
    np.testing.assert_array_equal(a[1], b[1])


# ------------------------------------------------------------------ SwiGLU / RMSNorm

def test_swiglu_closed_form():
    H = I = 4
    a = 3.0
    gu = np.zeros((2 * I, H), np.float32)
    gu[:I] = np.eye(I) * a
    gu[I:] = np.eye(I)
    dn = np.eye(H, dtype=np.float32)
    x = np.array([[0.0, 1.0, -2.0, 30.0], [0.5, -0.5, 8.0, -8.0]], np.float32)
    out = np.zeros_like(x)
    L.hyo_swiglu_ffn_f32(O.fp(x), O.fp(gu), O.fp(dn), O.fp(out), 2, H, I)
    g = a * x.astype(np.float64)
    ref = g / (1 + np.exp(-g)) * x
    np.testing.assert_allclose(out, ref, rtol=1e-6, atol=1e-7)
    assert out[0, 0] == 0.0                        # silu(0) = 0
    assert abs(out[0, 3] - 90.0 * 30.0) < 1e-2     # silu(g) -> g for large g
    # silu on the FIRST half: swapping halves changes the answer
    sw = np.concatenate([gu[I:], gu[:I]])
    out2 = np.zeros_like(x)
    L.hyo_swiglu_ffn_f32(O.fp(x), O.fp(sw), O.fp(dn), O.fp(out2), 2, H, I)
    assert not np.allclose(out, out2)


def test_rms_norm_closed_form():
    x = np.array([[3.0, 4.0, 0.0, 0.0]], np.float32)
    w = np.array([1.0, 2.0, 1.0, 1.0], np.float32)
    out = np.zeros_like(x)
    L.hyo_rms_norm_f32(O.fp(x), O.fp(w), O.fp(out), 1, 4, 0.0)
    np.testing.assert_allclose(out[0], [3 / 2.5, 2 * 4 / 2.5, 0, 0], rtol=1e-6)


# ------------------------------------------------------------------ whole-layer brute force

def _ref64_moe(x, wr, gu, dn, sgu, sdn, K):
    x = x.astype(np.float64)
    lg = x @ wr.astype(np.float64).T
    p = np.exp(lg - lg.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    out = np.zeros_like(x)
    I = gu.shape[1] // 2

    def ffn(xx, g_u, d):
        t = xx @ g_u.astype(np.float64).T
        g, u = t[..., :I], t[..., I:]
        return (g / (1 + np.exp(-g)) * u) @ d.astype(np.float64).T

    for t in range(x.shape[0]):
        order = np.argsort(-p[t], kind="stable")[:K]
        wts = p[t, order] / p[t, order].sum()
        for e, wt in zip(order, wts):
            out[t] += wt * ffn(x[t], gu[e], dn[e])
    if sgu is not None:
        out += ffn(x, sgu, sdn)
    return out


def test_moe_forward_full_and_twin_vs_float64():
    T, H, I, E, K = 6, 64, 32, 8, 2
    seed = 21
    x = O.synth(seed, 0, O.T_X, 0, (T, H), 1.0)
    wr = O.synth(seed, 0, O.T_ROUTER, 0, (E, H), 0.3)
    gu = O.synth(seed, 0, O.T_GU, 0, (E, 2 * I, H), 0.1)
    dn = O.synth(seed, 0, O.T_DN, 0, (E, H, I), 0.1)
    sgu = O.synth(seed, 0, O.T_GU, E, (2 * I, H), 0.1)
    sdn = O.synth(seed, 0, O.T_DN, E, (H, I), 0.1)
    ref = _ref64_moe(x, wr, gu, dn, sgu, sdn, K)
    full = np.zeros((T, H), np.float32)
    cfg = O.default_cfg(E, K)
    assert L.hyo_moe_forward_full(O.fp(x), T, H, O.fp(wr), O.fp(sgu), O.fp(sdn), O.fp(gu), O.fp(dn),
                                  E, I, C.byref(cfg), O.fp(full)) == 0
    twin = np.zeros((T, H), np.float32)
    probs = np.zeros((T, E), np.float32)
    tw = np.zeros((T, K), np.float32)
    ti = np.zeros((T, K), np.int32)
    assert L.hyo_moe_forward_cpu(O.fp(x), O.fp(wr), O.fp(sgu), O.fp(sdn), O.fp(gu), O.fp(dn),
                                 T, H, E, I, K, O.fp(twin), O.fp(probs), O.fp(tw), O.ip(ti)) == 0
    scale = np.abs(ref).max()
    assert np.abs(full - ref).max() <= 1e-5 * scale
    assert np.abs(twin - ref).max() <= 1e-5 * scale
    np.testing.assert_allclose(probs.sum(1), 1.0, rtol=1e-5)


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0, O.F32])
def test_q_layer_vs_float64(wtype):
    """q semantics == float64 arithmetic on the dequantized operands (exact block dots)."""
    T, H, I, E, K = 5, 128, 64, 8, 2
    layer = O.synth_layer(H, I, E, K, wtype, seed=9, std=0.05)
    x = O.synth(9, 0, O.T_X, 0, (T, H), 1.0)
    out, lg, w, idx = O.moe_forward_q(layer, x, debug=True)
    np.testing.assert_array_equal(lg, O.router_logits_blocked(x, layer.router))
    w2, idx2 = O.route_topk(lg, K)
    np.testing.assert_array_equal(idx, idx2)
    np.testing.assert_array_equal(w, w2)
    gu, dn, sgu, sdn = layer.dequant()

    def act(v):  # the activation as the layer's dot sees it
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
            ref[t] += w[t, k] * ffn(x[t], gu[idx[t, k]], dn[idx[t, k]])
        ref[t] += ffn(x[t], sgu, sdn)
    err = np.abs(out - ref).max() / np.abs(ref).max()
    assert err < 2e-4, err


def test_q_stack_is_composition():
    T, H, I, E, K = 4, 64, 32, 8, 2
    layers = [O.synth_layer(H, I, E, K, O.Q8_0, seed=3, layer=l, std=0.05) for l in range(3)]
    x = O.synth(3, 0, O.T_X, 0, (T, H), 1.0)
    got = O.moe_stack_q(layers, x, eps=1e-5)
    cur = x.copy()
    for lyr in layers:
        ss = O.router_logits_blocked(cur, cur)[np.arange(T), np.arange(T)]  # blocked sum of squares
        rms = (np.float32(1.0) / np.sqrt(ss / np.float32(H) + np.float32(1e-5))).astype(np.float32)
        xn = (cur * rms[:, None]).astype(np.float32)
        cur = (cur + O.moe_forward_q(lyr, xn)).astype(np.float32)
    np.testing.assert_array_equal(got, cur)


def test_blocked_rms_norm_weight_properties():
    """The weighted blocked RMSNorm: unit weight and w = 1 agree bit for bit; a
    power-of-two weight scales the output exactly; a constant row has the closed form
    c / sqrt(c^2 + eps) * w; and it stays within float rounding of the reference's
    sequential-order rms_norm_f32 (src/rms_norm.cpp:9-33)."""
    rng = np.random.default_rng(11)
    T, H = 5, 4096
    x = rng.standard_normal((T, H)).astype(np.float32) * 3
    unit = O.rms_norm_blocked(x)
    np.testing.assert_array_equal(O.rms_norm_blocked(x, np.ones(H, np.float32)), unit)
    pw = np.exp2(rng.integers(-3, 4, size=H)).astype(np.float32)
    np.testing.assert_array_equal(O.rms_norm_blocked(x, pw), unit * pw)
    w = rng.standard_normal(H).astype(np.float32)
    got = O.rms_norm_blocked(x, w, eps=1e-5)
    np.testing.assert_array_equal(got, (unit * w).astype(np.float32))
    ref = np.empty_like(x)
    L = O.lib()
    L.hyo_rms_norm_f32(O.fp(x), O.fp(w), O.fp(ref), T, H, np.float32(1e-5))
    assert np.abs(got - ref).max() / np.abs(ref).max() < 2e-6
    c = np.full((1, 64), 2.0, np.float32)   # sum of squares 256 is exact in any order
    want = np.float32(2.0) * (np.float32(1.0) / np.sqrt(np.float32(4.0) + np.float32(1e-5)))
    np.testing.assert_array_equal(O.rms_norm_blocked(c, eps=1e-5)[0], np.full(64, want, np.float32))


def test_q_stack_with_norm_weights_is_composition():
    """h <- h + MoE(RMSNorm(h) * w_l) per layer (src/decoder_layer.cpp:33-42), built
    from the layer forward and the blocked RMSNorm; None weights give the unit stack."""
    T, H, I, E, K = 4, 64, 32, 8, 2
    layers = [O.synth_layer(H, I, E, K, O.Q4_0, seed=9, layer=l, std=0.05) for l in range(3)]
    rng = np.random.default_rng(4)
    ws = [rng.standard_normal(H).astype(np.float32), None, 0.5 + rng.random(H).astype(np.float32)]
    x = O.synth(9, 0, O.T_X, 0, (T, H), 1.0)
    got = O.moe_stack_qw(layers, ws, x, eps=1e-5)
    cur = x.copy()
    for lyr, w in zip(layers, ws):
        cur = (cur + O.moe_forward_q(lyr, O.rms_norm_blocked(cur, w, eps=1e-5))).astype(np.float32)
    np.testing.assert_array_equal(got, cur)
    np.testing.assert_array_equal(O.moe_stack_qw(layers, [None] * 3, x), O.moe_stack_q(layers, x))


def test_rows_match_full_layer():
    T, H, I, E, K = 9, 64, 32, 8, 3
    layer = O.synth_layer(H, I, E, K, O.Q4_0, seed=5, std=0.05)
    x = O.synth(5, 0, O.T_X, 0, (T, H), 1.0)
    full = O.moe_forward_q(layer, x, nthreads=2)
    rows = np.array([8, 0, 3])
    np.testing.assert_array_equal(O.moe_forward_q_rows(layer, x, rows), full[rows])
