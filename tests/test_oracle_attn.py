"""Pins of the attention oracle (oracle/hy_oracle_attn.c) against independent
computations: torch's float64 scaled_dot_product_attention / matmul with the rotary
embedding done as complex multiplication, closed forms, and the structure the
reference fixes (causality, GQA head mapping, text / image positions of the 2D
table)."""
import numpy as np
import pytest
import torch

import hy_oracle_attn as A

SHAPE = dict(H=64, nh=4, nkv=2, hd=16)


def _weights(seed, std=0.2):
    return A.synth_weights(SHAPE["H"], SHAPE["nh"], SHAPE["nkv"], SHAPE["hd"], seed=seed, std=std, norm_jitter=0.3)


def _rope_complex(x, pos, theta):
    """x [T][heads][hd] float64, rotated as complex pairs (x[2d] + i x[2d+1]) * e^{i pos f_d}."""
    T, nhd, hd = x.shape
    f = 1.0 / theta ** (np.arange(0, hd, 2, dtype=np.float64) / hd)
    z = x[..., 0::2] + 1j * x[..., 1::2]
    z = z * np.exp(1j * np.outer(pos, f))[:, None, :]
    out = np.empty_like(x)
    out[..., 0::2], out[..., 1::2] = z.real, z.imag
    return out


def _reference_f64(w, x, eps, theta, positions, causal=True):
    T, H = x.shape
    nh, nkv, hd = w.nh, w.nkv, w.hd
    qkv = torch.from_numpy(x.astype(np.float64)) @ torch.from_numpy(w.qkv_w.astype(np.float64)).T
    qkv = qkv.numpy()
    q = qkv[:, :nh * hd].reshape(T, nh, hd)
    k = qkv[:, nh * hd:(nh + nkv) * hd].reshape(T, nkv, hd)
    v = qkv[:, (nh + nkv) * hd:].reshape(T, nkv, hd)
    pos = np.arange(T) if positions is None else np.asarray(positions, np.float64)
    q, k = _rope_complex(q, pos, theta), _rope_complex(k, pos, theta)
    rn = lambda a, wt: a / np.sqrt((a * a).mean(-1, keepdims=True) + eps) * wt.astype(np.float64)
    q, k = rn(q, w.q_norm), rn(k, w.k_norm)
    g = nh // nkv
    qt = torch.from_numpy(q).permute(1, 0, 2)[None]
    kt = torch.from_numpy(np.repeat(k, g, axis=1)).permute(1, 0, 2)[None].contiguous()
    vt = torch.from_numpy(np.repeat(v, g, axis=1)).permute(1, 0, 2)[None].contiguous()
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, is_causal=causal)
    merged = o[0].permute(1, 0, 2).reshape(T, nh * hd)
    out = merged @ torch.from_numpy(w.o_w.astype(np.float64)).T
    return out.numpy(), q, k, v


def _rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


@pytest.mark.parametrize("T,positions", [(1, None), (7, None), (9, [3, 1, 4, 1, 5, 9, 2, 6, 5])])
def test_matches_torch_float64(T, positions):
    w = _weights(seed=T)
    x = np.random.default_rng(100 + T).standard_normal((T, SHAPE["H"])).astype(np.float32)
    out, dq, dk, dv = A.attention_forward(w, x, eps=1e-5, theta=10000.0, positions=positions)
    ref, q, k, v = _reference_f64(w, x, 1e-5, 10000.0, positions)
    assert _rel(out, ref) < 2e-5
    assert _rel(dq, q) < 2e-5 and _rel(dk, k) < 2e-5 and _rel(dv, v) < 2e-5


def test_single_token_returns_its_value_rows():
    """One token attends to itself with weight exactly 1: the merged row is v of the
    head's kv group, and out = o_w @ merged."""
    w = _weights(seed=3)
    x = np.random.default_rng(3).standard_normal((1, SHAPE["H"])).astype(np.float32)
    out, _, _, dv = A.attention_forward(w, x)
    g = SHAPE["nh"] // SHAPE["nkv"]
    merged = np.concatenate([dv[0, h // g] for h in range(SHAPE["nh"])])
    np.testing.assert_allclose(out[0], w.o_w.astype(np.float64) @ merged, rtol=0, atol=2e-6 * np.abs(out).max())


def test_zero_keys_average_the_values():
    """Zero key rows (so every score is 0) give uniform causal weights: token t's
    head output is the mean of v over tokens 0..t."""
    w = _weights(seed=4)
    nh, nkv, hd = w.nh, w.nkv, w.hd
    w.qkv_w[nh * hd:(nh + nkv) * hd] = 0.0
    T = 6
    x = np.random.default_rng(4).standard_normal((T, SHAPE["H"])).astype(np.float32)
    eye = A.AttnWeights(w.qkv_w, np.eye(SHAPE["H"], nh * hd, dtype=np.float32), w.q_norm, w.k_norm, nh, nkv, hd)
    out, _, dk, dv = A.attention_forward(eye, x)
    assert not dk.any()
    g = nh // nkv
    for t in range(T):
        want = np.concatenate([dv[:t + 1, h // g].astype(np.float64).mean(0) for h in range(nh)])
        np.testing.assert_allclose(out[t], want, rtol=1e-6, atol=1e-6)


def test_causal_prefix_unchanged():
    w = _weights(seed=5)
    x = np.random.default_rng(5).standard_normal((8, SHAPE["H"])).astype(np.float32)
    a, *_ = A.attention_forward(w, x)
    x2 = x.copy()
    x2[-1] += 1.0
    b, *_ = A.attention_forward(w, x2)
    np.testing.assert_array_equal(a[:-1], b[:-1])
    assert not np.array_equal(a[-1], b[-1])


def test_rope_identity_at_zero_and_norm_preserving():
    rng = np.random.default_rng(6)
    q = rng.standard_normal((5, 3, 16)).astype(np.float32)
    k = rng.standard_normal((5, 2, 16)).astype(np.float32)
    rq, rk = A.rope_f32(q, k, positions=[0, 0, 0, 0, 0])
    np.testing.assert_array_equal(rq, q)
    np.testing.assert_array_equal(rk, k)
    rq, rk = A.rope_f32(q, k)
    pn = lambda a: np.hypot(a[..., 0::2].astype(np.float64), a[..., 1::2].astype(np.float64))
    np.testing.assert_allclose(pn(rq), pn(q), rtol=2e-6)
    np.testing.assert_array_equal(A.rope_f32(q, k, positions=np.arange(5))[0], rq)


def test_2d_table_text_rows_equal_1d_rope():
    """Text positions use y = x = p, so a text-only table applied by apply_rope_2d
    equals rope_f32 at positions 0..T-1 bit for bit (same cosf / sinf arguments)."""
    rng = np.random.default_rng(7)
    T, hd = 6, 16
    q = rng.standard_normal((T, 4, hd)).astype(np.float32)
    k = rng.standard_normal((T, 2, hd)).astype(np.float32)
    cos, sin = A.build_2d_rope(T, hd, text_len=T, img_h=1, img_w=1)
    a = A.apply_rope_2d(q, k, cos, sin)
    b = A.rope_f32(q, k)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])


def test_2d_table_image_grid_structure():
    """Image tokens: pairs d with (d/2) even follow the row, the others the column,
    offset by beta = text_len + (h*w - h)/2 (rows) or (h*w - w)/2 (columns); each
    pair's value is stored at both of its positions."""
    text, ih, iw, hd = 2, 3, 4, 16
    cos, sin = A.build_2d_rope(text + ih * iw, hd, text, ih, iw)
    th = 1.0 / 10000.0 ** (np.arange(0, hd, 2) / hd)
    by, bx = text + (ih * iw - ih) / 2.0, text + (ih * iw - iw) / 2.0
    for p in range(text, text + ih * iw):
        r, c = divmod(p - text, iw)
        for d in range(hd // 2):
            pos = by + r if (d // 2) % 2 == 0 else bx + c
            assert cos[p, 2 * d] == cos[p, 2 * d + 1] and sin[p, 2 * d] == sin[p, 2 * d + 1]
            assert abs(cos[p, 2 * d] - np.cos(pos * th[d])) < 2e-6 and abs(sin[p, 2 * d] - np.sin(pos * th[d])) < 2e-6
    # a 1x1 image right after no text sits at position 0: the identity rotation
    c1, s1 = A.build_2d_rope(1, hd, 0, 1, 1)
    assert (c1 == 1).all() and (s1 == 0).all()


def test_cache_one_token_at_a_time_matches_causal_forward():
    """Feeding tokens one per call through the KV cache with text-only 2D tables is
    causal attention with 1D rotary positions: it agrees with attention_forward to
    float rounding (the cache branch normalizes as x * (rms * w))."""
    w = _weights(seed=8)
    T = 7
    x = np.random.default_rng(8).standard_normal((T, SHAPE["H"])).astype(np.float32)
    full, *_ = A.attention_forward(w, x)
    cos, sin = A.build_2d_rope(T, w.hd, T, 1, 1)
    cache = A.KVCache(w.nkv, w.hd, max_len=16)
    got = np.stack([A.attention_cached(w, x[t:t + 1], cache, cos=cos[t:t + 1], sin=sin[t:t + 1])[0]
                    for t in range(T)])
    assert cache.cur_len == T
    assert _rel(got, full) < 1e-5


def test_cache_chunk_attends_to_every_position():
    """A multi-token call lets every new token see all cached positions, later new
    tokens included (the reference's cache branch has no mask): the float64
    non-causal attention over prefix + chunk."""
    w = _weights(seed=9)
    x = np.random.default_rng(9).standard_normal((9, SHAPE["H"])).astype(np.float32)
    cache = A.KVCache(w.nkv, w.hd, max_len=9)
    A.attention_cached(w, x[:4], cache)
    got = A.attention_cached(w, x[4:], cache)
    ref, *_ = _reference_f64(w, x, 1e-5, 10000.0, positions=[0] * 9, causal=False)   # no rotation
    assert _rel(got, ref[4:]) < 2e-5
    with pytest.raises(ValueError):
        A.attention_cached(w, x[:1], cache)
