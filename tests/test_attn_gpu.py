"""GPU attention (include/hy_attn.h) against the attention oracle
(oracle/hy_oracle_attn.c, the reference's fp32 algorithm).

The GPU computes the same fp32 mathematics in other summation orders (MFMA tiles,
online softmax), so the bar is a float tolerance, stated here: normwise relative error
max|a-b| / max|b| <= 1e-4 (ten times tighter than the 1e-3 the layer outputs are held
to) and cosine similarity >= 0.99999."""
import numpy as np
import pytest

import hy_oracle_attn as A

pytestmark = pytest.mark.gpu

TOL = 1e-4


def check(got, ref, what):
    got, ref = got.astype(np.float64).ravel(), ref.astype(np.float64).ravel()
    err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-30)
    cos = got @ ref / (np.linalg.norm(got) * np.linalg.norm(ref) + 1e-300)
    assert err <= TOL and cos >= 0.99999, f"{what}: rel_err={err:.3e} cos={cos:.8f}"


SHAPES = [dict(H=256, nh=8, nkv=2, hd=64), dict(H=512, nh=4, nkv=1, hd=128)]


def _ctx(gpu, shp, max_tokens=128, max_cache=0, seed=0):
    w = A.synth_weights(shp["H"], shp["nh"], shp["nkv"], shp["hd"], seed=seed, std=0.05, norm_jitter=0.2)
    m = gpu.Attn(shp["H"], shp["nh"], shp["nkv"], shp["hd"], max_tokens, max_cache=max_cache)
    m.upload(w.qkv_w, w.o_w, w.q_norm, w.k_norm)
    return m, w


@pytest.mark.parametrize("shp", SHAPES, ids=["hd64", "hd128"])
@pytest.mark.parametrize("T", [1, 5, 32, 33, 100])
def test_forward_matches_oracle(gpu, shp, T):
    m, w = _ctx(gpu, shp, seed=T)
    rng = np.random.default_rng(T)
    x = rng.standard_normal((T, shp["H"])).astype(np.float32)
    for positions in (None, rng.integers(0, 3 * T + 5, size=T).astype(np.int32)):
        out, dq, dk, dv = m.run(x, positions=positions, debug=True)
        ref, rq, rk, rv = A.attention_forward(w, x, positions=positions)
        tag = f"T={T} hd={shp['hd']} positions={'given' if positions is not None else 'none'}"
        check(dq, rq, tag + " q")
        check(dk, rk, tag + " k")
        check(dv, rv, tag + " v")
        check(out, ref, tag + " out")
    m.close()


def test_forward_full_head_shape(gpu):
    """HunyuanImage-3's attention shape (hidden 4096, 32 query / 8 kv heads of 128)
    at 64 tokens."""
    shp = dict(H=4096, nh=32, nkv=8, hd=128)
    m, w = _ctx(gpu, shp, max_tokens=64, seed=3)
    x = np.random.default_rng(3).standard_normal((64, 4096)).astype(np.float32)
    out = m.run(x)
    ref, *_ = A.attention_forward(w, x)
    check(out, ref, "full shape")
    m.close()


def _attn64(q, k, v, nh, nkv, causal=True, q_pos0=0):
    """float64 GQA attention of given q [T][nh][hd], k / v [L][nkv][hd] -> [T][nh*hd]."""
    T, _, hd = q.shape
    L = k.shape[0]
    out = np.empty((T, nh, hd))
    for hh in range(nh):
        g = hh // (nh // nkv)
        s = q[:, hh, :].astype(np.float64) @ k[:, g, :].astype(np.float64).T / np.sqrt(hd)
        if causal:
            s = np.where(np.arange(L)[None, :] <= q_pos0 + np.arange(T)[:, None], s, -np.inf)
        s = np.exp(s - s.max(1, keepdims=True))
        out[:, hh, :] = (s / s.sum(1, keepdims=True)) @ v[:, g, :].astype(np.float64)
    return out.reshape(T, nh * hd)


@pytest.mark.parametrize("T", [1024, 2048])
def test_flash_split_and_whole_tiles(gpu, T):
    """32 query / 8 kv heads: T=1024 runs the split over the keys (chunks of 8 key
    blocks per query tile, merged in chunk order); T=2048 fills 512 work groups and
    runs whole tiles.  The output against float64 attention of the device's own q / k /
    v followed by the output projection."""
    shp = dict(H=256, nh=32, nkv=8, hd=64)
    m, w = _ctx(gpu, shp, max_tokens=T, seed=T)
    x = np.random.default_rng(T).standard_normal((T, shp["H"])).astype(np.float32)
    out, dq, dk, dv = m.run(x, debug=True)
    q = dq.reshape(T, 32, 64)
    k, v = dk.reshape(T, 8, 64), dv.reshape(T, 8, 64)
    ref = _attn64(q, k, v, 32, 8) @ w.o_w.astype(np.float64).T
    check(out, ref, f"flash T={T}")
    m.close()


def test_cached_decode_long_cache(gpu):
    """Decode against a long cache (one query tile per kv group: the keys are split
    into chunks of one block): 2 900 cached positions, then chunks of 1 and 4 tokens."""
    shp = SHAPES[0]
    m, w = _ctx(gpu, shp, max_tokens=2900, max_cache=2910, seed=5)
    cache = A.KVCache(shp["nkv"], shp["hd"], max_len=2910)
    rng = np.random.default_rng(5)
    for n in (2900, 1, 4):
        x = rng.standard_normal((n, shp["H"])).astype(np.float32)
        xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((n, shp["H"]))
        m.forward_cached(xb, n, ob)
        ref = A.attention_cached(w, x, cache)
        check(ob.numpy(), ref, f"cached +{n} at {cache.cur_len - n}")
    m.close()


@pytest.mark.parametrize("shp", SHAPES, ids=["hd64", "hd128"])
@pytest.mark.parametrize("waves", [0, 7, 1])
def test_cached_decode_waves(gpu, shp, waves):
    """Decode (1..8 new tokens: the row-packed decode kernel and its merge) against a
    cache of 700 positions, with the waves uncapped (one 32-key block each), capped at 7
    (several blocks a wave, the last wave's range ragged) and at 1 (the whole cache in
    one wave, nothing to join)."""
    m, w = _ctx(gpu, shp, max_tokens=700, max_cache=760, seed=7)
    m.set_decode_waves(waves)
    cache = A.KVCache(shp["nkv"], shp["hd"], max_len=760)
    rng = np.random.default_rng(7)
    for n in (700, 1, 2, 3, 8, 5):
        x = rng.standard_normal((n, shp["H"])).astype(np.float32)
        xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((n, shp["H"]))
        m.forward_cached(xb, n, ob)
        ref = A.attention_cached(w, x, cache)
        check(ob.numpy(), ref, f"cached +{n} at {cache.cur_len - n} waves={waves}")
    m.close()


def test_cached_decode_full_head_shape(gpu):
    """Decode at HunyuanImage-3's head shape (32 query / 8 kv heads of 128; hidden 256
    keeps the oracle's projections short): 1, 4, 5 and 8 new tokens (both decode tiles)
    against 520 cached positions, each kv group's keys over many waves."""
    shp = dict(H=256, nh=32, nkv=8, hd=128)
    m, w = _ctx(gpu, shp, max_tokens=520, max_cache=560, seed=9)
    cache = A.KVCache(shp["nkv"], shp["hd"], max_len=560)
    rng = np.random.default_rng(9)
    for n in (520, 1, 4, 5, 8):
        x = rng.standard_normal((n, shp["H"])).astype(np.float32)
        xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((n, shp["H"]))
        m.forward_cached(xb, n, ob)
        ref = A.attention_cached(w, x, cache)
        check(ob.numpy(), ref, f"cached +{n} at {cache.cur_len - n}")
    m.close()


def test_forward_is_causal(gpu):
    shp = SHAPES[0]
    m, _ = _ctx(gpu, shp)
    x = np.random.default_rng(1).standard_normal((70, shp["H"])).astype(np.float32)
    a = m.run(x)
    x2 = x.copy()
    x2[40:] += 1.0
    b = m.run(x2)
    np.testing.assert_array_equal(a[:40], b[:40])
    m.close()


def test_2d_tables_match_oracle(gpu):
    for text, ih, iw in ((5, 3, 4), (0, 8, 8), (16, 1, 1)):
        seq = text + ih * iw
        for hd in (64, 128):
            cos, sin = gpu.build_2d_rope(seq, hd, text, ih, iw)
            rc, rs = A.build_2d_rope(seq, hd, text, ih, iw)
            assert np.abs(cos.numpy() - rc).max() < 4e-6 and np.abs(sin.numpy() - rs).max() < 4e-6


@pytest.mark.parametrize("shp", SHAPES, ids=["hd64", "hd128"])
def test_cached_matches_oracle(gpu, shp):
    """Chunks of new tokens through the KV cache with 2D rotary tables (device-built,
    the same tables given to the oracle), then a chunk without rotation."""
    m, w = _ctx(gpu, shp, max_tokens=64, max_cache=80, seed=11)
    cache = A.KVCache(shp["nkv"], shp["hd"], max_len=80)
    rng = np.random.default_rng(11)
    text, ih, iw = 4, 6, 6
    cos_d, sin_d = gpu.build_2d_rope(text + ih * iw, shp["hd"], text, ih, iw)
    cos, sin = cos_d.numpy(), sin_d.numpy()
    pos = 0
    for n in (3, 1, 36):
        x = rng.standard_normal((n, shp["H"])).astype(np.float32)
        cs, sn = gpu.Buf.from_array(cos[pos:pos + n]), gpu.Buf.from_array(sin[pos:pos + n])
        xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((n, shp["H"]))
        m.forward_cached(xb, n, ob, cs, sn)
        ref = A.attention_cached(w, x, cache, cos=cos[pos:pos + n], sin=sin[pos:pos + n])
        check(ob.numpy(), ref, f"cached chunk at {pos} (+{n})")
        pos += n
        assert m.cache_len() == pos == cache.cur_len
    x = rng.standard_normal((5, shp["H"])).astype(np.float32)
    xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((5, shp["H"]))
    m.forward_cached(xb, 5, ob)
    check(ob.numpy(), A.attention_cached(w, x, cache), "cached chunk without rotation")
    m.close()


def test_cache_overflow_and_reset(gpu):
    shp = SHAPES[0]
    m, _ = _ctx(gpu, shp, max_tokens=16, max_cache=10)
    x = np.random.default_rng(2).standard_normal((8, shp["H"])).astype(np.float32)
    xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((8, shp["H"]))
    m.forward_cached(xb, 8, ob)
    first = ob.numpy()
    with pytest.raises(gpu.HyError):
        m.forward_cached(xb, 8, ob)
    assert m.cache_len() == 8
    m.cache_reset()
    assert m.cache_len() == 0
    m.forward_cached(xb, 8, ob)
    np.testing.assert_array_equal(ob.numpy(), first)
    m.close()


def test_invalid_calls_rejected(gpu):
    shp = SHAPES[0]
    m = gpu.Attn(shp["H"], shp["nh"], shp["nkv"], shp["hd"], 16)
    xb, ob = gpu.Buf.empty((4, shp["H"])), gpu.Buf.empty((4, shp["H"]))
    with pytest.raises(gpu.HyError):   # weights not uploaded
        m.forward(xb, 4, ob)
    w = A.synth_weights(shp["H"], shp["nh"], shp["nkv"], shp["hd"])
    m.upload(w.qkv_w, w.o_w, w.q_norm, w.k_norm)
    with pytest.raises(gpu.HyError):   # T above max_tokens
        m.forward(xb, 17, ob)
    with pytest.raises(gpu.HyError):   # no cache configured
        m.forward_cached(xb, 4, ob)
    m.close()


def test_decoder_layer_matches_oracle(gpu):
    """decoder_layer_forward_cpu (src/decoder_layer.cpp:9-48) on the device: the
    residual stream h = x + attention(RMSNorm(x) * w_in) to the float tolerance above,
    and out = h + MoE(RMSNorm(h) * w_post) bit for bit against the oracle's MoE half
    evaluated on the device's h (the MoE path is exact given its input)."""
    import hy_oracle as O
    H, I, E, K = 256, 128, 16, 4
    shp = dict(H=H, nh=8, nkv=2, hd=64)
    att, w = _ctx(gpu, shp, max_tokens=64, seed=21)
    rng = np.random.default_rng(21)
    w_in = (0.5 + rng.random(H)).astype(np.float32)
    w_post = (0.5 + rng.random(H)).astype(np.float32)
    att.set_input_norm(w_in)
    layer = O.synth_layer(H, I, E, K, O.Q8_0, seed=21, layer=0, std=0.05)
    moe = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=64)
    moe.synth(0, seed=21, std=0.05)
    moe.set_ffn_norm(0, w_post)
    for T in (1, 20, 64):
        x = rng.standard_normal((T, H)).astype(np.float32)
        xb, ob, hb = gpu.Buf.from_array(x), gpu.Buf.empty((T, H)), gpu.Buf.empty((T, H))
        att.decoder_layer_forward(moe, 0, xb, T, ob, debug_h=hb)
        h = hb.numpy()
        xn = np.empty_like(x)
        O.lib().hyo_rms_norm_f32(O.fp(x), O.fp(w_in), O.fp(xn), T, H, np.float32(1e-5))
        h_ref = (x + A.attention_forward(w, xn)[0]).astype(np.float32)
        check(h, h_ref, f"T={T} residual stream")
        ref = O.moe_stack_qw([layer], [w_post], h, eps=1e-5)
        np.testing.assert_array_equal(ob.numpy().view(np.uint32), ref.view(np.uint32), err_msg=f"T={T} out")
    other = gpu.Moe(2 * H, I, E, K, O.Q8_0, max_tokens=8)
    xb, ob = gpu.Buf.empty((4, H)), gpu.Buf.empty((4, H))
    with pytest.raises(gpu.HyError):
        att.decoder_layer_forward(other, 0, xb, 4, ob)
    other.close()
    moe.close()
    att.close()


@pytest.mark.parametrize("M,N,Kd", [(1, 6150, 4096), (2, 100, 48), (3, 1031, 272), (5, 4099, 1040),
                                    (8, 6144, 4096), (9, 517, 4096), (16, 4097, 336), (17, 100, 48),
                                    (300, 512, 256), (2048, 4096, 512), (1111, 6144, 64),
                                    (1300, 6200, 80), (1290, 6150, 4096), (2100, 8200, 64), (520, 6150, 1024)])
def test_gemm_both_tilings(gpu, M, N, Kd):
    """The projections' GEMM (hy_lm_head_f32) on each of its paths, ragged M and N, with
    and without the residual, against float64:
      * decode-sized GEMV, M <= 16 (one or two passes over W, ragged N, K not a multiple
        of the 256-float chunk a wave loads);
      * one-wave register kernel: small grids (17x100, 300x512, 1111x6144 with K=64);
      * LDS-staged, one 128 x 128 tile per work group: >= 1024 tiles (2100x8200), or
        K % 32 != 0 with >= 512 tiles (1300x6200x80, stages of 16 floats);
      * LDS-staged stream-K + fix-up: 64..1023 tiles with K % 32 == 0 (2048x4096x512,
        1290x6150x4096, 520x6150x1024)."""
    rng = np.random.default_rng(M)
    x = rng.standard_normal((M, Kd)).astype(np.float32)
    w = rng.standard_normal((N, Kd)).astype(np.float32)
    r = rng.standard_normal((M, N)).astype(np.float32)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    check(gpu.lm_head_f32(x, w), ref, f"gemm {M}x{N}x{Kd}")
    check(gpu.lm_head_f32(x, w, r), ref + r, f"gemm+resid {M}x{N}x{Kd}")


def test_gemm_stream_k_scratch_across_streams(gpu):
    """The stand-alone GEMM keeps one stream-K scratch per device: calls queued on two
    streams back to back (no host sync between them) are ordered on the device and
    both give the right product."""
    M, N, Kd = 1290, 6150, 1024   # a stream-K shape
    rng = np.random.default_rng(3)
    xs = [rng.standard_normal((M, Kd)).astype(np.float32) for _ in range(2)]
    w = rng.standard_normal((N, Kd)).astype(np.float32)
    wb = gpu.Buf.from_array(w)
    xb = [gpu.Buf.from_array(x) for x in xs]
    ob = [gpu.Buf.empty((M, N)) for _ in range(2)]
    streams = [gpu.Stream(), gpu.Stream()]
    for rep in range(3):
        for i in range(2):
            gpu.check(gpu.lib().hy_lm_head_f32(xb[i].ptr, wb.ptr, None, M, Kd, N, ob[i].ptr, streams[i].h))
    for s in streams:
        s.synchronize()
    for i in range(2):
        check(ob[i].numpy(), xs[i].astype(np.float64) @ w.astype(np.float64).T, f"stream {i}")
    for s in streams:
        s.close()
