"""The resident backbone (hy_model_*: HunyuanFullModel) on the GPU.

Each decoder layer is the decoder-layer entry point already held to the oracle in
test_attn_gpu.py; here the model's chain of layers must equal that entry point applied
layer by layer (bit for bit: same kernels, same inputs), the embedding lookup must be
exact, and the final RMSNorm + lm_head must match float64 on the device's final hidden
state to the attention tolerance (normwise 1e-4, cosine 0.99999)."""
import numpy as np
import pytest

import hy_oracle as O
import hy_oracle_attn as A

pytestmark = pytest.mark.gpu

H, I, E, K = 256, 128, 16, 4
NH, NKV, HD = 8, 2, 64
V, L, TM = 512, 3, 32


def _rel(a, b):
    a, b = a.astype(np.float64).ravel(), b.astype(np.float64).ravel()
    return np.abs(a - b).max() / np.abs(b).max(), a @ b / (np.linalg.norm(a) * np.linalg.norm(b))


@pytest.fixture(scope="module")
def model(gpu):
    rng = np.random.default_rng(77)
    m = gpu.Model(H, I, E, K, O.Q8_0, NH, NKV, HD, V, L, TM)
    emb = rng.standard_normal((V, H)).astype(np.float32)
    fn = (0.5 + rng.random(H)).astype(np.float32)
    lm = (rng.standard_normal((V, H)) * 0.05).astype(np.float32)
    m.upload_globals(emb, fn, lm)
    for l in range(L):
        w = A.synth_weights(H, NH, NKV, HD, seed=100 + l, std=0.05, norm_jitter=0.2)
        m.attn.upload(w.qkv_w, w.o_w, w.q_norm, w.k_norm, layer=l)
        m.attn.set_input_norm((0.5 + rng.random(H)).astype(np.float32), layer=l)
        m.moe.synth(l, seed=200 + l, std=0.05)
        m.moe.set_ffn_norm(l, (0.5 + rng.random(H)).astype(np.float32))
    yield m, emb, fn, lm
    m.close()


def test_layer_chain_equals_decoder_layers(gpu, model):
    m, emb, _, _ = model
    T = 20
    x = emb[np.random.default_rng(1).integers(0, V, size=T)]
    xb = gpu.Buf.from_array(x)
    cur = xb
    for l in range(L):
        nxt = gpu.Buf.empty((T, H))
        m.attn.decoder_layer_forward(m.moe, l, cur, T, nxt, layer=l)
        hb = gpu.Buf.empty((T, H))
        m.forward_hidden(xb, T, hb, n_layers=l + 1)
        np.testing.assert_array_equal(hb.numpy().view(np.uint32), nxt.numpy().view(np.uint32),
                                      err_msg=f"after layer {l}")
        cur = nxt
    full = gpu.Buf.empty((T, H))
    m.forward_hidden(xb, T, full)   # n_layers 0: all
    np.testing.assert_array_equal(full.numpy(), cur.numpy())


def test_forward_logits(gpu, model):
    m, emb, fn, lm = model
    T = 12
    ids = np.random.default_rng(2).integers(0, V, size=T).astype(np.int32)
    ids[5] = V + 7                     # outside the vocabulary: a zero embedding row
    ib, lb = gpu.Buf.from_array(ids), gpu.Buf.empty((T, V))
    m.forward(ib, T, lb)
    logits = lb.numpy()
    x = emb[np.clip(ids, 0, V - 1)].copy()
    x[5] = 0.0
    hb = gpu.Buf.empty((T, H))
    m.forward_hidden(gpu.Buf.from_array(x), T, hb)
    h = hb.numpy().astype(np.float64)
    hn = h / np.sqrt((h * h).mean(1, keepdims=True) + 1e-5) * fn.astype(np.float64)
    ref = hn @ lm.astype(np.float64).T
    err, cos = _rel(logits, ref)
    assert err < 1e-4 and cos > 0.99999, (err, cos)


def test_invalid_calls(gpu, model):
    m, *_ = model
    xb, hb = gpu.Buf.empty((4, H)), gpu.Buf.empty((4, H))
    with pytest.raises(gpu.HyError):
        m.forward_hidden(xb, 4, hb, n_layers=L + 1)
    with pytest.raises(gpu.HyError):
        m.forward_hidden(xb, TM + 1, hb)
    with pytest.raises(gpu.HyError):   # the MoE and attention configs must agree
        bad = gpu.ModelConfig(gpu.Config(H, I, E, K, L, TM, O.Q8_0, 1, 1, 1.0, 0, 0, 0, 0),
                              gpu.AttnConfig(2 * H, NH, NKV, HD, L, TM, 0, 1e-5, 1e4, 0), V)
        h = gpu.C.c_void_p()
        gpu.check(gpu.lib().hy_model_create(gpu.C.byref(bad), gpu.C.byref(h)))
