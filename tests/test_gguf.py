"""GGUF reader (host code, runs without a GPU) and layer upload from GGUF files (GPU).

The files are written by tests/gguf_io.py from the public GGUF layout; the reader
must give back exactly the bytes, dims, types and metadata written, reject corrupt
files with an error, and the layer uploaded from a file must compute bit for bit
what the oracle computes from the same weights."""
import struct

import numpy as np
import pytest

import gguf_io as G
import hy_oracle as O


def _write(tmp_path, name, blob):
    p = tmp_path / name
    p.write_bytes(blob)
    return str(p)


def _tensors(rng):
    f32 = rng.standard_normal((3, 40)).astype(np.float32)
    f16 = rng.standard_normal((2, 64)).astype(np.float16)
    q8 = rng.integers(0, 256, size=(5, 2 * 34), dtype=np.uint8)    # 5 rows x 64 elements
    q4 = rng.integers(0, 256, size=(4, 3 * 18), dtype=np.uint8)    # 4 rows x 96 elements
    return [("a.f32", G.GGML_F32, [40, 3], f32.tobytes()),
            ("b.f16", G.GGML_F16, [64, 2], f16.tobytes()),
            ("c.q8_0", G.GGML_Q8_0, [64, 5], q8.tobytes()),
            ("d.q4_0", G.GGML_Q4_0, [96, 2, 2], q4.tobytes()),
            ("e.unknown", 12, [256, 1], b"\x01" * 144)]


KVS = [("k.u8", G.T_U8, 200), ("k.i8", G.T_I8, -5), ("k.u16", G.T_U16, 60000), ("k.i32", G.T_I32, 7),
       ("k.u32", G.T_U32, 4096), ("k.u64", G.T_U64, 123456789), ("k.f32", G.T_F32, 0.25),
       ("k.f64", G.T_F64, 1.5), ("k.bool", G.T_BOOL, True), ("k.str", G.T_STR, "hunyuan3"),
       ("k.arr", G.T_ARR, (G.T_U32, [1, 2, 3])), ("k.sarr", G.T_ARR, (G.T_STR, ["x", "yz"])),
       ("k.neg", G.T_I32, -1)]


@pytest.mark.parametrize("version,alignment", [(3, None), (3, 64), (2, None), (3, 256)])
def test_roundtrip(hy, tmp_path, version, alignment):
    rng = np.random.default_rng(version * 1000 + (alignment or 0))
    ts = _tensors(rng)
    path = _write(tmp_path, "t.gguf", G.gguf_bytes(KVS, ts, version=version, alignment=alignment))
    f = hy.Gguf(path)
    assert f.n_tensors() == len(ts)
    for name, gt, ne, data in ts:
        t, nd, ne4, nbytes, got = f.tensor(name)
        assert t == gt and nd == len(ne) and ne4[:nd] == ne and all(v == 1 for v in ne4[nd:])
        if gt == 12:
            assert nbytes == 0 and got is None   # a type the reader does not size
        else:
            assert nbytes == len(data) and got == data
    assert f.get_u32("k.u8") == 200 and f.get_u32("k.u16") == 60000 and f.get_u32("k.u32") == 4096
    assert f.get_u32("k.u64") == 123456789 and f.get_u32("k.i32") == 7 and f.get_u32("k.bool") == 1
    assert f.get_f32("k.f32") == 0.25 and f.get_f32("k.f64") == 1.5
    for bad in ("k.i8", "k.neg", "k.str", "k.arr", "missing"):
        with pytest.raises(hy.HyError):
            f.get_u32(bad)
    with pytest.raises(hy.HyError):
        f.get_f32("k.u32")
    with pytest.raises(hy.HyError):
        f.tensor("no.such.tensor")
    f.close()


def test_data_offset_is_aligned(hy, tmp_path):
    """The data section starts at the next multiple of general.alignment."""
    ts = [("t", G.GGML_F32, [8], np.arange(8, dtype=np.float32).tobytes())]
    blob = G.gguf_bytes([("pad", G.T_STR, "x" * 13)], ts, alignment=128)
    path = _write(tmp_path, "a.gguf", blob)
    f = hy.Gguf(path)
    *_, data = f.tensor("t")
    assert np.frombuffer(data, np.float32).tolist() == list(range(8))
    f.close()


def _corrupt_cases():
    ts = [("t", G.GGML_Q8_0, [64, 2], bytes(136))]
    good = G.gguf_bytes([("k", G.T_U32, 1)], ts)
    yield "bad magic", b"GGUX" + good[4:]
    yield "version 1", good[:4] + struct.pack("<I", 1) + good[8:]
    yield "version 4", good[:4] + struct.pack("<I", 4) + good[8:]
    yield "truncated header", good[:20]
    yield "truncated kv", good[:30]
    yield "tensor past the end", good[:-64]
    yield "misaligned offset", G.gguf_bytes([], ts, data_offsets=[8])
    yield "offset past the end", G.gguf_bytes([], ts, data_offsets=[1 << 40])
    yield "huge tensor count", good[:8] + struct.pack("<Q", 1 << 60) + good[16:]
    yield "bad alignment", G.gguf_bytes([("general.alignment", G.T_U32, 24)], ts)
    yield "zero dims", G.gguf_bytes([], [("t", G.GGML_F32, [], b"")])
    yield "five dims", G.gguf_bytes([], [("t", G.GGML_F32, [1, 1, 1, 1, 1], bytes(4))])


@pytest.mark.parametrize("case,blob", list(_corrupt_cases()), ids=[c for c, _ in _corrupt_cases()])
def test_corrupt_files_rejected(hy, tmp_path, case, blob):
    path = _write(tmp_path, "bad.gguf", blob)
    with pytest.raises(hy.HyError):
        hy.Gguf(path)


def test_missing_file(hy, tmp_path):
    with pytest.raises(hy.HyError):
        hy.Gguf(str(tmp_path / "nope.gguf"))


# ------------------------------------------------------------------ GPU: layer upload

def decode_blocks(data, gtype, n):
    """GGUF Q8_0 / Q4_0 bytes -> f32 with numpy, written from the block layout
    (fp16 scale, then 32 int8, or 16 bytes whose low nibbles are elements 0..15 and
    high nibbles 16..31, value nibble - 8)."""
    bb = 34 if gtype == G.GGML_Q8_0 else 18
    b = np.frombuffer(data, np.uint8).reshape(-1, bb)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    if gtype == G.GGML_Q8_0:
        q = b[:, 2:].view(np.int8).astype(np.float32)
    else:
        q = np.concatenate([(b[:, 2:] & 15), (b[:, 2:] >> 4)], axis=1).astype(np.float32) - 8
    return (d * q).reshape(-1)[:n]


@pytest.mark.parametrize("gtype", [G.GGML_F32, G.GGML_F16, G.GGML_BF16, G.GGML_Q8_0, G.GGML_Q4_0],
                         ids=["f32", "f16", "bf16", "q8_0", "q4_0"])
def test_tensor_f32_every_loader_type(hy, tmp_path, gtype):
    """hy_gguf_tensor_f32 (read_tensor_data) gives back every type the reference loader
    reads: float types exactly, block types as d * q from an independent decoder,
    including a block whose fp16 scale is subnormal (kept, not flushed)."""
    rng = np.random.default_rng(gtype)
    a = (rng.standard_normal((5, 96)) * 3).astype(np.float32)
    a[2, :32] = rng.standard_normal(32) * 1e-4      # scale ~2e-6: an fp16 subnormal
    data, back = G.typed_tensor(a, gtype)
    f = hy.Gguf(_write(tmp_path, "t.gguf", G.gguf_bytes([], [("w", gtype, [96, 5], data)])))
    got = f.tensor_f32("w")
    assert got.shape == (5, 96)
    np.testing.assert_array_equal(got.view(np.uint32), back.reshape(5, 96).view(np.uint32))
    if gtype in (G.GGML_Q8_0, G.GGML_Q4_0):
        ref = decode_blocks(data, gtype, a.size).reshape(5, 96)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
        d = np.frombuffer(data[(2 * 3) * (34 if gtype == G.GGML_Q8_0 else 18):][:2], np.float16)[0]
        assert 0 < abs(float(d)) < 6.1e-5 and np.abs(got[2, :32]).max() > 0
    elif gtype == G.GGML_F16:
        np.testing.assert_array_equal(got, a.astype(np.float16).astype(np.float32))
    f.close()


def test_tensor_f32_rejects_other_types_and_sizes(hy, tmp_path):
    q41 = bytes(20 * 3)   # Q4_1: 20 bytes per block, a type the loader does not read
    ts = [("q41", 3, [96, 1], q41), ("f", G.GGML_F32, [8, 2], np.zeros(16, np.float32).tobytes())]
    f = hy.Gguf(_write(tmp_path, "o.gguf", G.gguf_bytes([], ts)))
    with pytest.raises(hy.HyError):
        f.tensor_f32("q41")
    out = np.empty(15, np.float32)
    with pytest.raises(hy.HyError):
        hy.check(hy.lib().hy_gguf_tensor_f32(f.h, b"f", out.ctypes.data, out.size))
    with pytest.raises(hy.HyError):
        f.tensor_f32("missing")
    f.close()


SHAPE = dict(H=256, I=128, E=16, K=4)


@pytest.mark.gpu
@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_0, O.F32])
def test_layer_from_gguf_matches_oracle(gpu, tmp_path, wtype):
    """Two layers in one file (blocks 3 and 7, as a converter writes per-layer
    names); each uploaded layer computes what the oracle computes on its weights."""
    H, I, E, K = SHAPE["H"], SHAPE["I"], SHAPE["E"], SHAPE["K"]
    layers = {b: O.synth_layer(H, I, E, K, wtype, seed=31 + b, layer=b, std=0.05) for b in (3, 7)}
    ts = G.layer_tensors(layers[3], 3) + G.layer_tensors(layers[7], 7)
    path = _write(tmp_path, "layers.gguf", G.gguf_bytes(G.layer_meta(layers[3]), ts))
    f = gpu.Gguf(path)
    m = gpu.Moe(H, I, E, K, wtype, num_layers=2, max_tokens=64)
    m.upload_gguf(0, f, 7)
    m.upload_gguf(1, f, 3)
    f.close()   # the weights are resident: the mapping may go
    for T in (1, 5, 40):
        x = O.synth(200 + T, 0, O.T_X, 0, (T, H), 1.0)
        for slot, block in ((0, 7), (1, 3)):
            got = m.run(slot, x)
            ref = O.moe_forward_q(layers[block], x)
            np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32),
                                          err_msg=f"wtype={wtype} T={T} block={block}")
    m.close()


@pytest.mark.gpu
def test_layer_from_gguf_with_ffn_norm(gpu, tmp_path):
    """blk.N.ffn_norm.weight (post_attention_layernorm) is picked up with the layer and
    applied by the stack; a file without it leaves unit weight; a wrong shape is an
    error."""
    H, I, E, K = SHAPE["H"], SHAPE["I"], SHAPE["E"], SHAPE["K"]
    layer = O.synth_layer(H, I, E, K, O.Q8_0, seed=21, std=0.05)
    w = (0.5 + np.random.default_rng(21).random(H)).astype(np.float32)
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=32)
    x = O.synth(22, 0, O.T_X, 0, (20, H), 1.0)
    xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((20, H))
    f = gpu.Gguf(_write(tmp_path, "n.gguf", G.gguf_bytes(G.layer_meta(layer), G.layer_tensors(layer, 2, ffn_norm=w))))
    m.upload_gguf(0, f, 2)
    f.close()
    m.stack_forward(0, 1, xb, 20, 1e-5, ob)
    np.testing.assert_array_equal(ob.numpy().view(np.uint32),
                                  O.moe_stack_qw([layer], [w], x, eps=1e-5).view(np.uint32))
    f = gpu.Gguf(_write(tmp_path, "u.gguf", G.gguf_bytes(G.layer_meta(layer), G.layer_tensors(layer, 2))))
    m.upload_gguf(0, f, 2)
    f.close()
    m.stack_forward(0, 1, xb, 20, 1e-5, ob)
    np.testing.assert_array_equal(ob.numpy().view(np.uint32), O.moe_stack_q([layer], x, eps=1e-5).view(np.uint32))
    f = gpu.Gguf(_write(tmp_path, "b.gguf", G.gguf_bytes(G.layer_meta(layer),
                                                           G.layer_tensors(layer, 2, ffn_norm=w[:-32]))))
    with pytest.raises(gpu.HyError):
        m.upload_gguf(0, f, 2)
    f.close()
    m.close()


@pytest.mark.gpu
def test_layer_from_gguf_without_shared_expert(gpu, tmp_path):
    H, I, E, K = SHAPE["H"], SHAPE["I"], SHAPE["E"], SHAPE["K"]
    layer = O.synth_layer(H, I, E, K, O.Q8_0, seed=5, std=0.05, shared=False)
    path = _write(tmp_path, "noshared.gguf", G.gguf_bytes(G.layer_meta(layer), G.layer_tensors(layer, 0)))
    f = gpu.Gguf(path)
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=16, has_shared=False)
    m.upload_gguf(0, f, 0)
    x = O.synth(9, 0, O.T_X, 0, (7, H), 1.0)
    np.testing.assert_array_equal(m.run(0, x).view(np.uint32), O.moe_forward_q(layer, x).view(np.uint32))
    m.close()
    f.close()


@pytest.mark.gpu
def test_layer_from_gguf_mismatches_rejected(gpu, tmp_path):
    H, I, E, K = SHAPE["H"], SHAPE["I"], SHAPE["E"], SHAPE["K"]
    layer = O.synth_layer(H, I, E, K, O.Q8_0, seed=6, std=0.05)
    good = G.layer_tensors(layer, 0)
    cases = {
        "missing expert": [t for t in good if "ffn_expert_5_down" not in t[0]],
        "type that would change the weights (F16 into Q8_0)":
            [(n, G.GGML_F16, ne, bytes(ne[0] * ne[1] * 2)) if "expert_2_gate_up" in n else (n, gt, ne, d)
             for n, gt, ne, d in good],
        "type the loader does not read (Q4_1)":
            [(n, 3, ne, bytes(ne[0] * ne[1] // 32 * 20)) if "expert_3_down" in n else (n, gt, ne, d)
             for n, gt, ne, d in good],
        "wrong shape": [(n, gt, [ne[0], ne[1] // 2], d[: len(d) // 2]) if "shared_down" in n else (n, gt, ne, d)
                        for n, gt, ne, d in good],
    }
    m = gpu.Moe(H, I, E, K, O.Q8_0, max_tokens=8)
    for case, ts in cases.items():
        f = gpu.Gguf(_write(tmp_path, "m.gguf", G.gguf_bytes(G.layer_meta(layer), ts)))
        with pytest.raises(gpu.HyError):
            m.upload_gguf(0, f, 0)
        f.close()
    meta = [(k, t, (v * 2 if k == "hunyuan.num_experts" else v)) for k, t, v in G.layer_meta(layer)]
    f = gpu.Gguf(_write(tmp_path, "meta.gguf", G.gguf_bytes(meta, good)))
    with pytest.raises(gpu.HyError):
        m.upload_gguf(0, f, 0)
    with pytest.raises(gpu.HyError):   # the layer was never loaded
        xb, ob = gpu.Buf.empty((2, H)), gpu.Buf.empty((2, H))
        m.forward(0, xb, 2, ob)
    f.close()
    m.close()


def _f32_layer(seed, H, I, E):
    r = O.synth(seed, 0, O.T_ROUTER, 0, (E, H), 0.05)
    gu = O.synth(seed, 0, O.T_GU, 0, (E, 2 * I, H), 0.05)
    dn = O.synth(seed, 0, O.T_DN, 0, (E, H, I), 0.05)
    sgu = O.synth(seed, 0, O.T_GU, E, (2 * I, H), 0.05)
    sdn = O.synth(seed, 0, O.T_DN, E, (H, I), 0.05)
    w = (0.5 + np.random.default_rng(seed).random(H)).astype(np.float32)
    return r, gu, dn, sgu, sdn, w


@pytest.mark.gpu
@pytest.mark.parametrize("ftype,wtype", [(G.GGML_Q8_0, O.Q8_0), (G.GGML_Q4_0, O.Q4_0), (G.GGML_F16, O.F32),
                                         (G.GGML_BF16, O.F32), (G.GGML_Q8_0, O.F32), (G.GGML_Q4_0, O.Q8_0)],
                         ids=["q8_0", "q4_0", "f16->f32", "bf16->f32", "q8_0->f32", "q4_0->q8_0"])
def test_layer_from_single_type_file(gpu, tmp_path, ftype, wtype):
    """A file with every tensor in one type, as the reference converter writes it:
    router and ffn_norm are read as f32 whatever their type; expert matrices go as
    stored, become f32 in an F32 context, or Q4_0 re-encodes exactly into Q8_0.  The
    stack (RMSNorm -> MoE -> residual) equals the oracle on the values read back."""
    H, I, E, K = SHAPE["H"], SHAPE["I"], SHAPE["E"], SHAPE["K"]
    r, gu, dn, sgu, sdn, w = _f32_layer(40 + ftype, H, I, E)
    ts, back = G.typed_layer_tensors(r, gu, dn, sgu, sdn, 1, ftype, ffn_norm=w)
    f = gpu.Gguf(_write(tmp_path, "one.gguf", G.gguf_bytes([], ts)))
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=64)
    m.upload_gguf(0, f, 1)
    f.close()
    if wtype == O.F32:
        layer = O.Layer(H, I, E, K, O.F32, back["router"], back["sgu"], back["sdn"], back["gu"], back["dn"])
    else:   # the oracle computes on the file's own blocks (Q4_0 values are Q8_0 values)
        def blocks(b, rows, cols):
            return np.frombuffer(b, np.uint8).reshape(rows, O.row_bytes(ftype, cols))
        raw = back["raw"]
        layer = O.Layer(H, I, E, K, ftype, back["router"], blocks(raw["sgu"], 2 * I, H), blocks(raw["sdn"], H, I),
                        np.stack([blocks(b, 2 * I, H) for b in raw["gu"]]),
                        np.stack([blocks(b, H, I) for b in raw["dn"]]))
    for T in (3, 40):
        x = O.synth(300 + T, 0, O.T_X, 0, (T, H), 1.0)
        xb, ob = gpu.Buf.from_array(x), gpu.Buf.empty((T, H))
        m.stack_forward(0, 1, xb, T, 1e-5, ob)
        ref = O.moe_stack_qw([layer], [back["ffn_norm"]], x, eps=1e-5)
        np.testing.assert_array_equal(ob.numpy().view(np.uint32), ref.view(np.uint32), err_msg=f"T={T}")
    m.close()


@pytest.mark.gpu
@pytest.mark.parametrize("ftype,wtype", [(G.GGML_F16, O.Q8_0), (G.GGML_Q8_0, O.Q4_0), (G.GGML_F32, O.Q4_0)])
def test_layer_file_type_that_would_change_weights_rejected(gpu, tmp_path, ftype, wtype):
    H, I, E, K = SHAPE["H"], SHAPE["I"], SHAPE["E"], SHAPE["K"]
    r, gu, dn, sgu, sdn, w = _f32_layer(50, H, I, E)
    ts, _ = G.typed_layer_tensors(r, gu, dn, sgu, sdn, 0, ftype)
    f = gpu.Gguf(_write(tmp_path, "x.gguf", G.gguf_bytes([], ts)))
    m = gpu.Moe(H, I, E, K, wtype, max_tokens=8)
    with pytest.raises(gpu.HyError, match="would change the weights"):
        m.upload_gguf(0, f, 0)
    f.close()
    m.close()


# ------------------------------------------------------------------ GPU: attention + globals

@pytest.mark.gpu
@pytest.mark.parametrize("gtype", [G.GGML_F32, G.GGML_F16, G.GGML_BF16, G.GGML_Q8_0, G.GGML_Q4_0],
                         ids=["f32", "f16", "bf16", "q8_0", "q4_0"])
def test_attention_from_gguf(gpu, tmp_path, gtype):
    """blk.N.attn_* (any type the reference loader reads) uploaded from a file compute exactly what the
    same values uploaded directly compute; attn_norm.weight becomes the layer's input
    norm."""
    import hy_oracle_attn as A
    H, nh, nkv, hd = 256, 8, 2, 64
    w = A.synth_weights(H, nh, nkv, hd, seed=gtype, std=0.05, norm_jitter=0.2)
    in_norm = (0.5 + np.random.default_rng(gtype).random(H)).astype(np.float32)
    ts, vals = G.attn_tensors(w, 4, gtype, in_norm=in_norm)
    f = gpu.Gguf(_write(tmp_path, "a.gguf", G.gguf_bytes([], ts)))
    a = gpu.Attn(H, nh, nkv, hd, 32, num_layers=2)
    a.upload_gguf(1, f, 4)
    f.close()
    a.upload(vals["attn_qkv.weight"], vals["attn_output.weight"], vals["attn_q_norm.weight"],
             vals["attn_k_norm.weight"], layer=0)
    a.set_input_norm(vals["attn_norm.weight"], layer=0)
    x = np.random.default_rng(9).standard_normal((20, H)).astype(np.float32)
    np.testing.assert_array_equal(a.run(x, layer=1), a.run(x, layer=0))
    moe = gpu.Moe(H, 128, 16, 4, O.Q8_0, max_tokens=32)
    moe.synth(0, seed=1, std=0.05)
    xb = gpu.Buf.from_array(x)
    o0, o1 = gpu.Buf.empty((20, H)), gpu.Buf.empty((20, H))
    a.decoder_layer_forward(moe, 0, xb, 20, o0, layer=0)
    a.decoder_layer_forward(moe, 0, xb, 20, o1, layer=1)
    np.testing.assert_array_equal(o0.numpy(), o1.numpy())
    moe.close()
    a.close()


@pytest.mark.gpu
def test_attention_gguf_rejects_bad_tensors(gpu, tmp_path):
    import hy_oracle_attn as A
    H, nh, nkv, hd = 256, 8, 2, 64
    w = A.synth_weights(H, nh, nkv, hd, seed=3)
    good, _ = G.attn_tensors(w, 0)
    a = gpu.Attn(H, nh, nkv, hd, 16)
    cases = {
        "missing k norm": [t for t in good if "attn_k_norm" not in t[0]],
        "wrong shape": [(n, gt, [ne[0] // 2, ne[1]], d[: len(d) // 2]) if "attn_qkv" in n else (n, gt, ne, d)
                        for n, gt, ne, d in good],
        "type the loader does not read (Q4_1)": [(n, 3, ne, bytes(len(d) // 4 * 20 // 32)) if "attn_output" in n
                                                  else (n, gt, ne, d) for n, gt, ne, d in good],
    }
    for case, ts in cases.items():
        f = gpu.Gguf(_write(tmp_path, "bad.gguf", G.gguf_bytes([], ts)))
        with pytest.raises(gpu.HyError):
            a.upload_gguf(0, f, 0)
        f.close()
    a.close()


@pytest.mark.gpu
@pytest.mark.parametrize("gtype", [G.GGML_F32, G.GGML_BF16, G.GGML_Q8_0], ids=["f32", "bf16", "q8_0"])
def test_model_globals_from_gguf(gpu, tmp_path, gtype):
    """token_embd / output_norm / output from a file give the same logits as the same
    values uploaded directly."""
    import hy_oracle_attn as A
    H, I, E, K, nh, nkv, hd, V, L = 256, 128, 16, 4, 8, 2, 64, 300, 1
    rng = np.random.default_rng(5)
    emb = rng.standard_normal((V, H)).astype(np.float32)
    fn = (0.5 + rng.random(H)).astype(np.float32)
    lm = (rng.standard_normal((V, H)) * 0.05).astype(np.float32)
    ts, vals = G.global_tensors(emb, fn, lm, gtype)
    path = _write(tmp_path, "g.gguf", G.gguf_bytes([], ts))
    models = []
    for from_file in (True, False):
        m = gpu.Model(H, I, E, K, O.Q8_0, nh, nkv, hd, V, L, 16)
        w = A.synth_weights(H, nh, nkv, hd, seed=7, std=0.05)
        m.attn.upload(w.qkv_w, w.o_w, w.q_norm, w.k_norm)
        m.moe.synth(0, seed=7, std=0.05)
        if from_file:
            f = gpu.Gguf(path)
            m.upload_globals_gguf(f)
            f.close()
        else:
            m.upload_globals(vals["token_embd.weight"], vals["output_norm.weight"], vals["output.weight"])
        models.append(m)
    ids = gpu.Buf.from_array(rng.integers(0, V, size=9).astype(np.int32))
    outs = []
    for m in models:
        lb = gpu.Buf.empty((9, V))
        m.forward(ids, 9, lb)
        outs.append(lb.numpy())
        m.close()
    np.testing.assert_array_equal(outs[0], outs[1])
