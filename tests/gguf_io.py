"""Minimal GGUF writer for test fixtures (public GGUF layout, versions 2 and 3):

    magic "GGUF" | u32 version | u64 n_tensors | u64 n_kv
    n_kv x (string key, u32 type, value)
    n_tensors x (string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset)
    padding to the alignment, then the tensor data (each tensor aligned)

Strings are u64 length + bytes; everything is little-endian.  Test infrastructure
only: it writes the files the reader under test parses.
"""
import struct

import numpy as np

(T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64,
 T_F64) = range(13)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_BF16 = 0, 1, 2, 8, 30

_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
        T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == T_STR:
        return _str(v)
    if t == T_ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, i) for i in items)
    return struct.pack(_FMT[t], v)


def gguf_bytes(kvs, tensors, version=3, alignment=None, data_offsets=None):
    """kvs: [(key, type, value)]; tensors: [(name, ggml_type, ne (innermost first),
    data bytes)].  alignment: written as general.alignment when given (else 32 is
    used).  data_offsets: override the tensor offsets (for corrupt-file tests)."""
    al = alignment or 32
    kv = list(kvs) + ([("general.alignment", T_U32, alignment)] if alignment else [])
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv)))
    for key, t, v in kv:
        out += _str(key) + struct.pack("<I", t) + _value(t, v)
    offs, o = [], 0
    for _, _, _, data in tensors:
        offs.append(o)
        o += (len(data) + al - 1) // al * al
    if data_offsets is not None:
        offs = list(data_offsets)
    for (name, gt, ne, _), off in zip(tensors, offs):
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        out += struct.pack("<IQ", gt, off)
    out += b"\0" * ((-len(out)) % al)
    base = len(out)
    for (_, _, _, data), off in zip(tensors, offs):
        end = base + off + len(data)
        if base + off - len(out) > (1 << 24):
            continue   # an offset far past any real data (corrupt-file tests): no data
        if len(out) < end:
            out += b"\0" * (end - len(out))
        out[base + off:end] = data
    out += b"\0" * ((-len(out)) % al)
    return bytes(out)


def layer_tensors(layer, block, ffn_norm=None):
    """The reference converter's tensor names for one MoE layer (oracle Layer, GGUF
    layout: ne0 = in-features); ffn_norm: the post-attention RMSNorm weight [H]."""
    H, I, E, wt = layer.H, layer.I, layer.E, layer.wtype
    p = f"blk.{block}."
    ts = [(p + "ffn_gate.weight", GGML_F32, [H, E], np.ascontiguousarray(layer.router, np.float32).tobytes())]
    if ffn_norm is not None:
        nw = np.ascontiguousarray(ffn_norm, np.float32)
        ts.append((p + "ffn_norm.weight", GGML_F32, [nw.size], nw.tobytes()))
    if layer.shared_gu is not None:
        ts.append((p + "ffn_shared_gate_up.weight", wt, [H, 2 * I], layer.shared_gu.tobytes()))
        ts.append((p + "ffn_shared_down.weight", wt, [I, H], layer.shared_dn.tobytes()))
    for e in range(E):
        ts.append((p + f"ffn_expert_{e}_gate_up.weight", wt, [H, 2 * I], layer.gu[e].tobytes()))
        ts.append((p + f"ffn_expert_{e}_down.weight", wt, [I, H], layer.dn[e].tobytes()))
    return ts


def layer_meta(layer):
    return [("general.architecture", T_STR, "hunyuan3"),
            ("hunyuan.hidden_size", T_U32, layer.H),
            ("hunyuan.moe_intermediate_size", T_U32, layer.I),
            ("hunyuan.num_experts", T_U32, layer.E),
            ("hunyuan.moe_topk", T_U32, layer.K),
            ("hunyuan.rms_norm_eps", T_F32, 1e-5)]


def float_tensor(a, gtype):
    """(bytes, values the reader gives back as f32) of a float array stored as F32,
    F16 or BF16 (BF16: the upper 16 bits of each f32)."""
    a = np.ascontiguousarray(a, np.float32)
    if gtype == GGML_F32:
        return a.tobytes(), a
    if gtype == GGML_F16:
        h = a.astype(np.float16)
        return h.tobytes(), h.astype(np.float32)
    if gtype == GGML_BF16:
        b = (a.view(np.uint32) >> 16).astype(np.uint16)
        return b.tobytes(), (b.astype(np.uint32) << 16).view(np.float32)
    raise ValueError(gtype)


def attn_tensors(w, block, gtype=GGML_F32, in_norm=None):
    """blk.N.attn_* of an attention layer (oracle AttnWeights), as the reference loader
    reads them; returns (tensors, the f32 values a reader recovers per name)."""
    p = f"blk.{block}."
    nq, H = w.nh * w.hd, w.H
    items = [("attn_qkv.weight", w.qkv_w, [H, w.qkv_w.shape[0]]), ("attn_output.weight", w.o_w, [nq, H]),
             ("attn_q_norm.weight", w.q_norm, [w.hd]), ("attn_k_norm.weight", w.k_norm, [w.hd])]
    if in_norm is not None:
        items.append(("attn_norm.weight", in_norm, [H]))
    ts, vals = [], {}
    for name, arr, ne in items:
        data, back = typed_tensor(arr, gtype)
        ts.append((p + name, gtype, ne, data))
        vals[name] = back.reshape(np.asarray(arr).shape)
    return ts, vals


def global_tensors(emb, final_norm, lm_head, gtype=GGML_F32):
    V, H = emb.shape
    ts, vals = [], {}
    for name, arr, ne in (("token_embd.weight", emb, [H, V]), ("output_norm.weight", final_norm, [H]),
                          ("output.weight", lm_head, [H, V])):
        data, back = typed_tensor(arr, gtype)
        ts.append((name, gtype, ne, data))
        vals[name] = back.reshape(np.asarray(arr).shape)
    return ts, vals


def typed_tensor(a, gtype):
    """(bytes, the f32 values a reader gives back) of a float array stored as F32, F16,
    BF16, Q8_0 or Q4_0 (blocks of 32 along the last axis, the oracle's quantizers)."""
    if gtype in (GGML_F32, GGML_F16, GGML_BF16):
        return float_tensor(a, gtype)
    import hy_oracle as O
    a = np.ascontiguousarray(a, np.float32)
    q = O.quantize(a, gtype)
    return q.tobytes(), O.dequantize(q, gtype, a.shape[-1])


def typed_layer_tensors(router, gu, dn, sgu, sdn, block, gtype, ffn_norm=None):
    """One MoE layer with every tensor in one ggml type, as the reference converter
    writes a file (one --type for all tensors).  router [E][H], gu [E][2I][H],
    dn [E][H][I], sgu / sdn the shared expert (or None), ffn_norm [H] or None.
    Returns (tensors, {role: the f32 values a reader recovers})."""
    E, H = router.shape
    I = dn.shape[2]
    p = f"blk.{block}."
    ts, back = [], {}

    def add(name, arr, ne, role):
        data, vals = typed_tensor(arr, gtype)
        ts.append((p + name, gtype, ne, data))
        back[role] = vals
        return data

    add("ffn_gate.weight", router, [H, E], "router")
    if ffn_norm is not None:
        add("ffn_norm.weight", ffn_norm, [H], "ffn_norm")
    raw = {"gu": [], "dn": []}
    if sgu is not None:
        raw["sgu"] = add("ffn_shared_gate_up.weight", sgu, [H, 2 * I], "sgu")
        raw["sdn"] = add("ffn_shared_down.weight", sdn, [I, H], "sdn")
    gus, dns = [], []
    for e in range(E):
        raw["gu"].append(add(f"ffn_expert_{e}_gate_up.weight", gu[e], [H, 2 * I], "gu"))
        gus.append(back["gu"])
        raw["dn"].append(add(f"ffn_expert_{e}_down.weight", dn[e], [I, H], "dn"))
        dns.append(back["dn"])
    back["gu"], back["dn"], back["raw"] = np.stack(gus), np.stack(dns), raw
    return ts, back
