"""ctypes bindings of the attention restatement (hy_oracle_attn.c, in liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the GPU attention path (parity tests,
smoke check, the benchmark's CPU-baseline leg).  The functions follow the
reference's fp32 algorithm operation for operation; see hy_oracle_attn.h.
"""
import ctypes as C

import numpy as np

import hy_oracle as O

_fp = C.POINTER(C.c_float)
_ip = C.POINTER(C.c_int32)
_u32 = C.c_uint32


class KVCacheC(C.Structure):
    _fields_ = [("k", _fp), ("v", _fp), ("max_len", _u32), ("cur_len", _u32)]


_bound = False


def lib():
    global _bound
    L = O.lib()
    if not _bound:
        sig = {
            "hyo_rope_f32": (None, [_fp, _fp, _u32, _u32, _u32, _u32, C.c_float, _ip]),
            "hyo_build_2d_rope": (None, [_u32, _u32, _u32, _u32, _u32, C.c_float, _fp, _fp]),
            "hyo_apply_rope_2d_f32": (None, [_fp, _fp, _fp, _fp, _u32, _u32, _u32, _u32]),
            "hyo_attention_forward": (None, [_fp, _fp, _fp, _fp, _fp, _u32, _u32, _u32, _u32, _u32, C.c_float,
                                             C.c_float, _ip, _fp, _fp, _fp, _fp]),
            "hyo_attention_cached": (C.c_int, [_fp, _fp, _fp, _fp, _fp, _u32, _u32, _u32, _u32, _u32, C.c_float,
                                               _fp, _fp, C.POINTER(KVCacheC), _fp]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _bound = True
    return L


def _fp_or_none(a):
    return None if a is None else O.fp(a)


class AttnWeights:
    """One layer's attention weights in the reference's layout: qkv_w
    [(nh + 2 nkv) hd][H] (rows: q heads, then k heads, then v heads), o_w [H][nh hd],
    q_norm / k_norm [hd]."""

    def __init__(self, qkv_w, o_w, q_norm, k_norm, nh, nkv, hd):
        self.qkv_w, self.o_w = O.f32(qkv_w), O.f32(o_w)
        self.q_norm, self.k_norm = O.f32(q_norm), O.f32(k_norm)
        self.nh, self.nkv, self.hd = nh, nkv, hd
        self.H = self.qkv_w.shape[1]
        assert self.qkv_w.shape == ((nh + 2 * nkv) * hd, self.H) and self.o_w.shape == (self.H, nh * hd)


def synth_weights(H, nh, nkv, hd, seed=0, std=0.02, norm_jitter=0.1):
    rng = np.random.default_rng(seed)
    qkv = (rng.standard_normal(((nh + 2 * nkv) * hd, H)) * std).astype(np.float32)
    o = (rng.standard_normal((H, nh * hd)) * std).astype(np.float32)
    qn = (1.0 + norm_jitter * rng.standard_normal(hd)).astype(np.float32)
    kn = (1.0 + norm_jitter * rng.standard_normal(hd)).astype(np.float32)
    return AttnWeights(qkv, o, qn, kn, nh, nkv, hd)


def rope_f32(q, k, theta=10000.0, positions=None):
    """q [T][nh][hd], k [T][nkv][hd] -> rotated copies."""
    q, k = O.f32(q).copy(), O.f32(k).copy()
    T, nh, hd = q.shape
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
    lib().hyo_rope_f32(O.fp(q), O.fp(k), T, nh, k.shape[1], hd, theta, None if pos is None else O.ip(pos))
    return q, k


def build_2d_rope(seq, n_elem, text_len, img_h, img_w, base=10000.0):
    cos = np.empty((seq, n_elem), np.float32)
    sin = np.empty((seq, n_elem), np.float32)
    lib().hyo_build_2d_rope(seq, n_elem, text_len, img_h, img_w, base, O.fp(cos), O.fp(sin))
    return cos, sin


def apply_rope_2d(q, k, cos, sin):
    q, k = O.f32(q).copy(), O.f32(k).copy()
    T, nh, hd = q.shape
    lib().hyo_apply_rope_2d_f32(O.fp(q), O.fp(k), O.fp(O.f32(cos)), O.fp(O.f32(sin)), T, nh, k.shape[1], hd)
    return q, k


def attention_forward(w: AttnWeights, x, eps=1e-5, theta=10000.0, positions=None):
    """attention_forward_cpu: returns out [T][H] and the debug q [T][nh][hd],
    k, v [T][nkv][hd]."""
    x = O.f32(x)
    T = x.shape[0]
    out = np.empty((T, w.H), np.float32)
    dq = np.empty((T, w.nh, w.hd), np.float32)
    dk = np.empty((T, w.nkv, w.hd), np.float32)
    dv = np.empty((T, w.nkv, w.hd), np.float32)
    pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.int32)
    lib().hyo_attention_forward(O.fp(x), O.fp(w.qkv_w), O.fp(w.o_w), O.fp(w.q_norm), O.fp(w.k_norm), T, w.H, w.nh,
                                w.nkv, w.hd, eps, theta, None if pos is None else O.ip(pos), O.fp(out), O.fp(dq),
                                O.fp(dk), O.fp(dv))
    return out, dq, dk, dv


class KVCache:
    """The reference's per-layer key / value cache, layout [nkv][max_len][hd]."""

    def __init__(self, nkv, hd, max_len):
        self.k = np.zeros((nkv, max_len, hd), np.float32)
        self.v = np.zeros((nkv, max_len, hd), np.float32)
        self.c = KVCacheC(O.fp(self.k), O.fp(self.v), max_len, 0)

    @property
    def cur_len(self):
        return self.c.cur_len


def attention_cached(w: AttnWeights, x, cache: KVCache, eps=1e-5, cos=None, sin=None):
    x = O.f32(x)
    T = x.shape[0]
    out = np.empty((T, w.H), np.float32)
    cs = None if cos is None else O.f32(cos)
    sn = None if sin is None else O.f32(sin)
    rc = lib().hyo_attention_cached(O.fp(x), O.fp(w.qkv_w), O.fp(w.o_w), O.fp(w.q_norm), O.fp(w.k_norm), T, w.H,
                                    w.nh, w.nkv, w.hd, eps, _fp_or_none(cs), _fp_or_none(sn), C.byref(cache.c),
                                    O.fp(out))
    if rc != 0:
        raise ValueError("cache overflow")
    return out
