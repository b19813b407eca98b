"""ctypes bindings for the CPU oracle (oracle/liboracle.so) and the reference build
(oracle/_ref/libhy_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and the benchmark's
CPU-baseline leg as the checker.  The product path never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# HY_ORACLE_LIB names another build of the same sources (the sanitizer test uses it).
LIB_PATH = os.environ.get("HY_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libhy_ref.so")

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
QK = 32
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}

_fp = C.POINTER(C.c_float)
_ip = C.POINTER(C.c_int32)
_up = C.POINTER(C.c_uint32)
_vp = C.c_void_p


class RoutingCfg(C.Structure):
    """MoERoutingConfig (reference src/hunyuan_moe_full.h:25-47)."""
    _fields_ = [
        ("num_experts", C.c_uint32), ("moe_topk", C.c_uint32),
        ("group_limited_greedy", C.c_int32), ("n_group", C.c_uint32), ("topk_group", C.c_uint32),
        ("drop_tokens", C.c_int32), ("random_routing_dropped_token", C.c_int32),
        ("capacity_factor", C.c_float), ("min_capacity", C.c_uint32),
        ("norm_topk_prob", C.c_int32), ("routed_scaling_factor", C.c_float),
        ("compute_aux_loss", C.c_int32),
    ]


class GateFull(C.Structure):
    _fields_ = [
        ("capacity", C.c_uint32), ("aux_loss", C.c_float), ("exp_capacity_rate", C.c_float),
        ("dispatch_mask", C.POINTER(C.c_uint8)), ("combine_weights", _fp),
        ("exp_counts", _ip), ("router_probs", _fp),
    ]


class QLayer(C.Structure):
    _fields_ = [
        ("H", C.c_uint32), ("I", C.c_uint32), ("E", C.c_uint32), ("K", C.c_uint32),
        ("wtype", C.c_int), ("norm_topk_prob", C.c_int), ("routed_scaling_factor", C.c_float),
        ("router", _fp), ("shared_gu", _vp), ("shared_dn", _vp), ("gu", _vp), ("dn", _vp),
        ("n_group", C.c_uint32), ("topk_group", C.c_uint32), ("capacity", C.c_uint32),
    ]


def _load(path):
    if not os.path.exists(path):
        raise OSError(f"{path} is not built (make -C oracle)")
    return C.CDLL(path, mode=os.RTLD_LAZY | os.RTLD_LOCAL)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        L = _load(LIB_PATH)
        sig = {
            "hyo_routing_cfg_default": (None, [C.POINTER(RoutingCfg)]),
            "hyo_fp16_to_fp32": (C.c_float, [C.c_uint16]),
            "hyo_fp32_to_fp16": (C.c_uint16, [C.c_float]),
            "hyo_fp16_to_fp32_ref": (C.c_float, [C.c_uint16]),
            "hyo_quantize_row_q8_0": (None, [_fp, _vp, C.c_size_t]),
            "hyo_quantize_row_q4_0": (None, [_fp, _vp, C.c_size_t]),
            "hyo_dequantize_row_q8_0": (None, [_vp, _fp, C.c_size_t]),
            "hyo_dequantize_row_q4_0": (None, [_vp, _fp, C.c_size_t]),
            "hyo_dequantize_row_q8_0_ref": (None, [_vp, _fp, C.c_size_t]),
            "hyo_dequantize_row_q4_0_ref": (None, [_vp, _fp, C.c_size_t]),
            "hyo_block_dots_q8_0_q8_0": (None, [_vp, _vp, C.c_size_t, _ip]),
            "hyo_block_dots_q4_0_q8_0": (None, [_vp, _vp, C.c_size_t, _ip]),
            "hyo_vec_dot_q8_0_q8_0": (C.c_float, [_vp, _vp, C.c_size_t]),
            "hyo_vec_dot_q4_0_q8_0": (C.c_float, [_vp, _vp, C.c_size_t]),
            "hyo_stream_key": (C.c_uint64, [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32]),
            "hyo_synth_normal": (C.c_float, [C.c_uint64, C.c_uint64, C.c_float]),
            "hyo_synth_fill": (None, [C.c_uint64, C.c_uint64, C.c_size_t, C.c_float, _fp]),
            "hyo_rms_norm_f32": (None, [_fp, _fp, _fp, C.c_uint32, C.c_uint32, C.c_float]),
            "hyo_swiglu_ffn_f32": (None, [_fp, _fp, _fp, _fp, C.c_uint32, C.c_uint32, C.c_uint32]),
            "hyo_softmax_f32": (None, [_fp, C.c_uint32]),
            "hyo_topk_f32": (None, [_fp, C.c_uint32, C.c_uint32, _fp, _ip]),
            "hyo_topkgating_easy": (None, [_fp, C.c_uint32, C.c_uint32, C.c_uint32, _fp, _ip]),
            "hyo_topkgating_full": (C.c_int, [_fp, C.c_uint32, C.POINTER(RoutingCfg), C.POINTER(GateFull)]),
            "hyo_gate_full_free": (None, [C.POINTER(GateFull)]),
            "hyo_einsum_dispatch": (None, [_fp, C.c_uint32, C.c_uint32, _vp, C.c_uint32, C.c_uint32, _fp]),
            "hyo_einsum_combine": (None, [_fp, _fp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _fp]),
            "hyo_router_logits_seq": (None, [_fp, _fp, C.c_uint32, C.c_uint32, C.c_uint32, _fp]),
            "hyo_moe_forward_full": (C.c_int, [_fp, C.c_uint32, C.c_uint32, _fp, _fp, _fp, _fp, _fp,
                                               C.c_uint32, C.c_uint32, C.POINTER(RoutingCfg), _fp]),
            "hyo_moe_forward_cpu": (C.c_int, [_fp, _fp, _fp, _fp, _fp, _fp, C.c_uint32, C.c_uint32,
                                              C.c_uint32, C.c_uint32, C.c_uint32, _fp, _fp, _fp, _ip]),
            "hyo_router_logits_blocked": (None, [_fp, _fp, C.c_uint32, C.c_uint32, C.c_uint32, _fp]),
            "hyo_route_topk": (None, [_fp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int, C.c_float, _fp, _ip]),
            "hyo_route_topk_groups": (None, [_fp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int, C.c_float,
                                             C.c_uint32, C.c_uint32, _fp, _ip, _fp]),
            "hyo_aux_loss_q": (C.c_float, [_fp, _ip, C.c_uint32, C.c_uint32, C.c_uint32]),
            "hyo_drop_capacity": (C.c_uint32, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, C.c_uint32]),
            "hyo_capacity_keep": (None, [_ip, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _vp]),
            "hyo_moe_route_q": (C.c_int, [C.POINTER(QLayer), _fp, C.c_uint32, _fp, _fp, _ip, _fp, _vp, C.c_int]),
            "hyo_moe_forward_q": (C.c_int, [C.POINTER(QLayer), _fp, C.c_uint32, _fp, _fp, _fp, _ip, C.c_int]),
            "hyo_moe_forward_q_rows": (C.c_int, [C.POINTER(QLayer), _fp, C.c_uint32, _up, C.c_uint32, _fp, C.c_int]),
            "hyo_moe_stack_q": (C.c_int, [C.POINTER(QLayer), C.c_uint32, _fp, C.c_uint32, C.c_float, _fp, C.c_int]),
            "hyo_moe_stack_qw": (C.c_int, [C.POINTER(QLayer), C.POINTER(_fp), C.c_uint32, _fp, C.c_uint32,
                                           C.c_float, _fp, C.c_int]),
            "hyo_select_q": (None, [_fp, C.c_uint32, C.c_uint32, _fp, _ip]),
            "hyo_rms_norm_blocked_rows": (None, [_fp, _fp, _fp, C.c_uint32, C.c_uint32, C.c_float]),
            "hyo_free": (None, [_vp]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own hunyuan_moe_full.cpp, built by `make -C oracle ref`."""
    global _ref
    if _ref is None:
        R = _load(REF_PATH)
        sig = {
            "ref_softmax_f32": (None, [_fp, C.c_uint32]),
            "ref_topk_f32": (None, [_fp, C.c_uint32, C.c_uint32, _fp, _ip]),
            "ref_topkgating_easy": (None, [_fp, C.c_uint32, C.c_uint32, C.c_uint32, _fp, _ip]),
            "ref_capacity_bound": (C.c_uint32, [C.c_uint32, C.POINTER(RoutingCfg)]),
            "ref_topkgating_full": (None, [_fp, C.c_uint32, C.POINTER(RoutingCfg), _vp, _fp, _ip, _fp,
                                           _up, _fp, _fp]),
            "ref_einsum_dispatch": (None, [_fp, C.c_uint32, C.c_uint32, _vp, C.c_uint32, C.c_uint32, _fp]),
            "ref_einsum_combine": (None, [_fp, _fp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _fp]),
            "ref_moe_forward_full_noshared": (None, [_fp, C.c_uint32, C.c_uint32, _fp, _fp, _fp, C.c_uint32,
                                                     C.c_uint32, C.POINTER(RoutingCfg), _fp]),
        }
        for name, (res, args) in sig.items():
            f = getattr(R, name)
            f.restype = res
            f.argtypes = args
        _ref = R
    return _ref


# ---------------------------------------------------------------- numpy helpers

def fp(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def ip(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_ip)


def vp(a):
    assert a.flags.c_contiguous
    return C.c_void_p(a.ctypes.data)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def default_cfg(E=64, K=8, **kw):
    c = RoutingCfg()
    lib().hyo_routing_cfg_default(C.byref(c))
    c.num_experts, c.moe_topk = E, K
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def row_bytes(wtype, n):
    if wtype == F32:
        return 4 * n
    return n // QK * BLOCK_BYTES[wtype]


def quantize(x, wtype):
    """Quantize the last axis of x (GGUF blocks), returns uint8 [..., row_bytes]."""
    x = f32(x)
    n = x.shape[-1]
    rows = x.reshape(-1, n)
    out = np.empty((rows.shape[0], row_bytes(wtype, n)), dtype=np.uint8)
    fn = lib().hyo_quantize_row_q8_0 if wtype == Q8_0 else lib().hyo_quantize_row_q4_0
    # one call over the contiguous whole: rows are concatenations of blocks
    fn(fp(rows), vp(out), rows.size)
    return out.reshape(x.shape[:-1] + (out.shape[-1],))


def dequantize(q, wtype, n):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows = q.reshape(-1, q.shape[-1])
    out = np.empty((rows.shape[0], n), dtype=np.float32)
    fn = lib().hyo_dequantize_row_q8_0 if wtype == Q8_0 else lib().hyo_dequantize_row_q4_0
    fn(vp(rows), fp(out), out.size)
    return out.reshape(q.shape[:-1] + (n,))


def synth(seed, layer, tensor, expert, shape, std, idx0=0):
    key = lib().hyo_stream_key(seed, layer, tensor, expert)
    out = np.empty(int(np.prod(shape)), dtype=np.float32)
    lib().hyo_synth_fill(key, idx0, out.size, std, fp(out))
    return out.reshape(shape)


# tensor ids of the synthetic generator (shared with the GPU generator)
T_X, T_ROUTER, T_GU, T_DN = 0, 1, 2, 3


class Layer:
    """One MoE layer's weights in GGUF layout (ggml ne0 = in-features)."""

    def __init__(self, H, I, E, K, wtype, router, shared_gu, shared_dn, gu, dn,
                 norm_topk_prob=True, routed_scaling_factor=1.0, n_group=0, topk_group=0, capacity=0):
        self.H, self.I, self.E, self.K, self.wtype = H, I, E, K, wtype
        self.router = f32(router)
        self.shared_gu = None if shared_gu is None else np.ascontiguousarray(shared_gu)
        self.shared_dn = None if shared_dn is None else np.ascontiguousarray(shared_dn)
        self.gu = np.ascontiguousarray(gu)
        self.dn = np.ascontiguousarray(dn)
        self.norm_topk_prob = norm_topk_prob
        self.routed_scaling_factor = routed_scaling_factor
        # group-limited greedy when both > 0; capacity > 0: token dropping at that capacity
        self.n_group, self.topk_group, self.capacity = n_group, topk_group, capacity

    def c(self):
        s = QLayer()
        s.H, s.I, s.E, s.K, s.wtype = self.H, self.I, self.E, self.K, self.wtype
        s.norm_topk_prob = int(self.norm_topk_prob)
        s.routed_scaling_factor = self.routed_scaling_factor
        s.router = fp(self.router)
        s.shared_gu = vp(self.shared_gu) if self.shared_gu is not None else None
        s.shared_dn = vp(self.shared_dn) if self.shared_dn is not None else None
        s.gu = vp(self.gu)
        s.dn = vp(self.dn)
        s.n_group, s.topk_group, s.capacity = int(self.n_group), int(self.topk_group), int(self.capacity)
        return s

    def dequant(self):
        """F32 copies [E,2I,H], [E,H,I], [2I,H], [H,I] of the (quantized) weights."""
        def dq(a, n):
            if self.wtype == F32:
                return a.view(np.float32).reshape(a.shape[:-1] + (n,)) if a.dtype == np.uint8 else f32(a)
            return dequantize(a, self.wtype, n)
        H, I = self.H, self.I
        gu = dq(self.gu, H).reshape(self.E, 2 * I, H)
        dn = dq(self.dn, I).reshape(self.E, H, I)
        sgu = dq(self.shared_gu, H).reshape(2 * I, H) if self.shared_gu is not None else None
        sdn = dq(self.shared_dn, I).reshape(H, I) if self.shared_dn is not None else None
        return gu, dn, sgu, sdn


def synth_layer(H, I, E, K, wtype, seed=42, layer=0, std=0.02, router_bias=None, shared=True):
    """Seeded random-init layer, weights ~N(0,std) quantized to wtype.

    router_bias: optional [E] additive logit bias folded into input feature 0 (the
    caller sets x[:, 0] = 1 so logits gain bias[e]).
    """
    router = synth(seed, layer, T_ROUTER, 0, (E, H), std)
    if router_bias is not None:
        router[:, 0] = np.asarray(router_bias, dtype=np.float32)

    def mk(tensor, expert, rows, cols, out=None):
        if wtype == F32:   # generated in place: a real-shape F32 layer is ~10 GB
            w = np.empty((rows, cols), np.float32) if out is None else out
            lib().hyo_synth_fill(lib().hyo_stream_key(seed, layer, tensor, expert), 0, w.size, std, fp(w))
            return w
        w = quantize(synth(seed, layer, tensor, expert, (rows, cols), std), wtype)
        if out is not None:
            out[...] = w
        return w

    def stacked(tensor, rows, cols):
        a = np.empty((E, rows, row_bytes(wtype, cols) // (4 if wtype == F32 else 1)),
                     np.float32 if wtype == F32 else np.uint8)
        for e in range(E):
            mk(tensor, e, rows, cols, out=a[e])
        return a

    gu = stacked(T_GU, 2 * I, H)
    dn = stacked(T_DN, H, I)
    sgu = mk(T_GU, E, 2 * I, H) if shared else None
    sdn = mk(T_DN, E, H, I) if shared else None
    return Layer(H, I, E, K, wtype, router, sgu, sdn, gu, dn)


def moe_forward_q(layer: Layer, x, nthreads=1, debug=False):
    x = f32(x)
    T = x.shape[0]
    out = np.empty((T, layer.H), dtype=np.float32)
    lg = np.empty((T, layer.E), dtype=np.float32) if debug else None
    w = np.empty((T, layer.K), dtype=np.float32) if debug else None
    idx = np.empty((T, layer.K), dtype=np.int32) if debug else None
    c = layer.c()
    rc = lib().hyo_moe_forward_q(C.byref(c), fp(x), T, fp(out),
                                 fp(lg) if debug else None, fp(w) if debug else None,
                                 ip(idx) if debug else None, nthreads)
    if rc != 0:
        raise ValueError("hyo_moe_forward_q rejected the layer")
    return (out, lg, w, idx) if debug else out


def moe_forward_q_rows(layer: Layer, x, rows, nthreads=1):
    x = f32(x)
    rows = np.ascontiguousarray(rows, dtype=np.uint32)
    out = np.empty((rows.size, layer.H), dtype=np.float32)
    c = layer.c()
    rc = lib().hyo_moe_forward_q_rows(C.byref(c), fp(x), x.shape[0],
                                      rows.ctypes.data_as(_up), rows.size, fp(out), nthreads)
    if rc != 0:
        raise ValueError("hyo_moe_forward_q_rows rejected the layer")
    return out


def moe_stack_q(layers, x, eps=1e-5, nthreads=1):
    x = f32(x)
    arr = (QLayer * len(layers))(*[l.c() for l in layers])
    out = np.empty_like(x)
    rc = lib().hyo_moe_stack_q(arr, len(layers), fp(x), x.shape[0], eps, fp(out), nthreads)
    if rc != 0:
        raise ValueError("hyo_moe_stack_q rejected the layers")
    return out


def moe_stack_qw(layers, norm_ws, x, eps=1e-5, nthreads=1):
    """The stack with a post-attention RMSNorm weight per layer (None entries: unit)."""
    x = f32(x)
    arr = (QLayer * len(layers))(*[l.c() for l in layers])
    keep = [None if w is None else f32(w) for w in norm_ws]
    ptrs = (_fp * len(layers))(*[None if w is None else fp(w) for w in keep])
    out = np.empty_like(x)
    rc = lib().hyo_moe_stack_qw(arr, ptrs, len(layers), fp(x), x.shape[0], eps, fp(out), nthreads)
    if rc != 0:
        raise ValueError("hyo_moe_stack_qw rejected the layers")
    return out


def rms_norm_blocked(x, w=None, eps=1e-5):
    """RMSNorm in the GPU kernels' blocked sum order (w None: unit weight)."""
    x = f32(x)
    out = np.empty_like(x)
    wk = None if w is None else f32(w)
    lib().hyo_rms_norm_blocked_rows(fp(x), None if wk is None else fp(wk), fp(out), x.shape[0], x.shape[1], eps)
    return out


def router_logits_blocked(x, wr):
    x, wr = f32(x), f32(wr)
    T, H = x.shape
    E = wr.shape[0]
    out = np.empty((T, E), dtype=np.float32)
    lib().hyo_router_logits_blocked(fp(x), fp(wr), T, H, E, fp(out))
    return out


def route_topk_groups(logits, K, norm=True, scale=1.0, n_group=0, topk_group=0):
    """q-semantics routing with group-limited greedy: weights, indices, masked probs."""
    logits = f32(logits)
    T, E = logits.shape
    w = np.empty((T, K), dtype=np.float32)
    idx = np.empty((T, K), dtype=np.int32)
    probs = np.empty((T, E), dtype=np.float32)
    lib().hyo_route_topk_groups(fp(logits), T, E, K, int(norm), scale, n_group, topk_group, fp(w), ip(idx),
                                fp(probs))
    return w, idx, probs


def aux_loss_q(probs, idx):
    probs, idx = f32(probs), np.ascontiguousarray(idx, dtype=np.int32)
    T, E = probs.shape
    return np.float32(lib().hyo_aux_loss_q(fp(probs), ip(idx), T, E, idx.shape[1]))


def drop_capacity(T, E, K, capacity_factor, min_capacity):
    return int(lib().hyo_drop_capacity(T, E, K, capacity_factor, min_capacity))


def capacity_keep(idx, E, capacity):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, K = idx.shape
    keep = np.empty((T, K), dtype=np.uint8)
    lib().hyo_capacity_keep(ip(idx), T, E, K, capacity, vp(keep))
    return keep.astype(bool)


def moe_route_q(layer: Layer, x, nthreads=1):
    """Routing of the whole batch: logits, weights, indices, masked probs, keep [T][K]."""
    x = f32(x)
    T = x.shape[0]
    lg = np.empty((T, layer.E), dtype=np.float32)
    w = np.empty((T, layer.K), dtype=np.float32)
    idx = np.empty((T, layer.K), dtype=np.int32)
    probs = np.empty((T, layer.E), dtype=np.float32)
    keep = np.empty((T, layer.K), dtype=np.uint8)
    c = layer.c()
    rc = lib().hyo_moe_route_q(C.byref(c), fp(x), T, fp(lg), fp(w), ip(idx), fp(probs), vp(keep), nthreads)
    if rc != 0:
        raise ValueError("hyo_moe_route_q rejected the layer")
    return lg, w, idx, probs, keep.astype(bool)


def route_topk(logits, K, norm=True, scale=1.0):
    logits = f32(logits)
    T, E = logits.shape
    w = np.empty((T, K), dtype=np.float32)
    idx = np.empty((T, K), dtype=np.int32)
    lib().hyo_route_topk(fp(logits), T, E, K, int(norm), scale, fp(w), ip(idx))
    return w, idx
