"""Python binding of libhy_moe.so (the C ABI in include/hy_moe.h), for the tests
and the benchmark.  Device memory is handled through the library's own helpers
(hy_malloc / hy_memcpy_*), host arrays are numpy.

The GPU path has no fallback: if libhy_moe.so is missing or no GPU is present the
calls raise.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhy_moe.so")
ROOT = os.path.dirname(HERE)
HEADER = os.path.join(ROOT, "include", "hy_moe.h")
ATTN_HEADER = os.path.join(ROOT, "include", "hy_attn.h")

F32, Q4_0, Q8_0 = 0, 2, 8
PATH_AUTO, PATH_VALU, PATH_MFMA = 0, 1, 2
TENSOR_X, TENSOR_ROUTER, TENSOR_GU, TENSOR_DN = 0, 1, 2, 3


class HyError(RuntimeError):
    pass


class Config(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("intermediate", C.c_uint32), ("num_experts", C.c_uint32),
        ("topk", C.c_uint32), ("num_layers", C.c_uint32), ("max_tokens", C.c_uint32),
        ("wtype", C.c_int32), ("has_shared", C.c_int32), ("norm_topk_prob", C.c_int32),
        ("routed_scaling_factor", C.c_float), ("group_limited_greedy", C.c_int32),
        ("drop_tokens", C.c_int32), ("compute_aux_loss", C.c_int32), ("device", C.c_int32),
        ("n_group", C.c_uint32), ("topk_group", C.c_uint32), ("capacity_factor", C.c_float),
        ("min_capacity", C.c_uint32),
    ]


class AttnConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("n_heads", C.c_uint32), ("n_kv_heads", C.c_uint32), ("head_dim", C.c_uint32),
        ("num_layers", C.c_uint32), ("max_tokens", C.c_uint32), ("max_cache", C.c_uint32),
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("device", C.c_int32),
    ]


class ModelConfig(C.Structure):
    _fields_ = [("moe", Config), ("attn", AttnConfig), ("vocab", C.c_uint32)]


_vp = C.c_void_p
_u32, _i32, _u64, _f = C.c_uint32, C.c_int32, C.c_uint64, C.c_float
_SIGS = {
    "hy_last_error": (C.c_char_p, []),
    "hy_moe_create": (C.c_int, [C.POINTER(Config), C.POINTER(_vp)]),
    "hy_moe_destroy": (C.c_int, [_vp]),
    "hy_moe_layer_bytes": (C.c_size_t, [_vp]),
    "hy_moe_upload_layer": (C.c_int, [_vp, _u32, _vp, _vp, _vp, _vp, _vp]),
    "hy_moe_synth_layer": (C.c_int, [_vp, _u32, _u64, _f, _vp]),
    "hy_moe_set_ffn_norm": (C.c_int, [_vp, _u32, _vp]),
    "hy_attn_create": (C.c_int, [C.POINTER(AttnConfig), C.POINTER(_vp)]),
    "hy_attn_destroy": (C.c_int, [_vp]),
    "hy_attn_upload": (C.c_int, [_vp, _u32, _vp, _vp, _vp, _vp]),
    "hy_attn_upload_gguf": (C.c_int, [_vp, _u32, _vp, _u32]),
    "hy_attn_synth_layer": (C.c_int, [_vp, _u32, _u64, _f]),
    "hy_attn_forward": (C.c_int, [_vp, _u32, _vp, _u32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "hy_attn_forward_cached": (C.c_int, [_vp, _u32, _vp, _u32, _vp, _vp, _vp, _vp]),
    "hy_attn_cache_reset": (C.c_int, [_vp]),
    "hy_attn_cache_len": (C.c_int, [_vp, _u32, C.POINTER(_u32)]),
    "hy_model_create": (C.c_int, [C.POINTER(ModelConfig), C.POINTER(_vp)]),
    "hy_model_destroy": (C.c_int, [_vp]),
    "hy_model_attn": (_vp, [_vp]),
    "hy_model_moe": (_vp, [_vp]),
    "hy_model_upload_globals": (C.c_int, [_vp, _vp, _vp, _vp]),
    "hy_model_upload_globals_gguf": (C.c_int, [_vp, _vp]),
    "hy_model_synth_globals": (C.c_int, [_vp, _u64, _f]),
    "hy_model_forward": (C.c_int, [_vp, _vp, _u32, _vp, _vp, _vp]),
    "hy_model_forward_hidden": (C.c_int, [_vp, _vp, _u32, _vp, _u32, _vp, _vp]),
    "hy_build_2d_rope": (C.c_int, [_u32, _u32, _u32, _u32, _u32, _f, _vp, _vp, _vp]),
    "hy_attn_set_input_norm": (C.c_int, [_vp, _u32, _vp]),
    "hy_decoder_layer_forward": (C.c_int, [_vp, _u32, _vp, _u32, _vp, _u32, _vp, _vp, _vp, _vp]),
    "hy_lm_head_f32": (C.c_int, [_vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp]),
    "hy_attn_set_decode_waves": (C.c_int, [_vp, _u32]),
    "hy_attn_prof_enable": (C.c_int, [_vp, _i32]),
    "hy_attn_prof_read": (C.c_int, [_vp, _u32, C.POINTER(_u64), C.POINTER(C.c_double)]),
    "hy_moe_forward": (C.c_int, [_vp, _u32, _vp, _u32, _vp, _vp]),
    "hy_moe_forward_debug": (C.c_int, [_vp, _u32, _vp, _u32, _vp, _vp, _vp, _vp, _vp]),
    "hy_moe_stack_forward": (C.c_int, [_vp, _u32, _u32, _vp, _u32, _f, _vp, _vp]),
    "hy_moe_set_path": (C.c_int, [_vp, _i32]),
    "hy_router_topk": (C.c_int, [_vp, _vp, _u32, _u32, _u32, _u32, _i32, _f, _vp, _vp, _vp, _vp]),
    "hy_topkgating_easy": (C.c_int, [_vp, _u32, _u32, _u32, _vp, _vp, _vp]),
    "hy_topk_rows": (C.c_int, [_vp, _u32, _u32, _u32, _vp, _vp, _vp]),
    "hy_route_logits_groups": (C.c_int, [_vp, _u32, _u32, _u32, _i32, _f, _u32, _u32, _vp, _vp, _vp, _vp]),
    "hy_aux_loss": (C.c_int, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "hy_moe_last_gate": (C.c_int, [_vp, C.POINTER(_f), C.POINTER(_u32), C.POINTER(_f)]),
    "hy_softmax_rows": (C.c_int, [_vp, _u32, _u32, _vp]),
    "hy_quantize_q8_0": (C.c_int, [_vp, _u32, _u32, _vp, _vp]),
    "hy_dequantize": (C.c_int, [_i32, _vp, C.c_size_t, _vp, _vp]),
    "hy_block_dots": (C.c_int, [_i32, _vp, _vp, _u32, _u32, _i32, _vp, _vp]),
    "hy_rms_norm": (C.c_int, [_vp, _u32, _u32, _f, _vp, _vp]),
    "hy_device_count": (C.c_int, [C.POINTER(C.c_int)]),
    "hy_set_device": (C.c_int, [C.c_int]),
    "hy_malloc": (C.c_int, [C.POINTER(_vp), C.c_size_t]),
    "hy_free": (C.c_int, [_vp]),
    "hy_memcpy_h2d": (C.c_int, [_vp, _vp, C.c_size_t]),
    "hy_memcpy_d2h": (C.c_int, [_vp, _vp, C.c_size_t]),
    "hy_memset": (C.c_int, [_vp, C.c_int, C.c_size_t]),
    "hy_copy_d2d": (C.c_int, [_vp, _vp, C.c_size_t, _vp]),
    "hy_gguf_open": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "hy_gguf_close": (C.c_int, [_vp]),
    "hy_gguf_n_tensors": (C.c_int, [_vp, C.POINTER(C.c_uint64)]),
    "hy_gguf_tensor": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_int32), C.POINTER(C.c_uint32),
                                 C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(_vp)]),
    "hy_gguf_tensor_f32": (C.c_int, [_vp, C.c_char_p, _vp, C.c_uint64]),
    "hy_gguf_get_u32": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_uint32)]),
    "hy_gguf_get_f32": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_float)]),
    "hy_moe_upload_layer_gguf": (C.c_int, [_vp, C.c_uint32, _vp, C.c_uint32]),
    "hy_dispatch_pairs": (C.c_int, [_vp, _vp, C.c_uint32, C.c_uint32, C.c_uint32, _vp, _vp, _vp, _vp]),
    "hy_dispatch_pairs_noalloc": (C.c_int, [_vp, _vp, C.c_uint32, C.c_uint32, C.c_uint32, _vp, _vp, _vp, _vp]),
    "hy_device_synchronize": (C.c_int, []),
    "hy_stream_create": (C.c_int, [C.POINTER(_vp)]),
    "hy_stream_destroy": (C.c_int, [_vp]),
    "hy_stream_synchronize": (C.c_int, [_vp]),
    "hy_event_create": (C.c_int, [C.POINTER(_vp)]),
    "hy_event_destroy": (C.c_int, [_vp]),
    "hy_event_record": (C.c_int, [_vp, _vp]),
    "hy_event_elapsed_ms": (C.c_int, [_vp, _vp, C.POINTER(C.c_float)]),
    "hy_graph_begin": (C.c_int, [_vp]),
    "hy_graph_end": (C.c_int, [_vp, C.POINTER(_vp)]),
    "hy_graph_launch": (C.c_int, [_vp, _vp]),
    "hy_graph_destroy": (C.c_int, [_vp]),
    "hy_synth_fill": (C.c_int, [_vp, C.c_size_t, _u64, _u32, _u32, _u32, _f, _vp]),
    "hy_moe_prof_enable": (C.c_int, [_vp, _i32]),
    "hy_moe_prof_read": (C.c_int, [_vp, _i32, C.POINTER(C.c_uint64), C.POINTER(C.c_double)]),
    "hy_moe_prof_name": (C.c_char_p, [_i32]),
    "hy_moe_prof_count": (_i32, []),
    "hy_moe_last_routing": (C.c_int, [_vp, C.POINTER(_u32), _vp]),
}

_lib = None


def lib():
    """Load libhy_moe.so; raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HyError(f"{LIB_PATH} is not built: run python hunyuan-image-3-80b.cpp_amd/build.py")
        L = C.CDLL(LIB_PATH, mode=os.RTLD_LAZY | os.RTLD_LOCAL)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise HyError(f"hy error {rc}: {lib().hy_last_error().decode()}")


def device_count():
    n = C.c_int(0)
    rc = lib().hy_device_count(C.byref(n))
    return n.value if rc == 0 else 0


# ------------------------------------------------------------------ device buffers

class Buf:
    """Device allocation of `nbytes`, freed with the object."""

    def __init__(self, nbytes, dtype=np.float32, shape=None):
        self.nbytes = int(max(nbytes, 1))
        self.dtype = np.dtype(dtype)
        self.shape = shape
        p = _vp()
        check(lib().hy_malloc(C.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, a.dtype, a.shape)
        check(lib().hy_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes))
        return b

    @classmethod
    def empty(cls, shape, dtype=np.float32):
        dt = np.dtype(dtype)
        return cls(int(np.prod(shape)) * dt.itemsize, dt, tuple(shape))

    def zero(self):
        check(lib().hy_memset(self.ptr, 0, self.nbytes))
        return self

    def numpy(self, shape=None, dtype=None):
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        shp = shape if shape is not None else (self.shape if self.shape is not None else (self.nbytes // dt.itemsize,))
        out = np.empty(shp, dtype=dt)
        check(lib().hy_device_synchronize())
        check(lib().hy_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            lib().hy_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync():
    check(lib().hy_device_synchronize())


class Stream:
    """A created HIP stream (hy_stream_create); .h is passed as the stream argument."""

    def __init__(self):
        self.h = C.c_void_p()
        check(lib().hy_stream_create(C.byref(self.h)))

    def synchronize(self):
        check(lib().hy_stream_synchronize(self.h))

    def close(self):
        if self.h:
            check(lib().hy_stream_destroy(self.h))
            self.h = C.c_void_p()


class Graph:
    """Work issued on `stream` by fn() captured once (hy_graph_begin / hy_graph_end) and
    replayed with launch()."""

    def __init__(self, stream: Stream, fn):
        self.stream = stream
        self.h = C.c_void_p()
        check(lib().hy_graph_begin(stream.h))
        try:
            fn()
        except Exception:
            g = C.c_void_p()
            lib().hy_graph_end(stream.h, C.byref(g))   # end the capture; keep the first error
            if g:
                lib().hy_graph_destroy(g)
            raise
        check(lib().hy_graph_end(stream.h, C.byref(self.h)))

    def launch(self):
        check(lib().hy_graph_launch(self.h, self.stream.h))

    def close(self):
        if self.h:
            check(lib().hy_graph_destroy(self.h))
            self.h = C.c_void_p()


# ------------------------------------------------------------------ context

class Moe:
    """A resident MoE stack (hy_moe_ctx)."""

    def __init__(self, H, I, E, K, wtype, num_layers=1, max_tokens=64, has_shared=True, norm_topk_prob=True,
                 routed_scaling_factor=1.0, device=0, group_limited_greedy=0, n_group=0, topk_group=0,
                 drop_tokens=0, capacity_factor=1.0, min_capacity=0, compute_aux_loss=0):
        c = Config()
        c.hidden, c.intermediate, c.num_experts, c.topk = H, I, E, K
        c.num_layers, c.max_tokens, c.wtype = num_layers, max_tokens, wtype
        c.has_shared, c.norm_topk_prob = int(has_shared), int(norm_topk_prob)
        c.routed_scaling_factor = routed_scaling_factor
        c.group_limited_greedy, c.n_group, c.topk_group = int(group_limited_greedy), n_group, topk_group
        c.drop_tokens, c.capacity_factor, c.min_capacity = int(drop_tokens), capacity_factor, min_capacity
        c.compute_aux_loss = int(compute_aux_loss)
        c.device = device
        self.cfg = c
        self.H, self.I, self.E, self.K, self.wtype = H, I, E, K, wtype
        self.max_tokens = max_tokens
        h = _vp()
        check(lib().hy_moe_create(C.byref(c), C.byref(h)))
        self.h = h.value

    def close(self):
        if getattr(self, "h", None) and getattr(self, "owned", True):
            lib().hy_moe_destroy(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def layer_bytes(self):
        return lib().hy_moe_layer_bytes(self.h)

    def upload(self, layer_idx, layer):
        """layer: an oracle Layer (GGUF-layout numpy arrays)."""
        def p(a):
            return None if a is None else np.ascontiguousarray(a).ctypes.data
        keep = [np.ascontiguousarray(a) for a in (layer.router, layer.shared_gu, layer.shared_dn, layer.gu, layer.dn)
                if a is not None]
        check(lib().hy_moe_upload_layer(self.h, layer_idx, p(layer.router), p(layer.shared_gu), p(layer.shared_dn),
                                        p(layer.gu), p(layer.dn)))
        del keep

    def upload_gguf(self, layer_idx, gguf, block):
        """Upload layer layer_idx from block `block` of an open Gguf file."""
        check(lib().hy_moe_upload_layer_gguf(self.h, layer_idx, gguf.h, block))

    def synth(self, layer_idx, seed=42, std=0.02, router_bias=None):
        b = None
        if router_bias is not None:
            b = np.ascontiguousarray(router_bias, dtype=np.float32)
        check(lib().hy_moe_synth_layer(self.h, layer_idx, seed, std, None if b is None else b.ctypes.data))

    def set_ffn_norm(self, layer_idx, w=None):
        """Post-attention RMSNorm weight [H] of a layer (None: unit weight)."""
        if w is None:
            check(lib().hy_moe_set_ffn_norm(self.h, layer_idx, None))
            return
        w = np.ascontiguousarray(w, dtype=np.float32)
        if w.shape != (self.H,):
            raise ValueError(f"ffn_norm weight must have shape ({self.H},), got {w.shape}")
        check(lib().hy_moe_set_ffn_norm(self.h, layer_idx, w.ctypes.data))

    def forward(self, layer_idx, x: Buf, T, out: Buf, stream=None):
        check(lib().hy_moe_forward(self.h, layer_idx, x.ptr, T, out.ptr, stream))

    def forward_debug(self, layer_idx, x: Buf, T, out: Buf, lg: Buf, w: Buf, idx: Buf, stream=None):
        check(lib().hy_moe_forward_debug(self.h, layer_idx, x.ptr, T, out.ptr, lg.ptr if lg else None,
                                         w.ptr if w else None, idx.ptr if idx else None, stream))

    def stack_forward(self, first, n, x: Buf, T, eps, out: Buf, stream=None):
        check(lib().hy_moe_stack_forward(self.h, first, n, x.ptr, T, eps, out.ptr, stream))

    def set_path(self, path):
        """0 = auto, 1 = VALU dot4 kernels, 2 = int8 MFMA grouped GEMM."""
        check(lib().hy_moe_set_path(self.h, path))

    def prof_enable(self, on=True):
        check(lib().hy_moe_prof_enable(self.h, int(on)))

    def prof_read(self):
        res = {}
        for k in range(lib().hy_moe_prof_count()):
            n = C.c_uint64()
            ms = C.c_double()
            check(lib().hy_moe_prof_read(self.h, k, C.byref(n), C.byref(ms)))
            res[lib().hy_moe_prof_name(k).decode()] = (n.value, ms.value)
        return res

    def last_routing(self):
        d = C.c_uint32()
        counts = np.zeros(self.E, dtype=np.int32)
        check(lib().hy_moe_last_routing(self.h, C.byref(d), counts.ctypes.data))
        return d.value, counts

    def last_gate(self):
        """(aux_loss, expert_capacity, exp_capacity_rate) of the last forward."""
        aux, cap, rate = C.c_float(), C.c_uint32(), C.c_float()
        check(lib().hy_moe_last_gate(self.h, C.byref(aux), C.byref(cap), C.byref(rate)))
        return np.float32(aux.value), cap.value, np.float32(rate.value)

    # convenience: host in, host out
    def run(self, layer_idx, x, debug=False):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        xb = Buf.from_array(x)
        ob = Buf.empty((T, self.H))
        if not debug:
            self.forward(layer_idx, xb, T, ob)
            return ob.numpy()
        lg = Buf.empty((T, self.E))
        w = Buf.empty((T, self.K))
        idx = Buf.empty((T, self.K), np.int32)
        self.forward_debug(layer_idx, xb, T, ob, lg, w, idx)
        return ob.numpy(), lg.numpy(), w.numpy(), idx.numpy()


# ------------------------------------------------------------------ stateless kernels

def router_topk(x, wr, K, norm=True, scale=1.0):
    x = np.ascontiguousarray(x, np.float32)
    wr = np.ascontiguousarray(wr, np.float32)
    T, H = x.shape
    E = wr.shape[0]
    xb, wb = Buf.from_array(x), Buf.from_array(wr)
    lg, w, idx = Buf.empty((T, E)), Buf.empty((T, K)), Buf.empty((T, K), np.int32)
    check(lib().hy_router_topk(xb.ptr, wb.ptr, T, H, E, K, int(norm), scale, lg.ptr, w.ptr, idx.ptr, None))
    return lg.numpy(), w.numpy(), idx.numpy()


def topkgating_easy(logits, K):
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    lb = Buf.from_array(logits)
    w, idx = Buf.empty((T, K)), Buf.empty((T, K), np.int32)
    check(lib().hy_topkgating_easy(lb.ptr, T, E, K, w.ptr, idx.ptr, None))
    return w.numpy(), idx.numpy()


def topk_rows(x, k):
    """topk_f32 over each row: values and indices [rows][k]."""
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    xb = Buf.from_array(x)
    v, i = Buf.empty((rows, k)), Buf.empty((rows, k), np.int32)
    check(lib().hy_topk_rows(xb.ptr, rows, n, k, v.ptr, i.ptr, None))
    return v.numpy(), i.numpy()


def route_logits_groups(logits, K, norm=1, scale=1.0, n_group=0, topk_group=0):
    """Weights, indices and the masked gates of topkgating_full's selection."""
    logits = np.ascontiguousarray(logits, np.float32)
    T, E = logits.shape
    lb = Buf.from_array(logits)
    w, idx, p = Buf.empty((T, K)), Buf.empty((T, K), np.int32), Buf.empty((T, E))
    check(lib().hy_route_logits_groups(lb.ptr, T, E, K, int(norm), scale, n_group, topk_group, w.ptr, idx.ptr,
                                       p.ptr, None))
    return w.numpy(), idx.numpy(), p.numpy()


def aux_loss(probs, counts):
    probs = np.ascontiguousarray(probs, np.float32)
    counts = np.ascontiguousarray(counts, np.int32)
    T, E = probs.shape
    pb, cb, ob = Buf.from_array(probs), Buf.from_array(counts), Buf.empty((1,))
    check(lib().hy_aux_loss(pb.ptr, cb.ptr, T, E, ob.ptr, None))
    return np.float32(ob.numpy()[0])


def softmax_rows(x):
    x = np.ascontiguousarray(x, np.float32)
    b = Buf.from_array(x)
    check(lib().hy_softmax_rows(b.ptr, x.shape[0], x.shape[1], None))
    return b.numpy()


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    xb = Buf.from_array(x)
    ob = Buf.empty((rows, n // 32 * 34), np.uint8)
    check(lib().hy_quantize_q8_0(xb.ptr, rows, n, ob.ptr, None))
    return ob.numpy()


def dequantize(blocks, wtype, n):
    bb = Buf.from_array(np.ascontiguousarray(blocks))
    ob = Buf.empty((n,))
    check(lib().hy_dequantize(wtype, bb.ptr, n, ob.ptr, None))
    return ob.numpy()


def block_dots(wtype, w_blocks, x_blocks, rows, n, path=0):
    wb = Buf.from_array(np.ascontiguousarray(w_blocks))
    xb = Buf.from_array(np.ascontiguousarray(x_blocks))
    ob = Buf.empty((rows, n // 32), np.int32)
    check(lib().hy_block_dots(wtype, wb.ptr, xb.ptr, rows, n, path, ob.ptr, None))
    return ob.numpy()


def rms_norm(x, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    xb = Buf.from_array(x)
    ob = Buf.empty(x.shape)
    check(lib().hy_rms_norm(xb.ptr, x.shape[0], x.shape[1], eps, ob.ptr, None))
    return ob.numpy()


def synth_fill(n, seed, layer, tensor, expert, std):
    b = Buf.empty((n,))
    check(lib().hy_synth_fill(b.ptr, n, seed, layer, tensor, expert, std, None))
    return b.numpy()


def header_symbols(path=HEADER):
    """Function names declared in a C header (default include/hy_moe.h)."""
    import re
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(hy_[a-z_0-9]+)\s*\(", txt, flags=re.M)))


class Gguf:
    """A GGUF file opened by the library's reader (memory mapped)."""

    def __init__(self, path):
        h = _vp()
        check(lib().hy_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h.value

    def n_tensors(self):
        n = C.c_uint64()
        check(lib().hy_gguf_n_tensors(self.h, C.byref(n)))
        return n.value

    def tensor(self, name):
        """(ggml_type, n_dims, ne[4], nbytes, bytes or None)"""
        t, nd, nb, d = C.c_int32(), C.c_uint32(), C.c_uint64(), _vp()
        ne = (C.c_uint64 * 4)()
        check(lib().hy_gguf_tensor(self.h, name.encode(), C.byref(t), C.byref(nd), ne, C.byref(nb), C.byref(d)))
        data = C.string_at(d.value, nb.value) if d.value else None
        return t.value, nd.value, list(ne), nb.value, data

    def tensor_f32(self, name):
        """The tensor's values as f32, shape (ne[n_dims-1], ..., ne[0])."""
        _, nd, ne, _, _ = self.tensor(name)
        out = np.empty(int(np.prod(ne)), np.float32)
        check(lib().hy_gguf_tensor_f32(self.h, name.encode(), out.ctypes.data, out.size))
        return out.reshape(tuple(reversed(ne[:nd])))

    def get_u32(self, key):
        v = C.c_uint32()
        check(lib().hy_gguf_get_u32(self.h, key.encode(), C.byref(v)))
        return v.value

    def get_f32(self, key):
        v = C.c_float()
        check(lib().hy_gguf_get_f32(self.h, key.encode(), C.byref(v)))
        return v.value

    def close(self):
        if self.h:
            lib().hy_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


ATTN_KERNELS = ("qkv_proj", "rope_qknorm", "attention", "o_proj")


class Attn:
    """Resident attention layers (include/hy_attn.h): weights, key / value caches and
    the fp32 kernels of attention_forward_cpu and the KV-cache branch.  `layer`
    arguments default to 0 (single-layer use)."""

    def __init__(self, H, nh, nkv, hd, max_tokens, max_cache=0, eps=1e-5, theta=10000.0, device=0, num_layers=1,
                 handle=None):
        self.H, self.nh, self.nkv, self.hd = H, nh, nkv, hd
        self.owned = handle is None
        if handle is not None:
            self.h = handle
            return
        cfg = AttnConfig(H, nh, nkv, hd, num_layers, max_tokens, max_cache, eps, theta, device)
        h = _vp()
        check(lib().hy_attn_create(C.byref(cfg), C.byref(h)))
        self.h = h

    def close(self):
        if self.h and self.owned:
            check(lib().hy_attn_destroy(self.h))
        self.h = None

    def upload(self, qkv_w, o_w, q_norm, k_norm, layer=0):
        arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (qkv_w, o_w, q_norm, k_norm)]
        nq, nk = self.nh * self.hd, self.nkv * self.hd
        want = [(nq + 2 * nk, self.H), (self.H, nq), (self.hd,), (self.hd,)]
        for a, w in zip(arrs, want):
            if a.shape != w:
                raise ValueError(f"attention weight shape {a.shape}, want {w}")
        check(lib().hy_attn_upload(self.h, layer, *[a.ctypes.data for a in arrs]))

    def upload_gguf(self, layer, gguf, block):
        check(lib().hy_attn_upload_gguf(self.h, layer, gguf.h, block))

    def synth(self, layer=0, seed=42, std=0.02):
        check(lib().hy_attn_synth_layer(self.h, layer, seed, std))

    def forward(self, x: Buf, T, out: Buf, positions=None, dq=None, dk=None, dv=None, stream=None, layer=0):
        check(lib().hy_attn_forward(self.h, layer, x.ptr, T, positions.ptr if positions is not None else None,
                                    out.ptr, dq.ptr if dq is not None else None, dk.ptr if dk is not None else None,
                                    dv.ptr if dv is not None else None, stream))

    def forward_cached(self, x: Buf, T, out: Buf, cos=None, sin=None, stream=None, layer=0):
        check(lib().hy_attn_forward_cached(self.h, layer, x.ptr, T, cos.ptr if cos is not None else None,
                                           sin.ptr if sin is not None else None, out.ptr, stream))

    def set_input_norm(self, w=None, layer=0):
        """input_layernorm weight [H] (None: unit) for decoder_layer_forward."""
        if w is None:
            check(lib().hy_attn_set_input_norm(self.h, layer, None))
            return
        w = np.ascontiguousarray(w, dtype=np.float32)
        if w.shape != (self.H,):
            raise ValueError(f"input norm weight must have shape ({self.H},), got {w.shape}")
        check(lib().hy_attn_set_input_norm(self.h, layer, w.ctypes.data))

    def decoder_layer_forward(self, moe, moe_layer, x: Buf, T, out: Buf, positions=None, debug_h=None,
                              stream=None, layer=0):
        """decoder_layer_forward_cpu: out = h + MoE(RMSNorm(h)), h = x + attention(RMSNorm(x))."""
        check(lib().hy_decoder_layer_forward(self.h, layer, moe.h, moe_layer, x.ptr, T,
                                             positions.ptr if positions is not None else None, out.ptr,
                                             debug_h.ptr if debug_h is not None else None, stream))

    def cache_reset(self):
        check(lib().hy_attn_cache_reset(self.h))

    def cache_len(self, layer=0):
        n = _u32()
        check(lib().hy_attn_cache_len(self.h, layer, C.byref(n)))
        return n.value

    def set_decode_waves(self, max_waves):
        check(lib().hy_attn_set_decode_waves(self.h, max_waves))

    def prof_enable(self, on):
        check(lib().hy_attn_prof_enable(self.h, 1 if on else 0))

    def prof_read(self):
        out = {}
        for k, name in enumerate(ATTN_KERNELS):
            n, ms = _u64(), C.c_double()
            check(lib().hy_attn_prof_read(self.h, k, C.byref(n), C.byref(ms)))
            out[name] = (n.value, ms.value)
        return out

    def run(self, x, positions=None, debug=False, layer=0):
        """Host convenience: x [T][H] -> out (and q, k, v when debug)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        xb, ob = Buf.from_array(x), Buf.empty((T, self.H))
        pb = Buf.from_array(np.ascontiguousarray(positions, dtype=np.int32)) if positions is not None else None
        dq = Buf.empty((T, self.nh, self.hd)) if debug else None
        dk = Buf.empty((T, self.nkv, self.hd)) if debug else None
        dv = Buf.empty((T, self.nkv, self.hd)) if debug else None
        self.forward(xb, T, ob, pb, dq, dk, dv, layer=layer)
        if debug:
            return ob.numpy(), dq.numpy(), dk.numpy(), dv.numpy()
        return ob.numpy()


class Model:
    """The resident backbone (HunyuanFullModel): embedding -> decoder layers -> final
    norm -> lm_head.  .attn / .moe are views of its two layer contexts."""

    def __init__(self, H, I, E, K, wtype, nh, nkv, hd, vocab, num_layers, max_tokens, eps=1e-5, theta=10000.0,
                 device=0, has_shared=True):
        mc = Config(H, I, E, K, num_layers, max_tokens, wtype, 1 if has_shared else 0, 1, 1.0, 0, 0, 0, device)
        ac = AttnConfig(H, nh, nkv, hd, num_layers, max_tokens, 0, eps, theta, device)
        cfg = ModelConfig(mc, ac, vocab)
        h = _vp()
        check(lib().hy_model_create(C.byref(cfg), C.byref(h)))
        self.h = h
        self.H, self.V, self.L = H, vocab, num_layers
        self.attn = Attn(H, nh, nkv, hd, max_tokens, handle=_vp(lib().hy_model_attn(h)))
        self.moe = Moe.__new__(Moe)
        self.moe.h = lib().hy_model_moe(h)
        self.moe.H, self.moe.I, self.moe.E, self.moe.K, self.moe.wtype = H, I, E, K, wtype
        self.moe.owned = False

    def close(self):
        if self.h:
            check(lib().hy_model_destroy(self.h))
            self.h = None

    def upload_globals(self, embedding=None, final_norm=None, lm_head=None):
        arrs = [None if a is None else np.ascontiguousarray(a, dtype=np.float32)
                for a in (embedding, final_norm, lm_head)]
        check(lib().hy_model_upload_globals(self.h, *[None if a is None else a.ctypes.data for a in arrs]))

    def upload_globals_gguf(self, gguf):
        check(lib().hy_model_upload_globals_gguf(self.h, gguf.h))

    def synth_globals(self, seed=42, std=0.02):
        check(lib().hy_model_synth_globals(self.h, seed, std))

    def forward(self, ids: Buf, T, logits: Buf, positions=None, stream=None):
        check(lib().hy_model_forward(self.h, ids.ptr, T, positions.ptr if positions is not None else None,
                                     logits.ptr, stream))

    def forward_hidden(self, embeds: Buf, T, hidden: Buf, n_layers=0, positions=None, stream=None):
        check(lib().hy_model_forward_hidden(self.h, embeds.ptr, T, positions.ptr if positions is not None else None,
                                            n_layers, hidden.ptr, stream))


def build_2d_rope(seq, n_elem, text_len, img_h, img_w, base=10000.0):
    """Device rotary tables (cos, sin) as Bufs [seq][n_elem]."""
    cos, sin = Buf.empty((seq, n_elem)), Buf.empty((seq, n_elem))
    check(lib().hy_build_2d_rope(seq, n_elem, text_len, img_h, img_w, base, cos.ptr, sin.ptr, None))
    return cos, sin


def lm_head_f32(x, w, resid=None):
    """Host convenience over hy_lm_head_f32: x [T][H] . w[V][H]^T (+ resid)."""
    x, w = np.ascontiguousarray(x, dtype=np.float32), np.ascontiguousarray(w, dtype=np.float32)
    T, Hd = x.shape
    V = w.shape[0]
    xb, wb, ob = Buf.from_array(x), Buf.from_array(w), Buf.empty((T, V))
    rb = Buf.from_array(np.ascontiguousarray(resid, dtype=np.float32)) if resid is not None else None
    check(lib().hy_lm_head_f32(xb.ptr, wb.ptr, rb.ptr if rb is not None else None, T, Hd, V, ob.ptr, None))
    return ob.numpy()
