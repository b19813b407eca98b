"""CPU-side checks of the C ABI: the library loads, exports every function
include/hy_moe.h declares, and rejects invalid configurations before touching a
device."""
import ctypes as C
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_header(hy):
    syms = hy.header_symbols()
    assert len(syms) >= 30
    L = hy.lib()
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_cxx_mirror_header_lists_reference_names():
    txt = open(os.path.join(ROOT, "include", "hunyuan_moe_full.h")).read()
    for name in ("MoERoutingConfig", "MoEGateOutput", "topkgating_full", "topkgating_easy", "einsum_dispatch",
                 "einsum_combine", "moe_forward_full", "softmax_f32", "topk_f32", "moe_forward_cpu",
                 "swiglu_ffn_f32", "MoEWeights", "rms_norm_f32"):
        assert name in txt, name


def _cfg(hy, **kw):
    c = hy.Config()
    c.hidden, c.intermediate, c.num_experts, c.topk = 256, 128, 16, 4
    c.num_layers, c.max_tokens, c.wtype, c.has_shared, c.norm_topk_prob = 1, 16, hy.Q8_0, 1, 1
    c.routed_scaling_factor = 1.0
    for k, v in kw.items():
        setattr(c, k, v)
    return c


@pytest.mark.parametrize("kw,code", [
    (dict(hidden=100), -1), (dict(intermediate=48), -1), (dict(num_experts=65), -1), (dict(topk=17), -1),
    (dict(topk=0), -1), (dict(max_tokens=0), -1), (dict(max_tokens=20000), -1), (dict(wtype=1), -2),
    (dict(group_limited_greedy=1), -2), (dict(drop_tokens=1), -2), (dict(compute_aux_loss=1), -2),
])
def test_invalid_configs_rejected_before_device(hy, kw, code):
    h = C.c_void_p()
    rc = hy.lib().hy_moe_create(C.byref(_cfg(hy, **kw)), C.byref(h))
    assert rc == code
    assert h.value is None
    assert hy.lib().hy_last_error().decode()
