"""CPU-side checks of the C ABI: the library loads, exports every function
include/hy_moe.h declares, and rejects invalid configurations before touching a
device."""
import ctypes as C
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_header(hy):
    syms = hy.header_symbols()
    assert len(syms) >= 30
    L = hy.lib()
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_library_exports_attention_header(hy):
    syms = hy.header_symbols(hy.ATTN_HEADER)
    assert len(syms) >= 10
    L = hy.lib()
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_attention_config_rejected_before_device(hy):
    """Unsupported shapes are refused before any device call."""
    for kw in (dict(hd=96), dict(nh=8, nkv=4), dict(max_tokens=0)):
        args = dict(H=256, nh=8, nkv=2, hd=64, max_tokens=16)
        args.update(kw)
        with pytest.raises(hy.HyError):
            hy.Attn(args["H"], args["nh"], args["nkv"], args["hd"], args["max_tokens"])


def test_cxx_mirror_header_lists_reference_names():
    txt = open(os.path.join(ROOT, "include", "hunyuan_moe_full.h")).read()
    for name in ("MoERoutingConfig", "MoEGateOutput", "topkgating_full", "topkgating_easy", "einsum_dispatch",
                 "einsum_combine", "moe_forward_full", "softmax_f32", "topk_f32"):
        assert name in txt, name
    model = open(os.path.join(ROOT, "include", "hunyuan_model_moe.h")).read()
    for name in ("HunyuanConfig", "moe_forward_cpu", "swiglu_ffn_f32", "MoEWeights", "rms_norm_f32",
                 "compute_derived", "qkv_total"):
        assert name in model, name


def test_cxx_mirror_headers_compile_with_reference_layout(tmp_path):
    """Both mirror headers compile together, and HunyuanConfig / MoEWeights have the
    reference's field order (offsets of the last fields pin the layout)."""
    import subprocess
    src = tmp_path / "t.cpp"
    src.write_text(
        '#include "hunyuan_model_moe.h"\n#include "hunyuan_moe_full.h"\n#include <cstddef>\n'
        'static_assert(offsetof(HunyuanConfig, rms_norm_eps) == 48, "");\n'
        'static_assert(offsetof(HunyuanConfig, use_qk_norm) == 56, "");\n'
        'static_assert(offsetof(HunyuanConfig, num_kv_groups) == 60, "");\n'
        'static_assert(sizeof(HunyuanConfig) == 76, "");\n'
        'static_assert(offsetof(MoEWeights, num_experts) == 4 * sizeof(std::vector<float>), "");\n'
        'int main() { HunyuanConfig c; c.compute_derived(); return c.qkv_total == 6144 ? 0 : 1; }\n')
    exe = tmp_path / "t"
    subprocess.run(["g++", "-std=c++17", f"-I{os.path.join(ROOT, 'include')}", str(src), "-o", str(exe)], check=True)
    assert subprocess.run([str(exe)]).returncode == 0


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
    (dict(group_limited_greedy=1, n_group=8, topk_group=65), -1),
    (dict(drop_tokens=1, capacity_factor=-1.0), -1), (dict(drop_tokens=1, capacity_factor=float("nan")), -1),
    (dict(drop_tokens=1, capacity_factor=1e30), -1),
])
def test_invalid_configs_rejected_before_device(hy, kw, code):
    h = C.c_void_p()
    rc = hy.lib().hy_moe_create(C.byref(_cfg(hy, **kw)), C.byref(h))
    assert rc == code
    assert h.value is None
    assert hy.lib().hy_last_error().decode()


def test_config_struct_layouts_match_header(hy, tmp_path):
    """The ctypes mirrors of hy_moe_config, hy_attn_config and hy_model_config have the
    C header's field offsets and sizes (fields appended later keep the earlier ones)."""
    structs = {"hy_moe_config": hy.Config, "hy_attn_config": hy.AttnConfig, "hy_model_config": hy.ModelConfig}
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "hy_moe.h"', '#include "hy_attn.h"',
             'int main(void) {']
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", f"-I{os.path.join(ROOT, 'include')}", str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    for line in filter(None, got):
        cname, f, v = line.split()
        py = structs[cname]
        want = C.sizeof(py) if f == "size" else getattr(py, f).offset
        assert int(v) == want, (cname, f, int(v), want)


def test_integration_ctypes_stub_matches_headers(hy):
    """The ctypes stub the integration guide (section "FFI stubs") gives callers: its
    structs have the package's layouts (pinned to the C headers above) and every
    argtypes list has the header's parameter count."""
    import re
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    code = text.split("## 3. FFI stubs", 1)[1].split("```python", 1)[1].split("```", 1)[0]
    code = code.replace("/path/to/repo/hunyuan-image-3-80b.cpp_amd/libhy_moe.so", hy.LIB_PATH)
    ns = {}
    exec(code, ns)
    for stub, ours in ((ns["HyMoeConfig"], hy.Config), (ns["HyAttnConfig"], hy.AttnConfig)):
        assert C.sizeof(stub) == C.sizeof(ours)
        assert [f for f, _ in stub._fields_] == [f for f, _ in ours._fields_]
    headers = "".join(open(os.path.join(ROOT, "include", h)).read() for h in ("hy_moe.h", "hy_attn.h"))
    lib = ns["lib"]
    for name in re.findall(r"lib\.(hy_\w+)\.argtypes", code):
        decl = re.search(r"\bint\s+" + name + r"\s*\(([^)]*)\)", headers)
        assert decl, name
        n_params = len([p for p in decl.group(1).split(",") if p.strip() and p.strip() != "void"])
        assert len(getattr(lib, name).argtypes) == n_params, name
