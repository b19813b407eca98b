"""MI355X-native HunyuanImage-3 MoE feed-forward block.

The product is libhy_moe.so (HIP kernels for gfx950 + a C ABI, include/hy_moe.h,
plus the C++ mirror of the reference API, include/hunyuan_moe_full.h).  This
package directory holds its sources (csrc/, host/), the build recipe (build.py)
and a ctypes binding (hy_moe.py) used by the tests and the benchmark.
"""
import importlib.util as _ilu
import os as _os

_here = _os.path.dirname(_os.path.abspath(__file__))


def _load(name):
    spec = _ilu.spec_from_file_location(f"hy3moe.{name}", _os.path.join(_here, f"{name}.py"))
    mod = _ilu.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


hy_moe = _load("hy_moe")
