"""KernelCache (reference _kernel_cache.py:192-229) and the fast_math
switch on the CPU: every category's HIP source compiles for gfx950 (hiprtc,
no device), keys include fast_math, and unknown / library-served categories
raise as documented."""
import numpy as np
import pytest

from macmetalpy_amd import _abi
from macmetalpy_amd._backend import rtc_build
from macmetalpy_amd._config import set_config
from macmetalpy_amd._fusion import RTC_OPTIONS, _Program, generate_source, InputNode, UnaryOpNode
from macmetalpy_amd._kernel_cache import KernelCache


@pytest.mark.parametrize("category,dtype", [
    ("elementwise", np.float32), ("elementwise", np.float16), ("elementwise", np.float64),
    ("elementwise", np.int32), ("elementwise", np.uint16), ("comparison", np.float32),
    ("comparison_bool", np.int64), ("where", np.float32), ("clip", np.int16),
])
def test_sources_compile(category, dtype):
    src = KernelCache().get_shader(category, dtype)
    assert len(rtc_build(src, RTC_OPTIONS)) > 1000
    if category == "elementwise":
        for name in ("add_op", "mul_op", "neg_op", "fill_scalar"):
            assert f"void {name}(" in src
        if np.dtype(dtype).kind == "f":
            assert "void sin_op(" in src and "void pow_op(" in src


def test_cache_keys_and_fast_math():
    kc = KernelCache()
    a = kc.get_shader("elementwise", np.float32)
    assert kc.get_shader("elementwise", "float32") is a
    set_config(fast_math=True)
    f = kc.get_shader("elementwise", np.float32)
    assert f is not a and "op_exp_fast(" in f and "op_exp_fast(" not in a
    # fast forms only where float32 / float16 compute; float64 stays exact
    from macmetalpy_amd._fusion import _ops_header
    kernels64 = kc.get_shader("elementwise", np.float64)[len(_ops_header()):]
    assert "void exp_op(" in kernels64 and "_fast(" not in kernels64
    assert kc.get_shader("comparison", np.float32) is kc.get_shader("comparison", np.float32)
    set_config(fast_math=False)
    assert kc.get_shader("elementwise", np.float32) is a


def test_unknown_and_library_categories():
    with pytest.raises(ValueError, match="Unknown shader category"):
        KernelCache().get_shader("nonsense", np.float32)
    with pytest.raises(NotImplementedError, match="mmp_reduce"):
        KernelCache().get_shader("reduction", np.float32)


def test_fused_source_uses_fast_forms_only_when_asked():
    class _Buf:
        pass
    x = InputNode(_Buf(), (8,), np.float32, (1,))
    root = UnaryOpNode("tanh_op", UnaryOpNode("exp_op", x, (8,), np.float32), (8,), np.float32)
    prog = _Program(root)
    exact = generate_source(prog, ["c"], 0, np.dtype(np.float32), False, "map", fast=False)
    fast = generate_source(prog, ["c"], 0, np.dtype(np.float32), False, "map", fast=True)
    assert "op_tanh(" in exact and "op_exp(" in exact and "_fast(t" not in exact
    assert "op_tanh_fast(" in fast and "op_exp_fast(" in fast
    assert len(rtc_build(fast, RTC_OPTIONS)) > 1000
    x64 = InputNode(_Buf(), (8,), np.float64, (1,))
    prog64 = _Program(UnaryOpNode("exp_op", x64, (8,), np.float64))
    src64 = generate_source(prog64, ["c"], 0, np.dtype(np.float64), False, "map", fast=True)
    assert "op_exp(t" in src64 and "op_exp_fast(t" not in src64
    assert _abi.FAST_MATH_OPS <= set(_abi.UNARY_OPS) | set(_abi.BINARY_OPS)


def test_submodule_imports_alias_the_same_modules():
    import macmetalpy
    from macmetalpy._kernel_cache import KernelCache as K2
    import macmetalpy._backend as b1
    import macmetalpy_amd._backend as b2
    assert K2 is KernelCache and b1 is b2 and macmetalpy.MetalBackend is b2.HipBackend
