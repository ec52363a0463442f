"""Global configuration (reference: src/macmetalpy/_config.py:11-64).

Same singleton and ``set_config`` keywords as the reference, plus the
switches this implementation adds:

* ``fusion`` -- build lazy expression DAGs and compile one kernel per DAG
  (default True).  False evaluates op by op with precompiled kernels, the
  "unfused" baseline of the fusion benchmark.
* ``native_dispatch`` -- route elementwise ops, their materialisation and
  fused row sums through the native gate (macmetalpy_amd._native; default
  True).  False runs the Python path for everything (same kernels, same
  results, more host time per op).  This is the counterpart of the
  reference's dispatch policy (its C gate plus the size thresholds of
  ndarray.py:41-44 that send small CPU-resident arrays to NumPy); there are
  no size thresholds here because nothing is computed on the host.
* ``float64_behavior`` keeps the reference's two values.  ``"cpu_fallback"``
  (the reference's default) keeps float64 precision; on MI355X float64 runs
  natively on the GPU, so nothing falls back to the CPU.  ``"downcast"``
  converts float64 inputs to float32 as the reference does.
"""
from __future__ import annotations

import threading
from typing import Literal

__all__ = ["MacMetalConfig", "get_config", "set_config"]


class MacMetalConfig:
    _instance: "MacMetalConfig | None" = None
    _lock = threading.Lock()

    def __new__(cls) -> "MacMetalConfig":
        with cls._lock:
            if cls._instance is None:
                inst = super().__new__(cls)
                inst.float64_behavior = "cpu_fallback"
                inst.warn_on_downcast = True
                inst.default_float_dtype = "float32"
                inst.fast_math = False
                inst.fusion = True
                inst.native_dispatch = True
                cls._instance = inst
            return cls._instance


def get_config() -> MacMetalConfig:
    inst = MacMetalConfig._instance
    return inst if inst is not None else MacMetalConfig()


def set_config(
    *,
    float64_behavior: Literal["downcast", "cpu_fallback"] | None = None,
    warn_on_downcast: bool | None = None,
    default_float_dtype: str | None = None,
    fast_math: bool | None = None,
    fusion: bool | None = None,
    native_dispatch: bool | None = None,
) -> None:
    """Update configuration values (reference: _config.py:43-64)."""
    cfg = get_config()
    policy = (cfg.float64_behavior, cfg.default_float_dtype)
    if float64_behavior is not None:
        if float64_behavior not in ("downcast", "cpu_fallback"):
            raise ValueError(
                f"float64_behavior must be 'downcast' or 'cpu_fallback', got {float64_behavior!r}")
        cfg.float64_behavior = float64_behavior
    if warn_on_downcast is not None:
        cfg.warn_on_downcast = bool(warn_on_downcast)
    if default_float_dtype is not None:
        cfg.default_float_dtype = default_float_dtype
    if (cfg.float64_behavior, cfg.default_float_dtype) != policy:
        _forget_result_dtypes()
    if fast_math is not None:
        cfg.fast_math = bool(fast_math)
    if fusion is not None:
        cfg.fusion = bool(fusion)
    if native_dispatch is not None and bool(native_dispatch) != cfg.native_dispatch:
        cfg.native_dispatch = bool(native_dispatch)
        from . import _gate
        _gate.apply(cfg.native_dispatch)


def _forget_result_dtypes() -> None:
    """Drop every cached result dtype: they follow float64_behavior and
    default_float_dtype (float64 results become float32 under "downcast"),
    so a policy change must resolve them again -- in the Python tables and
    in the native gate's C tables."""
    import sys
    pkg = __name__.rsplit(".", 1)[0]
    for mod, names in (("_dtypes", ("_UFUNC_CACHE",)),
                       ("_elementwise", ("_UNARY_DTYPES", "_BINARY_DTYPES")),
                       ("reductions", ("_OUT_DTYPE_CACHE",))):
        m = sys.modules.get(f"{pkg}.{mod}")
        for name in names if m is not None else ():
            getattr(m, name).clear()
    native = sys.modules.get(f"{pkg}._native")
    if native is not None:
        native.forget_dtypes()
