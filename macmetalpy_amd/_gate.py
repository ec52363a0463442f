"""Binding of the native dispatch gate (``macmetalpy_amd._native``).

``setup()`` hands the gate the Python classes it builds (ndarray, the
fusion nodes), the Python paths it falls back to, the dtype-resolution
functions that fill its result-dtype tables and the op tables; it then
takes over ``_elementwise.unary`` / ``binary`` and ``_fusion.materialize`` /
``run_sum``.
``bind_library(lib)`` gives it the entry-point addresses of the loaded
libmmp_hip.so (called when the device is initialised).  Reference: the
reference's C gate ``_accelerator.c`` is set up the same way, from Python,
with the ndarray class and dispatch tables (ndarray.py:2790-2882).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _abi
from . import _elementwise as ew
from . import _fusion
from ._config import get_config

try:
    from . import _native
except ImportError as exc:  # the product needs it: no silent Python-only mode
    raise ImportError(
        "macmetalpy_amd._native is not built; run `python -c 'import __graft_entry__ as g; "
        "g.build()'` or `python macmetalpy_amd/csrc/build.py`") from exc

__all__ = ["setup", "apply", "bind_library", "unbind_library", "stats"]

_LIB_FUNCS = ("mmp_alloc", "mmp_free", "mmp_unary", "mmp_binary", "mmp_binary_scalar",
              "mmp_rtc_launch", "mmp_reduce", "mmp_argreduce", "mmp_d2h", "mmp_h2d")


def _op_names():
    names = []
    for table in (_abi.UNARY_OPS, _abi.BINARY_OPS, _abi.EXPR_UNARY_OPS, _abi.EXPR_BINARY_OPS,
                  _abi.COMPARE_OPS):
        for k in table:
            if k not in names:
                names.append(k)
    return names


def _check(status: int, what: str) -> None:
    from ._backend import _check as check
    check(status, what)


def _reduce_dtype(code: int, dt):
    """Result dtype of the gate's reduction ``code`` on ``dt`` (the Python
    path's rule)."""
    from .reductions import _np_out_dtype
    if code in (_abi.REDUCE_ARGMAX, _abi.REDUCE_ARGMIN):
        return np.dtype(np.int64)
    if code in (_abi.REDUCE_MAX, _abi.REDUCE_MIN):
        return dt
    kind = {_abi.REDUCE_SUM: "sum", _abi.REDUCE_PROD: "prod", _abi.REDUCE_MEAN: "mean"}[code]
    return _np_out_dtype(kind, dt)


def _ensure_device() -> None:
    """Set up the device (binds the library to the gate), as the Python
    path's first upload would."""
    from ._backend import HipBackend
    HipBackend()


def setup() -> None:
    from .ndarray import ndarray
    dtypes = tuple(sorted(_abi.DTYPE_CODES, key=_abi.DTYPE_CODES.get))
    _native.init({
        "ndarray": ndarray,
        "InputNode": _fusion.InputNode, "CastNode": _fusion.CastNode,
        "UnaryOpNode": _fusion.UnaryOpNode, "BinaryOpNode": _fusion.BinaryOpNode,
        "ScalarNode": _fusion.ScalarNode, "WhereNode": _fusion.WhereNode,
        "unary_py": ew._unary_py, "binary_py": ew._binary_py,
        "materialize_py": _fusion._materialize_py,
        "run_sum_py": _fusion._run_sum_py,
        "compile_map": _fusion.compile_for_native,
        "check": _check,
        "unary_dtypes": ew._unary_dtypes, "binary_dtypes": ew._binary_dtypes,
        "prune": ew._prune_deps,
        "ensure_device": _ensure_device,
        "reduce_dtype": _reduce_dtype,
        "config": get_config(),
        "dtypes": dtypes,
        "max_depth": _fusion._MAX_DEPTH, "max_leaves": _fusion._MAX_LEAVES,
        "sum_blocks": _fusion._SUM_BLOCKS,
        "op_names": _op_names(),
        "unary_codes": {k: v[0] for k, v in _abi.UNARY_OPS.items()},
        "binary_codes": {k: v[0] for k, v in _abi.BINARY_OPS.items()},
        "fast_ops": set(_abi.FAST_MATH_OPS),
        "int_unary_ops": set(_abi.INT_UNARY_OPS),
    })
    apply(get_config().native_dispatch)


def apply(native: bool) -> None:
    """Route the hot path through the gate (True) or the Python path."""
    from . import reductions
    if native:
        ew.unary, ew.binary = _native.unary, _native.binary
        _fusion.materialize, _fusion.run_sum = _native.materialize, _native.run_sum
        reductions._native_reduce = _native.reduce
    else:
        ew.unary, ew.binary = ew._unary_py, ew._binary_py
        _fusion.materialize, _fusion.run_sum = _fusion._materialize_py, _fusion._run_sum_py
        reductions._native_reduce = None


def bind_library(lib) -> None:
    _native.set_library({name: ctypes.cast(getattr(lib, name), ctypes.c_void_p).value
                         for name in _LIB_FUNCS})


def unbind_library() -> None:
    """Detach the gate from the library and forget every compiled-kernel
    handle (used by tests that bind a host-only stand-in)."""
    _native.set_library(None)
    _fusion.clear_kernel_caches()


def stats() -> dict:
    """Counters: ops built natively, arrays materialised natively, calls
    handed to the Python path, host-resident operands uploaded by the gate,
    generated kernels known to the gate."""
    return _native.stats()
