"""dtype policy (reference: src/macmetalpy/_dtypes.py:77-146).

``resolve_dtype`` keeps the reference's mapping (int8/uint8 -> int16/uint16,
complex128 -> complex64, float64 per ``float64_behavior``).  Result dtypes of
ufuncs follow NumPy's own type resolution, obtained by calling the NumPy
ufunc on empty operands (cached), then resolved by the same policy.
"""
from __future__ import annotations

import warnings

import numpy as np

from ._abi import CTYPE_NAMES, DTYPE_CODES
from ._config import get_config

__all__ = ["resolve_dtype", "result_dtype", "ufunc_result_dtype", "is_float_dtype",
           "SUPPORTED_DTYPES", "dtype_code"]

SUPPORTED_DTYPES = frozenset(DTYPE_CODES)
_PASSTHROUGH = frozenset(SUPPORTED_DTYPES - {np.dtype(np.float64)})
_F64 = np.dtype(np.float64)


def is_float_dtype(dtype) -> bool:
    return np.issubdtype(np.dtype(dtype), np.floating)


def dtype_code(dtype) -> int:
    try:
        return DTYPE_CODES[np.dtype(dtype)]
    except KeyError:
        raise TypeError(f"Unsupported dtype for the MI355X device: {np.dtype(dtype)}") from None


def ctype_name(dtype) -> str:
    return CTYPE_NAMES[np.dtype(dtype)]


def resolve_dtype(dtype) -> np.dtype:
    """Map a requested dtype to a device dtype (None -> default float)."""
    if dtype is None:
        return np.dtype(get_config().default_float_dtype)
    dtype = np.dtype(dtype)
    if dtype in _PASSTHROUGH:
        return dtype
    cfg = get_config()
    if dtype == _F64:
        if cfg.float64_behavior == "downcast":
            if cfg.warn_on_downcast:
                warnings.warn("float64 is downcast to float32 (float64_behavior='downcast').",
                              UserWarning, stacklevel=3)
            return np.dtype(cfg.default_float_dtype)
        return dtype
    if dtype == np.int8:
        return np.dtype(np.int16)
    if dtype == np.uint8:
        return np.dtype(np.uint16)
    if dtype.kind == "c":
        raise TypeError(f"complex dtypes are not supported on the MI355X device: {dtype}")
    raise TypeError(f"Unsupported dtype for the MI355X device: {dtype}")


def result_dtype(dt1, dt2) -> np.dtype:
    """Binary promotion (reference: _dtypes.py:139-146)."""
    return resolve_dtype(np.result_type(dt1, dt2))


_UFUNC_CACHE: dict = {}


def ufunc_result_dtype(ufunc: np.ufunc, *operands) -> np.dtype:
    """Result dtype NumPy's ufunc would produce for these operand dtypes /
    Python scalars (NEP 50 weak scalars), resolved by the device policy.

    Raises NumPy's own TypeError / OverflowError for invalid combinations
    (e.g. ``negative`` of bool, an int scalar out of the array's range)."""
    key = None
    if all(isinstance(o, np.dtype) for o in operands):
        key = (ufunc, operands)
    elif all(isinstance(o, np.dtype) and o.kind == "f" or type(o) in (int, float, bool)
             for o in operands) and any(isinstance(o, np.dtype) for o in operands):
        # Python scalars are weak (NEP 50): with a floating array operand the
        # result depends on the scalars' types only, never on their values
        key = (ufunc, tuple(o if isinstance(o, np.dtype) else type(o) for o in operands))
    if key is not None:
        hit = _UFUNC_CACHE.get(key)
        if hit is not None:
            return hit
    args = [np.empty(0, dtype=o) if isinstance(o, np.dtype) else o for o in operands]
    with np.errstate(all="ignore"):
        res = ufunc(*args)
    dt = resolve_dtype(res.dtype)
    if key is not None:
        _UFUNC_CACHE[key] = dt
    return dt
