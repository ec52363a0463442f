"""NaN-aware reductions (reference: src/macmetalpy/nan_ops.py:112-612).

Floating inputs run single-pass device reductions that skip NaN
(``mmp_reduce`` with the MMP_R_NAN* ops, ``mmp_argreduce`` with
MMP_R_NANARG*); the reference replaces NaN in an extra pass
(``_nan_replace``, nan_ops.py:61-69) or reduces on the CPU below 4M
elements.  Integer and bool inputs cannot hold NaN and take the plain
reductions, as the reference does (nan_ops.py:128-130).

Semantics are NumPy's (the reference's CPU path): an all-NaN slice gives
0 for nansum, 1 for nanprod, NaN for nanmax / nanmin / nanmean / nanvar /
nanstd, and ``ValueError("All-NaN slice encountered")`` for nanargmax /
nanargmin.  NumPy's RuntimeWarnings for all-NaN slices are not raised
(that would need a device-to-host read on every call).  Float sums and
means accumulate in float64 and round once.
"""
from __future__ import annotations

import numpy as np

from . import _abi
from . import reductions as _r
from .creation import asarray
from ._elementwise import where as _where
from .ufunc_ops import fmax, fmin, isnan, sqrt, square

__all__ = ["nansum", "nanprod", "nanmax", "nanmin", "nanmean", "nanvar", "nanstd",
           "nanargmax", "nanargmin", "nancumsum", "nancumprod"]

_NoValue = np._NoValue


def _no_where(name, where):
    if where is not _NoValue:
        raise NotImplementedError(f"{name}(where=...) is not supported on the device")


def _is_float(a) -> bool:
    return a._dtype.kind == "f"


def _zeroed(a, fill):
    """``a`` with NaN replaced by ``fill`` (lazy; fuses into the consumer)."""
    return _where(isnan(a), fill, a)


def nansum(a, axis=None, dtype=None, out=None, keepdims=False, initial=_NoValue,
           where=_NoValue):
    """Sum treating NaN as zero (reference nan_ops.py:112-168)."""
    _no_where("nansum", where)
    a = asarray(a)
    if not _is_float(a):
        return _r.sum(a, axis=axis, dtype=dtype, out=out, keepdims=keepdims, initial=initial)
    if dtype is not None and np.dtype(dtype).kind != "f":
        r = _r.sum(_zeroed(a, 0), axis=axis, dtype=dtype, keepdims=keepdims)
    else:
        r = _r._reduce(a, "nansum", axis, dtype, None, keepdims)
    if initial is not _NoValue:
        r = r + initial
    return _r._finish(r, out)


def nanprod(a, axis=None, dtype=None, out=None, keepdims=False, initial=_NoValue,
            where=_NoValue):
    """Product treating NaN as one (reference nan_ops.py:171-212)."""
    _no_where("nanprod", where)
    a = asarray(a)
    if not _is_float(a):
        return _r.prod(a, axis=axis, dtype=dtype, out=out, keepdims=keepdims, initial=initial)
    if dtype is not None and np.dtype(dtype).kind != "f":
        r = _r.prod(_zeroed(a, 1), axis=axis, dtype=dtype, keepdims=keepdims)
    else:
        r = _r._reduce(a, "nanprod", axis, dtype, None, keepdims)
    if initial is not _NoValue:
        r = r * initial
    return _r._finish(r, out)


def nanmax(a, axis=None, out=None, keepdims=False, initial=_NoValue, where=_NoValue):
    """Maximum ignoring NaN (reference nan_ops.py:273-323); NaN for an
    all-NaN slice."""
    _no_where("nanmax", where)
    a = asarray(a)
    if not _is_float(a):
        return _r.max(a, axis=axis, out=out, keepdims=keepdims, initial=initial)
    r = _r._reduce(a, "nanmax", axis, None, None, keepdims)
    if initial is not _NoValue:
        r = fmax(r, initial)
    return _r._finish(r, out)


def nanmin(a, axis=None, out=None, keepdims=False, initial=_NoValue, where=_NoValue):
    """Minimum ignoring NaN (reference nan_ops.py:326-376)."""
    _no_where("nanmin", where)
    a = asarray(a)
    if not _is_float(a):
        return _r.min(a, axis=axis, out=out, keepdims=keepdims, initial=initial)
    r = _r._reduce(a, "nanmin", axis, None, None, keepdims)
    if initial is not _NoValue:
        r = fmin(r, initial)
    return _r._finish(r, out)


def nanmean(a, axis=None, dtype=None, out=None, keepdims=False, where=_NoValue):
    """Mean of the non-NaN elements (reference nan_ops.py:379-432): float64
    (sum, count) accumulated in one pass, divided once."""
    _no_where("nanmean", where)
    a = asarray(a)
    if not _is_float(a):
        return _r.mean(a, axis=axis, dtype=dtype, out=out, keepdims=keepdims)
    return _r._finish(_r._reduce(a, "nanmean", axis, dtype, None, keepdims), out)


def nanvar(a, axis=None, dtype=None, out=None, ddof=0, keepdims=False, where=_NoValue, *,
           correction=None, mean=None):
    """Variance of the non-NaN elements (reference nan_ops.py:484-559):
    sum of squared deviations from the NaN-skipping mean over
    (count - ddof); NaN where count - ddof <= 0.  Three passes: mean,
    squared deviations (fused with the NaN mask), count."""
    _no_where("nanvar", where)
    if correction is not None:
        ddof = correction
    if mean is not None:
        raise NotImplementedError("nanvar(mean=...) is not supported on the device")
    a = asarray(a)
    if not _is_float(a):
        return _r.var(a, axis=axis, dtype=dtype, out=out, ddof=ddof, keepdims=keepdims)
    if dtype is not None:
        a = a.astype(dtype)
    m = _r._reduce(a, "nanmean", axis, None, None, True)
    ssd = _r._reduce(_zeroed(square(a - m), 0), "sum", axis, None, None, keepdims)
    cnt = _r._reduce(~isnan(a), "sum", axis, None, None, keepdims)
    dof = (cnt - ddof).astype(a._dtype)
    v = _where(dof > 0, ssd / dof, np.nan)
    return _r._finish(v.astype(a._dtype), out)


def nanstd(a, axis=None, dtype=None, out=None, ddof=0, keepdims=False, where=_NoValue, *,
           correction=None, mean=None):
    """Standard deviation of the non-NaN elements (reference
    nan_ops.py:444-481): sqrt(nanvar)."""
    v = nanvar(a, axis=axis, dtype=dtype, ddof=ddof, keepdims=keepdims, where=where,
               correction=correction, mean=mean)
    return _r._finish(sqrt(v), out)


def nanargmax(a, axis=None, out=None, keepdims=False):
    """Index of the first maximum ignoring NaN (reference
    nan_ops.py:562-584); ValueError for an all-NaN slice."""
    a = asarray(a)
    if not _is_float(a):
        return _r.argmax(a, axis=axis, out=out, keepdims=keepdims)
    return _r._argreduce(a, _abi.REDUCE_NANARGMAX, axis, out, keepdims)


def nanargmin(a, axis=None, out=None, keepdims=False):
    """Index of the first minimum ignoring NaN (reference nan_ops.py:587-612)."""
    a = asarray(a)
    if not _is_float(a):
        return _r.argmin(a, axis=axis, out=out, keepdims=keepdims)
    return _r._argreduce(a, _abi.REDUCE_NANARGMIN, axis, out, keepdims)


def nancumsum(a, axis=None, dtype=None, out=None):
    """Cumulative sum treating NaN as zero (reference nan_ops.py:215-241)."""
    a = asarray(a)
    if _is_float(a):
        a = _zeroed(a, 0)
    return _r.cumsum(a, axis=axis, dtype=dtype, out=out)


def nancumprod(a, axis=None, dtype=None, out=None):
    """Cumulative product treating NaN as one (reference nan_ops.py:244-270)."""
    a = asarray(a)
    if _is_float(a):
        a = _zeroed(a, 1)
    return _r.cumprod(a, axis=axis, dtype=dtype, out=out)
