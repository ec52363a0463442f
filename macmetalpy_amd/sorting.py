"""Sorting (reference: src/macmetalpy/sorting.py:21-263).

``sort`` / ``argsort`` run the device radix sort (``mmp_sort``) along one
axis for every dtype and shape; the reference sorts 1-D float32 / int32 /
uint32 / int16 / uint16 arrays of at least 256K elements with a bitonic
network and everything else with NumPy on the CPU.  ``searchsorted`` is a
device binary search per value (``mmp_searchsorted``).

Semantics are NumPy's: NaN sorts last; ``argsort`` returns int64 positions
and is stable (equal to ``kind='stable'``; NumPy's default introsort may
order equal keys differently, the sorted values are the same);
``sort(kind='stable')`` gathers the values by the stable order and so
matches NumPy bit for bit, while the default keeps every value's bits
except the sign of NaNs.
"""
from __future__ import annotations

import numpy as np

from ._backend import HipBackend
from ._dtypes import dtype_code, resolve_dtype
from .creation import asarray
from .ndarray import ndarray, _normalize_axis, _prod

__all__ = ["sort", "argsort", "searchsorted"]

_STABLE_KINDS = ("stable", "mergesort")


def _check_order(order):
    if order is not None:
        raise NotImplementedError("sort(order=...) needs structured dtypes, which are not "
                                  "supported on the device")


def _rows_last(a, axis):
    """(contiguous array with ``axis`` last, permutation used or None)."""
    if axis is None:
        return a.ravel()._ensure_contiguous(), None
    ax = _normalize_axis(axis, a.ndim)
    if ax == a.ndim - 1:
        return a._ensure_contiguous(), None
    perm = [i for i in range(a.ndim) if i != ax] + [ax]
    return a.transpose(perm)._contiguous_copy(), perm


def _restore(res, perm):
    if perm is None:
        return res
    inv = [0] * len(perm)
    for i, p in enumerate(perm):
        inv[p] = i
    return res.transpose(inv)._contiguous_copy()


def _run(a, axis, want_values, want_indices, stable):
    a = asarray(a)
    if a.ndim == 0:
        if axis is not None:
            raise np.exceptions.AxisError(f"axis {axis} is out of bounds for array of dimension 0")
        a = a.reshape((1,))
    x, perm = _rows_last(a, axis)
    shape = x._shape
    length = shape[-1] if shape else 1
    rows = _prod(shape[:-1]) if len(shape) > 1 else 1
    vals = ndarray._empty_device(shape, x._dtype) if want_values else None
    idx = ndarray._empty_device(shape, np.int64) if want_indices else None
    if x.size:
        HipBackend().sort(dtype_code(x._dtype), rows, length, x._ptr,
                          vals._ptr if vals is not None else None,
                          idx._ptr if idx is not None else None, stable)
    return (_restore(vals, perm) if vals is not None else None,
            _restore(idx, perm) if idx is not None else None)


def sort(a, axis=-1, kind=None, order=None, *, stable=None):
    """Sorted copy along ``axis`` (None: flattened), ascending, NaN last
    (reference sorting.py:21-37)."""
    _check_order(order)
    if stable is not None and kind is None:
        kind = "stable" if stable else "quicksort"
    vals, _ = _run(a, axis, True, False, kind in _STABLE_KINDS)
    return vals


def argsort(a, axis=-1, kind=None, order=None, *, stable=None):
    """Indices (int64) that sort ``a`` along ``axis``; always stable
    (reference sorting.py:40-56 returns int32 indices from an unstable
    bitonic network)."""
    _check_order(order)
    _, idx = _run(a, axis, False, True, True)
    return idx


def _take_1d(a, indices):
    """a[indices] for 1-D ``a`` and int64 device ``indices`` (range-checked)."""
    from . import reductions
    n = a.size
    if indices.size:
        lo, hi = int(reductions.min(indices)), int(reductions.max(indices))
        if lo < -n or hi >= n:
            raise IndexError(f"index {lo if lo < -n else hi} is out of bounds for axis 0 "
                             f"with size {n}")
        if lo < 0:
            indices = indices + (indices < 0) * n
            indices = indices.astype(np.int64)._ensure_contiguous()
    out = ndarray._empty_device(indices._shape, a._dtype)
    if indices.size:
        HipBackend().take(a._dtype.itemsize, n, a._ptr, indices.size, indices._ptr, out._ptr)
    return out


def searchsorted(a, v, side="left", sorter=None):
    """Insertion indices (int64) of ``v`` into the ascending 1-D ``a``
    (reference sorting.py:218-263); NaN is ordered last, and both are
    compared in their common dtype as NumPy does.  With ``sorter``, ``a`` is
    read through it (gathered on the device)."""
    if side not in ("left", "right"):
        raise ValueError(f"side must be 'left' or 'right' (got {side!r})")
    a = asarray(a)
    if a.ndim != 1:
        raise ValueError("object too deep for desired array" if a.ndim > 1 else
                         "object of too small depth for desired array")
    from ._elementwise import is_scalar
    kv = v if is_scalar(v) and not isinstance(v, ndarray) else None
    vv = asarray(v)
    common = resolve_dtype(np.result_type(a._dtype, kv if kv is not None else vv._dtype))
    if sorter is not None:
        s = asarray(sorter)
        if s.shape != a.shape:
            raise ValueError("sorter.size must equal a.size")
        a = _take_1d(a._ensure_contiguous(), s.astype(np.int64)._ensure_contiguous())
    ac = (a if a._dtype == common else a.astype(common))._ensure_contiguous()
    vc = (vv if vv._dtype == common else vv.astype(common))._ensure_contiguous()
    out = ndarray._empty_device(vv._shape, np.int64)
    if vc.size:
        HipBackend().searchsorted(dtype_code(common), ac.size, ac._ptr if ac.size else 0,
                                  vc.size, vc._ptr, side == "right", out._ptr)
    return out
