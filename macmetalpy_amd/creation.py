"""Array creation (reference: src/macmetalpy/creation.py:36-114).

As in the reference, creation routines return host-resident arrays backed
by NumPy; the data moves to HBM on the first device operation
(``ndarray._ensure_gpu``).  ``dtype=None`` means the configured default
float dtype (float32), as the reference's ``resolve_dtype(None)``.
"""
from __future__ import annotations

import numpy as np

from ._dtypes import resolve_dtype
from .ndarray import ndarray

__all__ = ["empty", "zeros", "ones", "full", "arange", "array", "asarray",
           "zeros_like", "ones_like", "empty_like", "full_like", "linspace", "eye",
           "ascontiguousarray"]


def _shape(shape):
    return (int(shape),) if isinstance(shape, (int, np.integer)) else tuple(int(s) for s in shape)


def _validate_device(device):
    if device is not None and device not in ("cpu", "gpu"):
        raise ValueError(f"Unsupported device: {device!r}")


def empty(shape, dtype=None, order="C", *, like=None, device=None) -> ndarray:
    _validate_device(device)
    return ndarray._from_np_direct(np.empty(_shape(shape), dtype=resolve_dtype(dtype)))


def zeros(shape, dtype=None, order="C", *, like=None, device=None) -> ndarray:
    _validate_device(device)
    return ndarray._from_np_direct(np.zeros(_shape(shape), dtype=resolve_dtype(dtype)))


def ones(shape, dtype=None, order="C", *, like=None, device=None) -> ndarray:
    _validate_device(device)
    return ndarray._from_np_direct(np.ones(_shape(shape), dtype=resolve_dtype(dtype)))


def full(shape, fill_value, dtype=None, order="C", *, like=None, device=None) -> ndarray:
    _validate_device(device)
    if dtype is None:
        dtype = np.asarray(fill_value).dtype
    return ndarray._from_np_direct(np.full(_shape(shape), fill_value, dtype=resolve_dtype(dtype)))


def arange(start, stop=None, step=1, dtype=None, *, like=None, device=None) -> ndarray:
    _validate_device(device)
    if stop is None:
        start, stop = 0, start
    if dtype is None:
        dtype = np.result_type(type(start), type(stop), type(step))
    return ndarray._from_np_direct(np.arange(start, stop, step, dtype=resolve_dtype(dtype)))


def linspace(start, stop, num=50, endpoint=True, retstep=False, dtype=None, axis=0):
    r = np.linspace(start, stop, num, endpoint=endpoint, retstep=retstep, axis=axis)
    if retstep:
        arr, step = r
        return ndarray._from_np_direct(arr.astype(resolve_dtype(dtype))), step
    return ndarray._from_np_direct(r.astype(resolve_dtype(dtype)))


def eye(N, M=None, k=0, dtype=None) -> ndarray:
    return ndarray._from_np_direct(np.eye(N, M, k, dtype=resolve_dtype(dtype)))


def array(obj, dtype=None, copy=True) -> ndarray:
    """New array from a list / NumPy array / ndarray (reference :85-101)."""
    if isinstance(obj, ndarray):
        if obj._np_data is None:
            out = obj.copy() if dtype is None else obj.astype(dtype)
            return out
        data = obj._np_data
    else:
        data = np.asarray(obj)
    if dtype is not None:
        data = data.astype(resolve_dtype(dtype))
    elif copy and isinstance(obj, np.ndarray):
        data = data.copy()
    return ndarray._from_np_direct(data)


def asarray(obj, dtype=None) -> ndarray:
    if isinstance(obj, ndarray):
        if dtype is None or np.dtype(dtype) == obj._dtype:
            return obj
        return obj.astype(dtype)
    data = np.asarray(obj)
    if dtype is not None:
        data = data.astype(resolve_dtype(dtype))
    return ndarray._from_np_direct(data)


def ascontiguousarray(a, dtype=None) -> ndarray:
    a = asarray(a, dtype)
    if a._np_data is not None:
        return a
    return a._ensure_contiguous()


def _like_dtype(a, dtype):
    return a.dtype if dtype is None else dtype


def zeros_like(a, dtype=None, order="K", *, device=None) -> ndarray:
    return zeros(np.shape(a) if not isinstance(a, ndarray) else a.shape,
                 dtype=_like_dtype(asarray(a), dtype))


def ones_like(a, dtype=None, order="K", *, device=None) -> ndarray:
    return ones(np.shape(a) if not isinstance(a, ndarray) else a.shape,
                dtype=_like_dtype(asarray(a), dtype))


def empty_like(a, dtype=None, order="K", *, device=None) -> ndarray:
    return empty(np.shape(a) if not isinstance(a, ndarray) else a.shape,
                 dtype=_like_dtype(asarray(a), dtype))


def full_like(a, fill_value, dtype=None, order="K", *, device=None) -> ndarray:
    return full(np.shape(a) if not isinstance(a, ndarray) else a.shape, fill_value,
                dtype=_like_dtype(asarray(a), dtype))
