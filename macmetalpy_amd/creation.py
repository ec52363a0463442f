"""Array creation (reference: src/macmetalpy/creation.py:36-114).

As in the reference, creation routines return host-resident arrays backed
by NumPy; the data moves to HBM on the first device operation
(``ndarray._ensure_gpu``).  The exception is ``empty`` / ``zeros`` /
``ones`` / ``full`` of at least ``DEVICE_CREATE_MIN`` elements with a
scalar fill: those are allocated in HBM and filled there (the reference's
unified memory makes a host array free to hand to the GPU; over PCIe a
1 GiB upload costs ~28 ms, a device fill ~0.2 ms).  ``dtype=None`` means
the configured default float dtype (float32), as the reference's
``resolve_dtype(None)``.
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


DEVICE_CREATE_MIN = 1 << 16


def _device_const(shape, dtype, value):
    """HBM array of ``shape`` filled with ``value`` (None: uninitialised)."""
    from ._backend import HipBackend
    from ._dtypes import dtype_code
    arr = ndarray._empty_device(shape, dtype)
    if value is not None and arr.size:
        HipBackend().fill(dtype_code(dtype), arr.size, np.array(value).astype(dtype), arr._ptr)
    return arr


def _on_device(shape) -> bool:
    n = 1
    for s in shape:
        n *= s
    return n >= DEVICE_CREATE_MIN


def empty(shape, dtype=None, order="C", *, like=None, device=None) -> ndarray:
    _validate_device(device)
    shape, dtype = _shape(shape), resolve_dtype(dtype)
    if _on_device(shape):
        return _device_const(shape, dtype, None)
    return ndarray._from_np_direct(np.empty(shape, dtype=dtype))


def zeros(shape, dtype=None, order="C", *, like=None, device=None) -> ndarray:
    _validate_device(device)
    shape, dtype = _shape(shape), resolve_dtype(dtype)
    if _on_device(shape):
        return _device_const(shape, dtype, 0)
    return ndarray._from_np_direct(np.zeros(shape, dtype=dtype))


def ones(shape, dtype=None, order="C", *, like=None, device=None) -> ndarray:
    _validate_device(device)
    shape, dtype = _shape(shape), resolve_dtype(dtype)
    if _on_device(shape):
        return _device_const(shape, dtype, 1)
    return ndarray._from_np_direct(np.ones(shape, dtype=dtype))


def full(shape, fill_value, dtype=None, order="C", *, like=None, device=None) -> ndarray:
    _validate_device(device)
    if dtype is None:
        dtype = np.asarray(fill_value).dtype
    shape, dtype = _shape(shape), resolve_dtype(dtype)
    if _on_device(shape) and np.ndim(fill_value) == 0 and not isinstance(fill_value, ndarray):
        return _device_const(shape, dtype, fill_value)
    return ndarray._from_np_direct(np.full(shape, fill_value, dtype=dtype))


def arange(start, stop=None, step=1, dtype=None, *, like=None, device=None) -> ndarray:
    _validate_device(device)
    if stop is None:
        start, stop = 0, start
    if dtype is None:
        dtype = np.result_type(type(start), type(stop), type(step))
    return ndarray._from_np_direct(np.arange(start, stop, step, dtype=resolve_dtype(dtype)))


def linspace(start, stop, num=50, endpoint=True, retstep=False, dtype=None, axis=0):
    """NumPy's linspace; without ``dtype`` the result keeps NumPy's dtype
    (float64 for real bounds), as the reference's does (creation.py:159-173)."""
    r = np.linspace(start, stop, num, endpoint=endpoint, retstep=retstep, axis=axis)
    arr, step = r if retstep else (r, None)
    arr = arr.astype(resolve_dtype(arr.dtype if dtype is None else dtype), copy=False)
    if retstep:
        return ndarray._from_np_direct(arr), step
    return ndarray._from_np_direct(arr)


def eye(N, M=None, k=0, dtype=None) -> ndarray:
    """Ones on diagonal k; without ``dtype`` the library's default float, as
    the reference's eye (creation.py:176-181)."""
    return ndarray._from_np_direct(np.eye(N, M, k, dtype=resolve_dtype(dtype)))


def array(obj, dtype=None, copy=True) -> ndarray:
    """New array from a list / NumPy array / ndarray (reference :85-101)."""
    if isinstance(obj, ndarray):
        if obj._np_data is None:
            out = obj.copy() if dtype is None else obj.astype(dtype)
            return out
        data = obj._np_data
    elif dtype is not None:
        # NumPy's own conversion: Python ints outside the dtype raise
        data = np.asarray(obj, dtype=resolve_dtype(dtype))
        if copy and data is obj:
            data = data.copy()
        return ndarray._from_np_direct(data)
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
    data = np.asarray(obj) if dtype is None else np.asarray(obj, dtype=resolve_dtype(dtype))
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
