"""ctypes loader for oracle/liboracle.so (test oracle only)."""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None


def lib():
    global _lib
    if _lib is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            from .build import build
            build(verbose=False)
        L = ctypes.CDLL(path)
        vp, i64 = ctypes.c_void_p, ctypes.c_int64
        L.oracle_floor_divide_i32.argtypes = [vp, vp, vp, i64]
        L.oracle_mod_i32.argtypes = [vp, vp, vp, i64]
        L.oracle_cumsum_i32.argtypes = [vp, vp, i64]
        L.oracle_sum_f32.argtypes = [vp, i64]
        L.oracle_sum_f32.restype = ctypes.c_double
        L.oracle_argmax_f32.argtypes = [vp, i64]
        L.oracle_argmax_f32.restype = ctypes.c_int64
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def floor_divide_i32(a, b):
    a, b = _c(a, np.int32), _c(b, np.int32)
    out = np.empty_like(a)
    lib().oracle_floor_divide_i32(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
    return out


def mod_i32(a, b):
    a, b = _c(a, np.int32), _c(b, np.int32)
    out = np.empty_like(a)
    lib().oracle_mod_i32(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
    return out


def cumsum_i32(x):
    x = _c(x, np.int32).ravel()
    out = np.empty(x.size, np.int64)
    lib().oracle_cumsum_i32(x.ctypes.data, out.ctypes.data, x.size)
    return out


def sum_f32(x):
    x = _c(x, np.float32).ravel()
    return lib().oracle_sum_f32(x.ctypes.data, x.size)


def argmax_f32(x):
    x = _c(x, np.float32).ravel()
    return int(lib().oracle_argmax_f32(x.ctypes.data, x.size))
