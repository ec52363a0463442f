"""Module-level math names of the reference (src/macmetalpy/math_ops.py).

The elementwise functions live in ``ufunc_ops``; this module re-exports the
names the reference defines here (sqrt, exp, log, abs, power, sin, tanh,
square, negative, mod, isnan, ...) plus ``dot``, and defines ``where``,
``clip`` and ``count_nonzero`` (math_ops.py:106-200, 693).
"""
from __future__ import annotations

import numpy as np

from .linalg_top import dot  # noqa: F401
from .ufunc_ops import (  # noqa: F401
    abs, arccos, arcsin, arctan, ceil, cos, cosh, exp, floor, log, log2, log10, mod,
    negative, power, remainder, sign, sin, sinh, sqrt, square, tan, tanh, isnan, isinf,
    isfinite, maximum, minimum,
)
from . import _elementwise as _ew

__all__ = ["where", "clip", "count_nonzero"]


def where(condition, x=None, y=None):
    """Elements of ``x`` where ``condition`` is true, else of ``y``
    (reference math_ops.py:106-155; NumPy's result dtype and broadcasting).
    The one-argument form is ``nonzero(condition)``."""
    if x is None and y is None:
        from .indexing import nonzero
        return nonzero(condition)
    if x is None or y is None:
        raise ValueError("either both or neither of x and y should be given")
    return _ew.where(condition, x, y)


def clip(a, a_min=None, a_max=None, out=None, *, min=None, max=None):
    """Limit values to [a_min, a_max] (reference math_ops.py:167-200):
    minimum(maximum(a, a_min), a_max), NaN-propagating, as NumPy's clip loop.
    Either bound may be None."""
    if min is not None and a_min is None:
        a_min = min
    if max is not None and a_max is None:
        a_max = max
    from .creation import asarray
    r = asarray(a)
    if r.dtype.kind in "iu":
        # a Python int bound beyond the dtype on its own side clips nothing
        # (NumPy ignores it); beyond the other side it raises OverflowError
        info = np.iinfo(r.dtype)
        if type(a_min) is int and a_min < info.min:
            a_min = None
        if type(a_max) is int and a_max > info.max:
            a_max = None
    if a_min is None and a_max is None:
        r = r.copy()
    if a_min is not None:
        r = maximum(r, a_min)
    if a_max is not None:
        r = minimum(r, a_max)
    if out is not None:
        return out._inplace(r)
    return r


def count_nonzero(a, axis=None, keepdims=False):
    """Number of nonzero elements (reference math_ops.py:693): a Python
    int for axis=None, else an int64 array; one fused pass that counts
    ``a != 0`` (NaN counts)."""
    from . import reductions
    from .creation import asarray
    a = asarray(a)
    r = reductions.sum(a != 0, axis=axis, keepdims=keepdims)
    if axis is None and not keepdims:
        return int(r)
    return r
