"""Reductions and scans (reference: src/macmetalpy/reductions.py:74-163,
314-418, 661-681 and ndarray._reduce / _reduce_axis / _prefix_scan,
ndarray.py:1895-2152).

Result dtypes and special cases follow NumPy (the reference's CPU path):
integer sums and cumulative sums widen to 64 bits, ``mean`` of integers is
float64 (resolved by the float64 policy), ``argmax`` returns int64 indices
with the first-NaN rule, empty ``max``/``argmax`` raise.  Accuracy: float
sums, means and scans accumulate in float64 on the device and round once.

When the input is a lazy expression and the reduction is ``sum``/``mean``
over the last axis or all axes, the reduction is fused into the expression
kernel (one pass over HBM); the reference materialises the expression and,
for axis reductions, loses it (ndarray.py:697-702).
"""
from __future__ import annotations

import builtins
import warnings

import numpy as np

from . import _abi
from ._backend import HipBackend
from ._config import get_config
from ._dtypes import dtype_code, resolve_dtype
from .ndarray import ndarray, _normalize_axis, _prod

__all__ = ["sum", "mean", "prod", "max", "min", "amax", "amin", "argmax", "argmin", "any", "all",
           "cumsum", "cumprod", "var", "std"]

_OUT_DTYPE_CACHE: dict = {}

# The native gate's reduction (macmetalpy_amd._native.reduce), bound by the
# package when native dispatch is on: reduce(code, x, axis) does a plain
# whole-array or last-axis reduction of a device-resident contiguous array
# in C and returns None for everything else.
_native_reduce = None


def _np_out_dtype(kind: str, dt: np.dtype) -> np.dtype:
    key = (kind, dt)
    r = _OUT_DTYPE_CACHE.get(key)
    if r is None:
        z = np.zeros(1, dtype=dt)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            r = {"sum": np.sum, "prod": np.prod, "mean": np.mean, "cumsum": np.cumsum,
                 "cumprod": np.cumprod, "var": np.var}[kind](z).dtype
        r = resolve_dtype(r)
        _OUT_DTYPE_CACHE[key] = r
    return r


def _asarray(a):
    from . import creation
    return creation.asarray(a)


def _axes(axis, ndim):
    if axis is None:
        return None
    if isinstance(axis, (tuple, list)):
        ax = tuple(sorted({_normalize_axis(a, ndim) for a in axis}))
    else:
        ax = (_normalize_axis(axis, ndim),)
    return ax


def _out_shape(shape, axes, keepdims):
    if axes is None:
        return tuple(1 for _ in shape) if keepdims else ()
    if keepdims:
        return tuple(1 if i in axes else s for i, s in enumerate(shape))
    return tuple(s for i, s in enumerate(shape) if i not in axes)


def _finish(res, out):
    if out is None:
        return res
    return out._inplace(res)


def _fused_ok(a, axes, kind, dtype):
    if a._fusion_node is None or dtype is not None or not get_config().fusion:
        return False
    if kind not in ("sum", "mean"):
        return False
    if a._dtype.kind not in "fiub":
        return False
    return axes is None or axes == (a.ndim - 1,)


def _layout(shape, axes):
    """(outer, len, inner) of a contiguous array for reducing ``axes``,
    or None when the reduced axes are not one contiguous run."""
    if axes is None:
        return 1, _prod(shape), 1
    if list(axes) != list(range(axes[0], axes[-1] + 1)):
        return None
    return _prod(shape[:axes[0]]), _prod(shape[axes[0]:axes[-1] + 1]), _prod(shape[axes[-1] + 1:])


_CODES = {"sum": _abi.REDUCE_SUM, "prod": _abi.REDUCE_PROD, "max": _abi.REDUCE_MAX,
          "min": _abi.REDUCE_MIN, "mean": _abi.REDUCE_MEAN,
          "nansum": _abi.REDUCE_NANSUM, "nanprod": _abi.REDUCE_NANPROD,
          "nanmax": _abi.REDUCE_NANMAX, "nanmin": _abi.REDUCE_NANMIN,
          "nanmean": _abi.REDUCE_NANMEAN}
# NaN-ignoring kinds share the result dtype and empty-slice rules of these
_BASE_KIND = {"nansum": "sum", "nanprod": "prod", "nanmax": "max", "nanmin": "min",
              "nanmean": "mean"}


def _reduce(a, kind, axis=None, dtype=None, out=None, keepdims=False):
    a = _asarray(a)
    axes = _axes(axis, a.ndim)
    if dtype is not None:
        a = a.astype(dtype)
    if kind in ("max", "min", "nanmax", "nanmin"):
        odt = a._dtype
    elif dtype is not None:
        odt = a._dtype          # NumPy accumulates in, and returns, the requested dtype
        if kind in ("mean", "nanmean") and odt.kind in "iu":
            # NumPy's mean with an integer dtype (numpy/_core/_methods.py
            # _mean; nanmean of integers is mean): the sum accumulates in
            # that dtype and wraps, then true_divide by the element count
            # (float64) is cast back, truncating.  The 64-bit sum cast to
            # the dtype has the wrapped sum's bits.
            n_red = _prod(a._shape) if axes is None else _prod(a._shape[i] for i in axes)
            if n_red and a.size:
                wide = np.uint64 if odt.kind == "u" else np.int64
                s = _reduce(a, "sum", axis, wide, None, keepdims).astype(odt)
                q = (s.astype(np.float64) / float(n_red)).astype(odt)
                return _finish(q, out)
        if odt.kind in "biu" and (odt.itemsize < 8 or kind in ("mean", "nanmean")):
            # 64-bit accumulation, then the cast: the low bits of an integer
            # sum / product are NumPy's wrapping accumulation in the narrow
            # type; a bool mean is nonzero exactly when some element is
            wide = (np.float64 if kind in ("mean", "nanmean")
                    else np.uint64 if odt.kind in "bu" else np.int64)
            r = _reduce(a, kind, axis, wide, None, keepdims)
            return _finish(r.astype(odt), out)
    else:
        odt = _np_out_dtype(_BASE_KIND.get(kind, kind), a._dtype)
    oshape = _out_shape(a._shape, axes, keepdims)
    red_len = _prod(a._shape) if axes is None else _prod(a._shape[i] for i in axes)

    if red_len == 0 or a.size == 0:
        return _finish(_empty_reduction(kind, oshape, odt, red_len), out)

    if _fused_ok(a, axes, kind, dtype):
        from ._fusion import CastNode, run_sum
        node = a._fusion_node
        if kind == "mean" and node._dtype.kind != "f":
            node = CastNode(node, np.dtype(np.float64))
        res = ndarray._empty_device(oshape, odt)
        run_sum(node, axes is not None, odt, res._ptr, kind == "mean")
        return _finish(res, out)

    x = a._ensure_contiguous()
    lay = _layout(x._shape, axes)
    if lay is None:
        # bring the reduced axes to the end (one strided copy), then reduce
        keep = [i for i in range(x.ndim) if i not in axes]
        xt = x.transpose(keep + list(axes))._contiguous_copy()
        lay = (_prod(xt._shape[:len(keep)]), _prod(xt._shape[len(keep):]), 1)
        x = xt
    outer, length, inner = lay
    res = ndarray._empty_device(oshape, odt)
    HipBackend().reduce(_CODES[kind], dtype_code(x._dtype), dtype_code(odt), outer, length,
                        inner, x._ptr, res._ptr)
    return _finish(res, out)


def _empty_reduction(kind, oshape, odt, red_len):
    from . import creation
    if kind in ("nanmax", "nanmin") and red_len == 0:
        raise ValueError(f"zero-size array to reduction operation f{kind[3:]} which has no "
                         "identity")
    kind = _BASE_KIND.get(kind, kind)
    if red_len == 0:
        if kind == "sum":
            return creation.zeros(oshape, dtype=odt)
        if kind == "prod":
            return creation.ones(oshape, dtype=odt)
        if kind == "mean":
            warnings.warn("Mean of empty slice.", RuntimeWarning, stacklevel=3)
            return creation.full(oshape, np.nan, dtype=odt)
        raise ValueError(f"zero-size array to reduction operation {kind}imum which has no identity"
                         if kind in ("max", "min") else
                         f"zero-size array to reduction operation {kind}")
    return creation.empty(oshape, dtype=odt)


def _masked(a, where, fill):
    """``a`` with the elements outside the ``where`` mask replaced by
    ``fill`` (lazy: fuses into the reduction that consumes it).  NumPy's
    reductions with ``where=`` skip those elements; for sum / prod / max /
    min that equals reducing the masked array (the reference's CPU branches
    hand ``where`` to NumPy, e.g. reductions.py:89-103)."""
    from ._broadcasting import broadcast_shapes
    from ._elementwise import where as _where
    a = _asarray(a)
    m = where if isinstance(where, ndarray) else _asarray(np.asarray(where, dtype=bool))
    if broadcast_shapes(m._shape, a._shape) != a._shape:
        raise ValueError(f"where mask of shape {m._shape} does not broadcast to {a._shape}")
    return _where(m, a, fill)


def sum(a, axis=None, dtype=None, out=None, keepdims=False, initial=np._NoValue,
        where=np._NoValue):
    """Sum of elements (reference reductions.py:74-113); ``where`` masks
    elements out (they count as 0)."""
    if (_native_reduce is not None and dtype is None and out is None and not keepdims
            and initial is np._NoValue and where is np._NoValue):
        r = _native_reduce(_abi.REDUCE_SUM, a, axis)
        if r is not None:
            return r
    if where is not np._NoValue:
        a = _masked(a, where, 0)
    r = _reduce(a, "sum", axis, dtype, None, keepdims)
    if initial is not np._NoValue:
        r = r + initial
    return _finish(r, out)


def mean(a, axis=None, dtype=None, out=None, keepdims=False, where=np._NoValue):
    """Arithmetic mean (reference reductions.py:116-163): the float64 sum
    divided by the count in float64, rounded once to the result dtype.  With
    ``where``: the masked sum over the number of selected elements (NaN
    where none is selected, as NumPy)."""
    if where is None or where is np._NoValue:
        if _native_reduce is not None and dtype is None and out is None and not keepdims:
            r = _native_reduce(_abi.REDUCE_MEAN, a, axis)
            if r is not None:
                return r
        return _reduce(a, "mean", axis, dtype, out, keepdims)
    a = _asarray(a)
    if dtype is not None:
        a = a.astype(dtype)                   # NumPy converts the elements first
    odt = _np_out_dtype("mean", a._dtype) if dtype is None else resolve_dtype(dtype)
    tot = _reduce(_masked(a, where, 0).astype(np.float64), "sum", axis, None, None, keepdims)
    everywhere = (a == a) | (a != a)          # True with a's shape (NaN included)
    cnt = _reduce(_masked(everywhere, where, False), "sum", axis, None, None, keepdims)
    return _finish((tot / cnt).astype(odt), out)


def prod(a, axis=None, dtype=None, out=None, keepdims=False, initial=np._NoValue,
         where=np._NoValue):
    if (_native_reduce is not None and dtype is None and out is None and not keepdims
            and initial is np._NoValue and where is np._NoValue):
        r = _native_reduce(_abi.REDUCE_PROD, a, axis)
        if r is not None:
            return r
    if where is not np._NoValue:
        a = _masked(a, where, 1)
    r = _reduce(a, "prod", axis, dtype, None, keepdims)
    if initial is not np._NoValue:
        r = r * initial
    return _finish(r, out)


def _extreme(a, kind, axis, out, keepdims, initial, where):
    if (_native_reduce is not None and out is None and not keepdims
            and initial is np._NoValue and where is np._NoValue):
        r = _native_reduce(_abi.REDUCE_MAX if kind == "max" else _abi.REDUCE_MIN, a, axis)
        if r is not None:
            return r
    from .ufunc_ops import maximum, minimum
    if where is not np._NoValue:
        if initial is np._NoValue:
            raise ValueError(f"reduction operation '{'maximum' if kind == 'max' else 'minimum'}'"
                             " does not have an identity, so to use a where mask one has to "
                             "specify 'initial'")
        a = _masked(a, where, initial)
    r = _reduce(a, kind, axis, None, None, keepdims)
    if initial is not np._NoValue:
        r = (maximum if kind == "max" else minimum)(r, initial)
    return _finish(r, out)


def max(a, axis=None, out=None, keepdims=False, initial=np._NoValue, where=np._NoValue):
    """Maximum; NaN propagates (NumPy).  ``where`` needs ``initial``."""
    return _extreme(a, "max", axis, out, keepdims, initial, where)


def min(a, axis=None, out=None, keepdims=False, initial=np._NoValue, where=np._NoValue):
    """Minimum; NaN propagates (NumPy).  ``where`` needs ``initial``."""
    return _extreme(a, "min", axis, out, keepdims, initial, where)


amax = max
amin = min


def any(a, axis=None, out=None, keepdims=False, where=np._NoValue):
    """True where any element along ``axis`` is nonzero (reference
    reductions.py:248-278).  One fused pass counts ``a != 0`` (NaN counts as
    true; masked-out elements count as false); an empty reduction is False.
    Returns a bool ndarray (0-d for axis=None), as the reference does."""
    a = _asarray(a)
    t = a != 0
    if where is not np._NoValue:
        t = _masked(t, where, False)
    r = _reduce(t, "sum", axis, None, None, keepdims) > 0
    return _finish(r, out)


def all(a, axis=None, out=None, keepdims=False, where=np._NoValue):
    """True where every element along ``axis`` is nonzero (reference
    reductions.py:281-311); counts ``a == 0`` (masked-out elements do not
    count) in one fused pass; an empty reduction is True."""
    a = _asarray(a)
    t = a == 0
    if where is not np._NoValue:
        t = _masked(t, where, False)
    r = _reduce(t, "sum", axis, None, None, keepdims) == 0
    return _finish(r, out)


def _argreduce(a, op, axis, out, keepdims):
    if (_native_reduce is not None and out is None and not keepdims
            and op in (_abi.REDUCE_ARGMAX, _abi.REDUCE_ARGMIN)):
        r = _native_reduce(op, a, axis)
        if r is not None:
            return r
    a = _asarray(a)
    name = {_abi.REDUCE_ARGMAX: "argmax", _abi.REDUCE_ARGMIN: "argmin",
            _abi.REDUCE_NANARGMAX: "nanargmax", _abi.REDUCE_NANARGMIN: "nanargmin"}[op]
    if a.size == 0:
        raise ValueError(f"attempt to get {name} of an empty sequence")
    x = a._ensure_contiguous()
    be = HipBackend()
    skip_nan = op in (_abi.REDUCE_NANARGMAX, _abi.REDUCE_NANARGMIN)
    if axis is None:
        res = ndarray._empty_device((), np.int64)
        be.argreduce(op, dtype_code(x._dtype), 1, x.size, 1, x._ptr, res._ptr)
        if skip_nan or not (keepdims or out is not None):
            idx = int(res.get())  # reference returns a Python int (reductions.py:407)
            if skip_nan and idx == _abi.ARG_NONE:
                raise ValueError("All-NaN slice encountered")
        if keepdims:
            return _finish(res.reshape((1,) * a.ndim), out)
        if out is not None:
            return _finish(res, out)
        return idx
    ax = _normalize_axis(axis, a.ndim)
    outer, length, inner = _prod(x._shape[:ax]), x._shape[ax], _prod(x._shape[ax + 1:])
    if length == 0:
        raise ValueError(f"attempt to get {name} of an empty sequence")
    oshape = _out_shape(x._shape, (ax,), keepdims)
    res = ndarray._empty_device(oshape, np.int64)
    be.argreduce(op, dtype_code(x._dtype), outer, length, inner, x._ptr, res._ptr)
    if skip_nan and res.size and int(max(res)) == _abi.ARG_NONE:
        raise ValueError("All-NaN slice encountered")
    return _finish(res, out)


def argmax(a, axis=None, out=None, keepdims=False):
    """Index of the first maximum (first NaN if any), int64 (reference
    reductions.py:381-418 returns int32 and ignores NaN)."""
    return _argreduce(a, _abi.REDUCE_ARGMAX, axis, out, keepdims)


def argmin(a, axis=None, out=None, keepdims=False):
    return _argreduce(a, _abi.REDUCE_ARGMIN, axis, out, keepdims)


def _scan(a, op, kind, axis, dtype, out):
    a = _asarray(a)
    if dtype is not None:
        a = a.astype(dtype)
        want = a._dtype
        if want.kind in "biu" and want.itemsize < 8:
            # accumulate in 64 bits: the low bits are NumPy's wrapping
            # accumulation in the requested integer type
            wide = np.dtype(np.uint64 if want.kind in "bu" else np.int64)
            r = _scan(a, op, kind, axis, wide, None)
            return _finish(r.astype(want), out)
        odt = want
    else:
        odt = _np_out_dtype(kind, a._dtype)
    x = a._ensure_contiguous()
    if axis is None:
        x = x.reshape(-1)
        outer, length, inner = 1, x.size, 1
        oshape = (x.size,)
    else:
        ax = _normalize_axis(axis, x.ndim)
        outer, length, inner = _prod(x._shape[:ax]), x._shape[ax], _prod(x._shape[ax + 1:])
        oshape = x._shape
    res = ndarray._empty_device(oshape, odt)
    if res.size:
        HipBackend().scan(op, dtype_code(x._dtype), dtype_code(odt), outer, length, inner,
                          x._ptr, res._ptr)
    return _finish(res, out)


def cumsum(a, axis=None, dtype=None, out=None):
    """Inclusive prefix sum (reference reductions.py:661-681); int32 input
    gives int64 output as in NumPy (the reference's GPU path keeps int32)."""
    return _scan(a, _abi.SCAN_CUMSUM, "cumsum", axis, dtype, out)


def cumprod(a, axis=None, dtype=None, out=None):
    return _scan(a, _abi.SCAN_CUMPROD, "cumprod", axis, dtype, out)


def var(a, axis=None, dtype=None, out=None, ddof=0, keepdims=False):
    """Variance as mean(|x - mean(x)|**2) * n / (n - ddof); with fusion on,
    the deviation, square and mean run as one kernel per pass."""
    from .ufunc_ops import square
    a = _asarray(a)
    if dtype is not None:
        a = a.astype(dtype)
    elif a._dtype.kind in "iub":
        a = a.astype(resolve_dtype(np.float64))
    axes = _axes(axis, a.ndim)
    n = a.size if axes is None else _prod(a._shape[i] for i in axes)
    m = mean(a, axis=axis, keepdims=True)
    if axes is None:
        m = m.reshape(())
    v = mean(square(a - m), axis=axis, keepdims=keepdims)
    if ddof:
        v = v * (n / builtins.max(n - ddof, 0)) if n - ddof > 0 else v * np.inf
    return _finish(v, out)


def std(a, axis=None, dtype=None, out=None, ddof=0, keepdims=False):
    from .ufunc_ops import sqrt
    return _finish(sqrt(var(a, axis=axis, dtype=dtype, ddof=ddof, keepdims=keepdims)), out)
