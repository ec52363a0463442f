"""Order statistics on the device: median, quantile, percentile and their
NaN-aware forms.

The reference computes these with NumPy on the host.  Here the data is
sorted along the axis by the device radix sort (NaN last) and the
statistic is read from the sorted rows: for the plain forms the positions
are the same for every row (basic slices), for the NaN-aware forms they
depend on each row's count of non-NaN values (one gather per position).

The arithmetic is NumPy's (numpy/lib/_function_base_impl.py _quantile,
_get_indexes, _get_gamma, _lerp; _nanfunctions_impl.py; ma median) step
for step, so results match NumPy bit for bit, dtypes included:

* q is taken in the data's float dtype when it is a Python scalar and the
  data is floating (percentile divides by 100 in that dtype), else as
  given (float64 for lists and arrays); the virtual index ``(n - 1) * q``
  is computed in q's dtype;
* linear / midpoint interpolate with gamma = virtual - previous (rounded
  to q's dtype; the previous index is -1 at and beyond the last value) by
  ``a + (b - a) * t`` below t = 0.5 and ``b - (b - a) * (1 - t)`` from 0.5,
  in the promotion of the data and q dtypes; lower / higher / nearest
  (and integer q with linear) take an element and keep the data dtype;
* a slice holding NaN gives NaN;
* median is the mean of the middle one or two values (float16 summed in
  float32, integers in float64); nanmedian follows NumPy's masked-array
  path for an axis of fewer than 600 values of an N-D array ((a + b) / 2
  in the data dtype) and otherwise the median of the non-NaN values.
"""
from __future__ import annotations

import numpy as np

from . import _elementwise as ew
from .ndarray import ndarray, _normalize_axis, _prod

__all__ = ["median", "quantile", "percentile", "nanmedian", "nanquantile", "nanpercentile"]

_METHODS = ("linear", "lower", "higher", "nearest", "midpoint")


def _asarray(a):
    from .creation import asarray
    return asarray(a)


def _prepare(a, axis):
    """(array with the reduced axes merged last, kept shape, keepdims shape)."""
    x = _asarray(a)
    if axis is None:
        return x.ravel(), (), (1,) * x.ndim
    axes = (axis,) if isinstance(axis, (int, np.integer)) else tuple(axis)
    axes = sorted({_normalize_axis(ax, x.ndim) for ax in axes})
    keep = [d for d in range(x.ndim) if d not in axes]
    kept = tuple(x.shape[d] for d in keep)
    kd = tuple(1 if d in axes else x.shape[d] for d in range(x.ndim))
    x = x.transpose(keep + axes).reshape(kept + (_prod([x.shape[d] for d in axes]),))
    return x, kept, kd


def _qarray(dt, q, percent):
    """q as NumPy's quantile / percentile convert it for data of dtype dt."""
    if isinstance(q, ndarray):
        q = q.get()
    if percent:
        qa = np.asanyarray(np.true_divide(q, dt.type(100) if dt.kind == "f" else 100))
    elif isinstance(q, (int, float)) and dt.kind == "f":
        qa = np.asanyarray(q, dtype=dt)
    else:
        qa = np.asanyarray(q)
    ok = qa.size == 0 or (bool(np.all(qa >= 0)) and bool(np.all(qa <= 1)))
    if not ok:
        raise ValueError("Percentiles must be in the range [0, 100]" if percent else
                         "Quantiles must be in the range [0, 1]")
    return qa


def _copy(v):
    return ew.unary("positive_op", v)


def _plain_one(s, n, qv, method):
    """Statistic of the sorted rows s (..., n) for one q (0-d array)."""
    int_q = qv.dtype.kind in "iub"
    last = s[..., n - 1]
    if method == "linear" and int_q or method in ("lower", "higher", "nearest"):
        if method in ("linear", "lower"):
            idx = np.floor((n - 1) * qv)
        elif method == "higher":
            idx = np.ceil((n - 1) * qv)
        else:
            idx = np.around((n - 1) * qv)
        r = _copy(s[..., int(np.clip(int(idx), 0, n - 1))])
    else:
        if method == "linear":
            v = (n - 1) * qv
        else:  # midpoint
            v = 0.5 * (np.floor((n - 1) * qv) + np.ceil((n - 1) * qv))
        if v >= n - 1:
            pi = ni = n - 1
            pf = -1
        elif v < 0:
            pi = ni = pf = 0
        else:
            pi = pf = int(np.floor(v))
            ni = pi + 1
        g = np.asanyarray(v) - np.asarray(pf, np.intp)
        if method == "midpoint":
            g = np.full(np.shape(g), 0.5)
            if v % 1 == 0:
                g[...] = 0.0
        t = np.asanyarray(g, dtype=np.asanyarray(v).dtype)[()]
        lo, hi = s[..., pi], s[..., ni]
        d = hi - lo
        r = hi - d * (1 - t) if t >= 0.5 else lo + d * t
    if s.dtype.kind == "f":
        r = ew.where(ew.unary("isnan_op", last), last, r)
    return r


def _nan_one(s, k, kept, qv, method):
    """NaN-aware statistic: k (kept + (1,)) non-NaN counts per row."""
    from .indexing import take_along_axis
    qdt = qv.dtype if qv.dtype.kind == "f" else np.dtype(np.float64)
    int_q = qv.dtype.kind in "iub"
    km1 = (k - 1).astype(qdt) if not int_q else (k - 1)
    q = qv[()]
    discrete = method in ("lower", "higher", "nearest") or (method == "linear" and int_q)

    def gather(idx):
        idx = ew.where(idx < 0, 0, ew.where(idx > k - 1, k - 1, idx))
        idx = ew.where(k > 0, idx, 0).astype(np.int64)
        return take_along_axis(s, idx, axis=-1).reshape(kept)

    if discrete:
        base = km1 * q
        if method in ("linear", "lower"):
            idx = ew.unary("floor_op", base)
        elif method == "higher":
            idx = ew.unary("ceil_op", base)
        else:
            idx = ew.unary("rint_op", base)
        r = gather(idx.astype(np.int64))
        nan_dt = s.dtype
    else:
        if method == "linear":
            v = km1 * q
        else:
            v = (ew.unary("floor_op", km1 * q) + ew.unary("ceil_op", km1 * q)) * qdt.type(0.5)
        prev = ew.unary("floor_op", v)
        above = v >= km1
        below = v < 0
        pf = ew.where(above, -1, ew.where(below, 0, prev)).astype(np.int64)
        pi = ew.where(above, k - 1, ew.where(below, 0, prev)).astype(np.int64)
        ni = ew.where(above, k - 1, ew.where(below, 0, prev + 1)).astype(np.int64)
        if method == "midpoint":
            g = ew.where(ew.binary("mod_op", v, 1) == 0, 0.0, 0.5).astype(qdt)
        else:
            g = (v.astype(np.float64) - pf).astype(qdt)
        lo, hi = gather(pi), gather(ni)
        g = g.reshape(kept)
        d = hi - lo
        r = ew.where(g >= 0.5, hi - d * (1 - g), lo + d * g)
        nan_dt = r.dtype
    return ew.where(k.reshape(kept) > 0, r, nan_dt.type(np.nan))


def _quantile(a, q, axis, keepdims, method, nan_aware, percent):
    if method not in _METHODS:
        raise ValueError(f"{method!r} is not a valid method. Use one of: {_METHODS}")
    from .sorting import sort
    x, kept, kd = _prepare(a, axis)
    qa = _qarray(x.dtype, q, percent)
    n = x.shape[-1]
    if n == 0:
        raise IndexError("cannot compute a quantile of an empty slice")
    s = sort(x, axis=-1)
    outs = []
    if nan_aware and s.dtype.kind == "f":
        from . import reductions
        k = reductions.sum(ew.unary("logical_not_op", ew.unary("isnan_op", s)), axis=-1)
        k = k.astype(np.int64).reshape(kept + (1,))
        for qv in qa.reshape(-1):
            outs.append(_nan_one(s, k, kept, np.asarray(qv, qa.dtype), method))
    else:
        for qv in qa.reshape(-1):
            outs.append(_plain_one(s, n, np.asarray(qv, qa.dtype), method))
    res = [o.reshape(kd) if keepdims else o for o in outs]
    if qa.ndim == 0:
        out = res[0]
    else:
        from .manipulation import stack
        out = stack(res, axis=0).reshape(qa.shape + tuple(res[0].shape))
    out._materialize_if_lazy()
    return out


def _out(r, out):
    if out is not None:
        out[...] = r
        return out
    return r


def _check(weights, name):
    if weights is not None:
        raise NotImplementedError(f"{name}(weights=...) is not supported on the device")


def quantile(a, q, axis=None, out=None, overwrite_input=False, method="linear",
             keepdims=False, *, weights=None, interpolation=None):
    _check(weights, "quantile")
    return _out(_quantile(a, q, axis, keepdims, interpolation or method, False, False), out)


def percentile(a, q, axis=None, out=None, overwrite_input=False, method="linear",
               keepdims=False, *, weights=None, interpolation=None):
    _check(weights, "percentile")
    return _out(_quantile(a, q, axis, keepdims, interpolation or method, False, True), out)


def nanquantile(a, q, axis=None, out=None, overwrite_input=False, method="linear",
                keepdims=False, *, weights=None, interpolation=None):
    _check(weights, "nanquantile")
    return _out(_quantile(a, q, axis, keepdims, interpolation or method, True, False), out)


def nanpercentile(a, q, axis=None, out=None, overwrite_input=False, method="linear",
                  keepdims=False, *, weights=None, interpolation=None):
    _check(weights, "nanpercentile")
    return _out(_quantile(a, q, axis, keepdims, interpolation or method, True, True), out)


def _mean2(lo, hi, dt):
    """NumPy's mean of two values of dtype dt (float16 summed in float32,
    integers in float64)."""
    if dt.kind in "iub":
        return (lo.astype(np.float64) + hi.astype(np.float64)) / 2
    if dt == np.float16:
        return ((lo.astype(np.float32) + hi.astype(np.float32)) / 2).astype(np.float16)
    return (lo + hi) / 2


def median(a, axis=None, out=None, overwrite_input=False, keepdims=False):
    from .sorting import sort
    x, kept, kd = _prepare(a, axis)
    n = x.shape[-1]
    dt = x.dtype
    if n == 0:
        from .creation import full
        r = full(kept, np.nan, dtype=np.float64 if dt.kind in "iub" else dt)
    else:
        s = sort(x, axis=-1)
        h = n // 2
        if n % 2:
            mid = s[..., h]
            r = mid.astype(np.float64) if dt.kind in "iub" else _copy(mid)
        else:
            r = _mean2(s[..., h - 1], s[..., h], dt)
        if dt.kind == "f":
            last = s[..., n - 1]
            r = ew.where(ew.unary("isnan_op", last), last, r)
    if keepdims:
        r = r.reshape(kd)
    r._materialize_if_lazy()
    return _out(r, out)


def nanmedian(a, axis=None, out=None, overwrite_input=False, keepdims=False):
    x0 = _asarray(a)
    if x0.dtype.kind != "f":
        return median(x0, axis=axis, out=out, keepdims=keepdims)
    from .sorting import sort
    from .indexing import take_along_axis
    from . import reductions
    x, kept, kd = _prepare(x0, axis)
    n = x.shape[-1]
    dt = x.dtype
    s = sort(x, axis=-1)
    k = reductions.sum(ew.unary("logical_not_op", ew.unary("isnan_op", s)), axis=-1)
    k = k.astype(np.int64).reshape(kept + (1,))
    h = k // 2
    odd = (k % 2) == 1
    lo_i = ew.where(odd, h, h - 1)
    lo_i = ew.where(lo_i < 0, 0, lo_i).astype(np.int64)
    hi_i = ew.where(k > 0, h, 0).astype(np.int64)
    hi_i = ew.where(hi_i > k - 1, ew.where(k > 0, k - 1, 0), hi_i).astype(np.int64)
    lo = take_along_axis(s, lo_i, axis=-1).reshape(kept)
    hi = take_along_axis(s, hi_i, axis=-1).reshape(kept)
    if kept != () and n < 600:
        r = (lo + hi) / 2               # masked-array median: sum in the dtype
    else:
        r = ew.where(odd.reshape(kept), _copy(hi), _mean2(lo, hi, dt))
    r = ew.where(k.reshape(kept) > 0, r, dt.type(np.nan))
    if keepdims:
        r = r.reshape(kd)
    r._materialize_if_lazy()
    return _out(r, out)
