"""NumPy routines built from the device ops: comparisons, rounding and
cleanup, set operations, binning and counting, selection, sorting variants,
statistics of pairs, calculus helpers and index helpers.

The reference implements these as NumPy calls on the host (logic_ops.py,
set_ops.py, math_ext.py, sorting.py, index_tricks.py, dtype_utils.py).
Here each is a composition of device kernels -- fused elementwise
expressions, reductions, the radix sort and binary search, gathers,
matmul -- following NumPy's definitions; dtype and shape helpers that
compute no array data are NumPy's own.
"""
from __future__ import annotations

import builtins

import numpy as np

from . import _elementwise as ew
from .ndarray import ndarray, _normalize_axis, _prod

__all__ = ["isclose", "allclose", "array_equal", "array_equiv", "isin", "in1d", "intersect1d",
           "union1d", "setdiff1d", "setxor1d", "round", "around", "fix", "nan_to_num", "real",
           "imag", "angle", "isreal", "iscomplex", "real_if_close", "sinc", "interp", "bincount",
           "digitize", "histogram", "histogram_bin_edges", "lexsort", "partition", "argpartition", "cov", "corrcoef",
           "select", "piecewise", "choose", "gradient", "trapezoid", "convolve", "correlate",
           "identity", "tri", "logspace", "geomspace", "vander", "indices", "ix_",
           "fill_diagonal", "diag_indices", "diag_indices_from", "tril_indices",
           "triu_indices", "tril_indices_from", "triu_indices_from", "ravel_multi_index",
           "unravel_index", "finfo", "iinfo", "result_type", "can_cast", "promote_types",
           "isscalar", "ndim", "shape", "size", "asnumpy", "get_array_module",
           "cumulative_sum", "cumulative_prod"]

finfo = np.finfo
iinfo = np.iinfo
promote_types = np.promote_types
isscalar = np.isscalar


def _asarray(a):
    from .creation import asarray
    return asarray(a)


def _dt(x):
    return x.dtype if isinstance(x, ndarray) else x


def result_type(*arrays_and_dtypes):
    return np.result_type(*[_dt(x) for x in arrays_and_dtypes])


def can_cast(from_, to, casting="safe"):
    return np.can_cast(_dt(from_), to, casting=casting)


def ndim(a):
    return a.ndim if isinstance(a, ndarray) else np.ndim(a)


def shape(a):
    return tuple(a.shape) if isinstance(a, ndarray) else np.shape(a)


def size(a, axis=None):
    if isinstance(a, ndarray):
        return a.size if axis is None else a.shape[axis]
    return np.size(a, axis)


def asnumpy(a):
    """Host copy (a NumPy array) of a device array."""
    return a.get() if isinstance(a, ndarray) else np.asarray(a)


def get_array_module(*args):
    import macmetalpy_amd
    return macmetalpy_amd


# ---------------------------------------------------------- comparisons
def isclose(a, b, rtol=1e-05, atol=1e-08, equal_nan=False):
    """``|a - b| <= atol + rtol * |b|`` for finite values, equality for
    infinities, NaN equal to NaN with ``equal_nan`` (NumPy 2's isclose),
    one fused kernel."""
    x, y = _asarray(a), _asarray(b)
    dt = np.result_type(x.dtype, y.dtype, 1.0)
    x, y = x.astype(dt), y.astype(dt)
    r = ((ew.unary("abs_op", x - y) <= atol + rtol * ew.unary("abs_op", y))
         & ew.unary("isfinite_op", y)) | (x == y)
    if equal_nan:
        r = r | (ew.unary("isnan_op", x) & ew.unary("isnan_op", y))
    return r


def allclose(a, b, rtol=1e-05, atol=1e-08, equal_nan=False):
    from .reductions import all as _all
    return bool(_all(isclose(a, b, rtol=rtol, atol=atol, equal_nan=equal_nan)))


def array_equal(a1, a2, equal_nan=False):
    from .reductions import all as _all
    x, y = _asarray(a1), _asarray(a2)
    if tuple(x.shape) != tuple(y.shape):
        return False
    if x.size == 0:
        return True
    eq = x == y
    if equal_nan and (x.dtype.kind == "f" or y.dtype.kind == "f"):
        eq = eq | (ew.unary("isnan_op", x) & ew.unary("isnan_op", y))
    return bool(_all(eq))


def array_equiv(a1, a2):
    from .reductions import all as _all
    from ._broadcasting import broadcast_shapes
    x, y = _asarray(a1), _asarray(a2)
    try:
        broadcast_shapes(tuple(x.shape), tuple(y.shape))
    except ValueError:
        return False
    return bool(_all(x == y))


# ------------------------------------------------------ rounding / clean
def round(a, decimals=0, out=None):
    """NumPy's round: rint for decimals = 0, else scale by 10**decimals,
    rint and unscale (divide / multiply order as NumPy's); integers with
    decimals >= 0 are returned unchanged."""
    x = _asarray(a)
    if x.dtype.kind in "iub":
        if decimals >= 0:
            r = x.copy()
        else:
            f = 10 ** (-decimals)
            r = (ew.unary("rint_op", x.astype(np.float64) / f) * f).astype(x.dtype)
    elif decimals == 0:
        r = ew.unary("rint_op", x)
    elif decimals > 0:
        f = x.dtype.type(10.0 ** decimals)
        r = ew.unary("rint_op", x * f) / f
    else:
        f = x.dtype.type(10.0 ** (-decimals))
        r = ew.unary("rint_op", x / f) * f
    if out is not None:
        out[...] = r
        return out
    return r


around = round


def fix(x, out=None):
    a = _asarray(x)
    r = ew.unary("trunc_op", a) if a.dtype.kind == "f" else a.copy()
    if out is not None:
        out[...] = r
        return out
    return r


def nan_to_num(x, copy=True, nan=0.0, posinf=None, neginf=None):
    a = _asarray(x)
    if a.dtype.kind != "f":
        return a.copy() if copy else a
    info = np.finfo(a.dtype)
    pos = info.max if posinf is None else posinf
    neg = info.min if neginf is None else neginf
    r = ew.where(ew.unary("isnan_op", a), a.dtype.type(nan), a)
    r = ew.where(ew.unary("isinf_op", a) & (a > 0), a.dtype.type(pos), r)
    r = ew.where(ew.unary("isinf_op", a) & (a < 0), a.dtype.type(neg), r)
    if not copy:
        a[...] = r
        return a
    return r


def real(val):
    return _asarray(val)


def imag(val):
    from .creation import zeros
    a = _asarray(val)
    return zeros(tuple(a.shape), dtype=a.dtype)


def angle(z, deg=False):
    """arctan2(0, z) for real z (pi for negative values and -0.0)."""
    a = _asarray(z)
    dt = np.result_type(a.dtype, 1.0)
    a = a.astype(dt)
    r = ew.binary("atan2_op", dt.type(0), a)
    return r * dt.type(180.0 / np.pi) if deg else r


def isreal(x):
    from .creation import ones
    a = _asarray(x)
    return ones(tuple(a.shape), dtype=np.bool_)


def iscomplex(x):
    from .creation import zeros
    a = _asarray(x)
    return zeros(tuple(a.shape), dtype=np.bool_)


def real_if_close(a, tol=100):
    return _asarray(a)


def sinc(x):
    """sin(pi y) / (pi y) with y = x, 1e-20 at 0 (NumPy's definition)."""
    a = _asarray(x)
    dt = np.result_type(a.dtype, 1.0)
    a = a.astype(dt)
    y = dt.type(np.pi) * ew.where(a == 0, dt.type(1.0e-20), a)
    return ew.unary("sin_op", y) / y


# ------------------------------------------------------------- set ops
def isin(element, test_elements, assume_unique=False, invert=False, *, kind=None):
    """Membership by binary search in the sorted test elements."""
    from .sorting import sort, searchsorted
    from .indexing import take
    e = _asarray(element)
    t = _asarray(test_elements).ravel()
    if t.size == 0:
        from .creation import zeros, ones
        return (ones if invert else zeros)(tuple(e.shape), dtype=np.bool_)
    dt = np.result_type(e.dtype, t.dtype)
    s = sort(t.astype(dt) if t.dtype != dt else t)
    ev = e.astype(dt) if e.dtype != dt else e
    pos = searchsorted(s, ev)
    pc = ew.where(pos >= s.size, s.size - 1, pos)
    found = take(s, pc.ravel().astype(np.int64)).reshape(tuple(e.shape)) == ev
    return ew.unary("logical_not_op", found) if invert else found


def in1d(ar1, ar2, assume_unique=False, invert=False, *, kind=None):
    return isin(_asarray(ar1).ravel(), ar2, invert=invert)


def intersect1d(ar1, ar2, assume_unique=False, return_indices=False):
    from .manipulation import unique, concatenate
    from .sorting import sort
    if return_indices:
        raise NotImplementedError("intersect1d(return_indices=True) is not supported on the device")
    a = _asarray(ar1).ravel() if assume_unique else unique(ar1)
    b = _asarray(ar2).ravel() if assume_unique else unique(ar2)
    aux = sort(concatenate([a, b]))
    if aux.size < 2:
        return aux[:0]
    mask = aux[1:] == aux[:-1]
    return aux[:-1][mask]


def union1d(ar1, ar2):
    from .manipulation import unique, concatenate
    return unique(concatenate([_asarray(ar1).ravel(), _asarray(ar2).ravel()]))


def setdiff1d(ar1, ar2, assume_unique=False):
    from .manipulation import unique
    a = _asarray(ar1).ravel() if assume_unique else unique(ar1)
    return a[isin(a, ar2, invert=True)]


def setxor1d(ar1, ar2, assume_unique=False):
    from .manipulation import unique, concatenate
    from .sorting import sort
    a = _asarray(ar1).ravel() if assume_unique else unique(ar1)
    b = _asarray(ar2).ravel() if assume_unique else unique(ar2)
    aux = sort(concatenate([a, b]))
    n = aux.size
    if n == 0:
        return aux
    flag = ndarray._empty_device((n + 1,), np.bool_)
    flag[0:1] = True
    flag[n:n + 1] = True
    if n > 1:
        flag[1:n] = aux[1:] != aux[:-1]
    return aux[flag[1:] & flag[:-1]]


# ------------------------------------------------------ binning / counts
def digitize(x, bins, right=False):
    """Bin index of each value (binary search over monotonic bins)."""
    from .sorting import searchsorted
    b = _asarray(bins)
    if b.ndim != 1:
        raise ValueError("bins must be 1-dimensional")
    a = _asarray(x)
    side = "left" if right else "right"
    bh = b.get() if b.size else np.zeros(0)
    if b.size > 1 and bh[0] > bh[-1]:            # decreasing bins
        return b.size - searchsorted(b[::-1], a, side=side)
    return searchsorted(b, a, side=side)


def bincount(x, weights=None, minlength=0):
    """Counts of non-negative integers with the device counting kernel;
    weight sums (float64) from the values sorted by key and the run
    boundaries found by binary search (a fixed summation order)."""
    from .sorting import sort, argsort, searchsorted
    from .indexing import take
    from . import reductions
    from .creation import arange, zeros
    a = _asarray(x)
    if a.ndim != 1:
        raise ValueError("object too deep for desired array")
    if a.dtype.kind not in "iub":
        raise TypeError(f"Cannot cast array data from dtype('{a.dtype}') to dtype('int64') "
                        "according to the rule 'safe'")
    if minlength < 0:
        raise ValueError("'minlength' must not be negative")
    if a.size == 0:
        return zeros((minlength,), dtype=np.float64 if weights is not None else np.int64)
    lo, hi = int(reductions.min(a)), int(reductions.max(a))
    if lo < 0 or hi > np.iinfo(np.int64).max:   # uint64 beyond 2^63 reads as negative
        raise ValueError("'list' argument must have no negative elements")
    nb = builtins.max(hi + 1, minlength)
    if weights is None:
        from ._backend import HipBackend
        from ._dtypes import dtype_code
        src = a._ensure_contiguous()
        out = ndarray._empty_device((nb,), np.int64)
        HipBackend().bincount(dtype_code(src.dtype), src.size, src._ptr, nb, out._ptr)
        return out
    ai = a.astype(np.int64)
    edges = arange(nb + 1, dtype=np.int64)
    w = _asarray(weights).astype(np.float64)
    order = argsort(ai)
    s = take(ai, order)
    cw = reductions.cumsum(take(w.ravel(), order))
    from .manipulation import concatenate
    cw = concatenate([zeros((1,), dtype=np.float64), cw])
    pos = searchsorted(s, edges, side="left")
    c = take(cw, pos)
    return c[1:] - c[:-1]


def _outer_edges(x, range):
    """First and last edge as NumPy takes them: the range's values, or the
    data's own min / max scalars (so float32 data gets float32 edges),
    widened by 0.5 when equal."""
    from . import reductions
    if range is not None:
        lo, hi = range
        if lo > hi:
            raise ValueError("max must be larger than min in range parameter.")
        if not (np.isfinite(lo) and np.isfinite(hi)):
            raise ValueError(f"supplied range of [{lo}, {hi}] is not finite")
    elif x.size == 0:
        lo, hi = 0, 1
    else:
        lo, hi = reductions.min(x).get()[()], reductions.max(x).get()[()]
        if not (np.isfinite(lo) and np.isfinite(hi)):
            raise ValueError(f"autodetected range of [{lo}, {hi}] is not finite")
    if lo == hi:
        lo, hi = lo - 0.5, hi + 0.5
    return lo, hi


def _hist_edges(x, bins, range):
    """Host bin edges of a 1-D histogram (a few values, computed as NumPy's
    _get_bin_edges does for integer and array bins)."""
    if isinstance(bins, str):
        raise NotImplementedError("histogram bin estimators (bins=str) are not supported")
    if np.ndim(bins) == 0:
        n = int(bins)
        if n < 1:
            raise ValueError("`bins` must be positive, when an integer")
        lo, hi = _outer_edges(x, range)
        bin_type = np.result_type(lo, hi, x.dtype)
        if np.issubdtype(bin_type, np.integer):
            bin_type = np.result_type(bin_type, float)
        return np.linspace(lo, hi, n + 1, endpoint=True, dtype=bin_type)
    edges = np.asarray(bins.get() if isinstance(bins, ndarray) else bins)
    if edges.ndim != 1:
        raise ValueError("`bins` must be 1d, when an array")
    if np.any(edges[:-1] > edges[1:]):
        raise ValueError("`bins` must increase monotonically, when an array")
    return edges


def histogram_bin_edges(a, bins=10, range=None, weights=None):
    return _asarray(_hist_edges(_asarray(a).ravel(), bins, range))


def histogram(a, bins=10, range=None, density=None, weights=None):
    """Counts per bin (right-open bins, the last one closed) from the sorted
    values and binary searches of the edges; edges as NumPy computes them."""
    from .sorting import sort, argsort, searchsorted
    from .indexing import take
    from . import reductions
    x = _asarray(a).ravel()
    edges = _hist_edges(x, bins, range)
    nb = edges.size - 1
    ge = _asarray(edges)
    exact = x.dtype.kind == "f" or x.dtype.itemsize <= 4
    if weights is None and exact and x.dtype != np.bool_ and nb >= 1:
        # counts by the device kernel; comparisons in double are exact for
        # these dtypes and for the edges (float16 / float32 / float64 / int)
        from ._backend import HipBackend
        from ._dtypes import dtype_code
        src = x._ensure_contiguous()
        e64 = _asarray(np.asarray(edges, dtype=np.float64))._ensure_gpu()
        hist = ndarray._empty_device((nb,), np.int64)
        HipBackend().histogram(dtype_code(src.dtype), src.size, src._ptr, nb + 1, e64._ptr, hist._ptr)
    elif weights is None:
        s = sort(x)
        left = searchsorted(s, ge, side="left")
        last = searchsorted(s, ge[nb:], side="right")
        pos = left.copy()
        pos[nb:] = last
        hist = pos[1:] - pos[:-1]
    else:
        w = _asarray(weights).ravel()
        order = argsort(x)
        s = take(x, order)
        cw = reductions.cumsum(take(w.astype(np.float64), order))
        from .manipulation import concatenate
        from .creation import zeros
        cw = concatenate([zeros((1,), dtype=cw.dtype), cw])
        left = searchsorted(s, ge, side="left")
        last = searchsorted(s, ge[nb:], side="right")
        pos = left.copy()
        pos[nb:] = last
        c = take(cw, pos)
        hist = (c[1:] - c[:-1]).astype(w.dtype)
    if density:
        width = _asarray(np.diff(edges))
        hist = hist / width / reductions.sum(hist)
    return hist, _asarray(edges)


def interp(x, xp, fp, left=None, right=None, period=None):
    """NumPy's interp (compiled_base.c): binary search for the interval,
    slope * (x - xp[j]) + fp[j] in float64, the other endpoint when that is
    NaN, fp[j] when both ends are equal; left / right outside."""
    from .sorting import searchsorted
    from .indexing import take
    if period is not None:
        raise NotImplementedError("interp(period=...) is not supported on the device")
    xs = _asarray(x).astype(np.float64)
    xpa = _asarray(xp).astype(np.float64).ravel()
    fpa = _asarray(fp).astype(np.float64).ravel()
    n = xpa.size
    if n == 0:
        raise ValueError("array of sample points is empty")
    if fpa.size != n:
        raise ValueError("fp and xp are not of the same length.")
    lval = fpa[0:1] if left is None else np.float64(left)
    rval = fpa[n - 1:n] if right is None else np.float64(right)
    lv = float(lval.get()[0]) if isinstance(lval, ndarray) else float(lval)
    rv = float(rval.get()[0]) if isinstance(rval, ndarray) else float(rval)
    j = searchsorted(xpa, xs, side="right") - 1
    jc = ew.where(j < 0, 0, ew.where(j > n - 2, builtins.max(n - 2, 0), j)).astype(np.int64)
    if n == 1:
        res = ew.where(xs < xpa[0], lv, ew.where(xs > xpa[0], rv, fpa[0]))
        return res
    x0, x1 = take(xpa, jc), take(xpa, jc + 1)
    f0, f1 = take(fpa, jc), take(fpa, jc + 1)
    slope = (f1 - f0) / (x1 - x0)
    r = slope * (xs - x0) + f0
    r = ew.where(ew.unary("isnan_op", r), slope * (xs - x1) + f1, r)
    r = ew.where(ew.unary("isnan_op", r) & (f0 == f1), f0, r)
    r = ew.where(xs == x0, f0, r)
    xl, xr = float(xpa[0].get()), float(xpa[n - 1].get())
    r = ew.where(xs == xr, fpa[n - 1], r)
    r = ew.where(xs < xl, lv, ew.where(xs > xr, rv, r))
    return ew.where(ew.unary("isnan_op", xs), xs, r)


# ------------------------------------------------------ sorting variants
def lexsort(keys, axis=-1):
    """Indices sorting by the last key, then the ones before (successive
    stable sorts)."""
    from .sorting import argsort
    from .indexing import take
    ks = [_asarray(k) for k in keys] if not isinstance(keys, ndarray) else \
        [keys[i] for i in builtins.range(keys.shape[0])]
    if not ks:
        raise TypeError("need sequence of keys with len > 0 in lexsort")
    if ks[0].ndim != 1:
        raise NotImplementedError("lexsort of N-D keys is not supported on the device")
    idx = argsort(ks[0], kind="stable")
    for k in ks[1:]:
        idx = take(idx, argsort(take(k, idx), kind="stable"))
    return idx


def _check_kth(a, kth, axis):
    x = _asarray(a)
    n = x.size if axis is None else x.shape[_normalize_axis(axis, x.ndim)]
    for k in np.atleast_1d(np.asarray(kth)).ravel():
        if not -n <= int(k) < n:
            raise ValueError(f"kth(={int(k)}) out of bounds ({n})")
    return x


def partition(a, kth, axis=-1, kind="introselect", order=None):
    """A full sort is a valid partition for every kth: element kth is in
    its sorted place, smaller ones before it and larger ones after."""
    from .sorting import sort
    x = _check_kth(a, kth, axis)
    return sort(x.ravel() if axis is None else x, axis=-1 if axis is None else axis)


def argpartition(a, kth, axis=-1, kind="introselect", order=None):
    from .sorting import argsort
    x = _check_kth(a, kth, axis)
    return argsort(x.ravel() if axis is None else x, axis=-1 if axis is None else axis)


# ------------------------------------------------------- pair statistics
def cov(m, y=None, rowvar=True, bias=False, ddof=None, fweights=None, aweights=None, *,
        dtype=None):
    """Covariance as NumPy computes it (float64 unless dtype says otherwise):
    centred rows, X @ X.T / (N - ddof), through the device matmul."""
    if fweights is not None or aweights is not None:
        raise NotImplementedError("cov with weights is not supported on the device")
    from . import reductions
    from .linalg_top import matmul
    from .manipulation import concatenate
    x = _asarray(m)
    if x.ndim > 2:
        raise ValueError("m has more than 2 dimensions")
    dt = np.result_type(x.dtype, np.float64) if dtype is None else np.dtype(dtype)
    X = x.reshape((1, x.size)) if x.ndim < 2 else x
    if not rowvar and X.shape[0] != 1:
        X = X.T
    if y is not None:
        yy = _asarray(y)
        Y = yy.reshape((1, yy.size)) if yy.ndim < 2 else yy
        if not rowvar and Y.shape[0] != 1:
            Y = Y.T
        X = concatenate([X, Y], axis=0)
    X = X.astype(dt)
    if ddof is None:
        ddof = 0 if bias else 1
    n = X.shape[1]
    fact = n - ddof
    Xc = X - reductions.mean(X, axis=1, keepdims=True)
    c = matmul(Xc, Xc.T.copy()) * dt.type(1.0 / fact) if fact > 0 else matmul(Xc, Xc.T.copy()) / fact
    if c.shape == (1, 1):
        return c.reshape(())
    return c


def corrcoef(x, y=None, rowvar=True, *, dtype=None):
    from .manipulation import diagonal
    c = cov(x, y, rowvar, dtype=dtype)
    if c.ndim == 0:
        return c / c
    d = diagonal(c).copy()
    sd = ew.unary("sqrt_op", d)
    r = c / sd.reshape((sd.size, 1))
    r = r / sd.reshape((1, sd.size))
    return ew.where(r > 1, 1.0, ew.where(r < -1, -1.0, r))


# --------------------------------------------------------------- select
def select(condlist, choicelist, default=0):
    if len(condlist) != len(choicelist):
        raise ValueError("list of cases must be same length as list of conditions")
    if not condlist:
        raise ValueError("select with an empty condition list is not possible")
    # Python scalars stay weakly typed in the result dtype (NumPy's select)
    def kind(c):
        if type(c) in (int, float, complex):
            return c
        return c.dtype if isinstance(c, ndarray) else np.asarray(c).dtype
    choices = list(choicelist)
    dt = np.result_type(*[kind(c) for c in choices], kind(default))
    r = None
    for cond, choice in zip(reversed(condlist), reversed(choices)):
        c = _asarray(cond)
        if c.dtype != np.bool_:
            raise TypeError("invalid entry in condlist: should be boolean ndarray")
        if r is None:
            base = dt.type(default) if np.isscalar(default) else _asarray(default).astype(dt)
        else:
            base = r
        r = ew.where(c, _asarray(choice).astype(dt), base).astype(dt)
    return r


def piecewise(x, condlist, funclist, *args, **kw):
    a = _asarray(x)
    if isinstance(condlist, (ndarray, np.ndarray)) and np.ndim(condlist) == a.ndim:
        condlist = [condlist]
    n = len(condlist)
    if len(funclist) not in (n, n + 1):
        raise ValueError(f"with {n} condition(s), either {n} or {n + 1} functions are expected")
    from .creation import zeros
    r = zeros(tuple(a.shape), dtype=a.dtype)
    if len(funclist) == n + 1:
        others = None
        for c in condlist:
            others = c if others is None else (others | c)
        f = funclist[-1]
        val = f(a, *args, **kw) if callable(f) else f
        r = ew.where(ew.unary("logical_not_op", others), val, r)
    for c, f in zip(condlist, funclist):
        val = f(a, *args, **kw) if callable(f) else f
        r = ew.where(c, val, r).astype(a.dtype)
    return r


def choose(a, choices, out=None, mode="raise"):
    from . import reductions
    idx = _asarray(a)
    n = len(choices)
    if mode == "raise" and idx.size:
        lo, hi = int(reductions.min(idx)), int(reductions.max(idx))
        if lo < 0 or hi >= n:
            raise ValueError("invalid entry in choice array")
    elif mode == "wrap":
        idx = idx % n
    elif mode == "clip":
        idx = ew.where(idx < 0, 0, ew.where(idx >= n, n - 1, idx))
    chs = [_asarray(c) for c in choices]
    dt = np.result_type(*[c.dtype for c in chs])
    r = chs[n - 1].astype(dt)
    for i in builtins.range(n - 2, -1, -1):
        r = ew.where(idx == i, chs[i].astype(dt), r)
    if out is not None:
        out[...] = r
        return out
    return r


# ------------------------------------------------------------- calculus
def gradient(f, *varargs, axis=None, edge_order=1):
    """Second-order central differences inside, one-sided (first order) at
    the edges, unit or scalar spacing."""
    a = _asarray(f)
    if edge_order != 1:
        raise NotImplementedError("gradient(edge_order=2) is not supported on the device")
    axes = builtins.range(a.ndim) if axis is None else (
        (axis,) if isinstance(axis, (int, np.integer)) else tuple(axis))
    axes = [_normalize_axis(x, a.ndim) for x in axes]
    sp = list(varargs) if varargs else [1.0] * len(axes)
    if len(sp) == 1 and len(axes) > 1:
        sp = sp * len(axes)
    dt = np.result_type(a.dtype, np.float64) if a.dtype.kind in "iub" else a.dtype
    x = a.astype(dt)
    outs = []
    for ax, h in zip(axes, sp):
        if not np.isscalar(h):
            raise NotImplementedError("gradient with coordinate arrays is not supported")
        n = a.shape[ax]
        if n < 2:
            raise ValueError("Shape of array too small to calculate a numerical gradient, at "
                             "least (edge_order + 1) elements are required.")
        out = ndarray._empty_device(tuple(a.shape), dt)

        def sl(s):
            return (slice(None),) * ax + (s,)
        if n > 2:
            out[sl(slice(1, -1))] = (x[sl(slice(2, None))] - x[sl(slice(None, -2))]) / dt.type(2.0 * h)
        out[sl(slice(0, 1))] = (x[sl(slice(1, 2))] - x[sl(slice(0, 1))]) / dt.type(h)
        out[sl(slice(n - 1, n))] = (x[sl(slice(n - 1, n))] - x[sl(slice(n - 2, n - 1))]) / dt.type(h)
        outs.append(out)
    return outs[0] if len(outs) == 1 else tuple(outs)


def trapezoid(y, x=None, dx=1.0, axis=-1):
    from .reductions import sum as _sum
    a = _asarray(y)
    ax = _normalize_axis(axis, a.ndim)
    hi = (slice(None),) * ax + (slice(1, None),)
    lo = (slice(None),) * ax + (slice(None, -1),)
    if x is None:
        d = dx
    else:
        xx = _asarray(x)
        if xx.ndim == 1:
            d = xx[1:] - xx[:-1]
            shp = [1] * a.ndim
            shp[ax] = d.shape[0]
            d = d.reshape(tuple(shp))
        else:
            d = xx[hi] - xx[lo]
    return _sum(d * (a[hi] + a[lo]) / 2.0, axis=ax)


def _corr_full(a, v):
    """sum_j a[k + j] * v[j] for every overlap offset (full correlation),
    accumulated over the shorter operand's length with fused multiply-adds."""
    from .creation import zeros
    n, m = a.size, v.size
    dt = np.result_type(a.dtype, v.dtype)
    out = zeros((n + m - 1,), dtype=dt)
    ap = a.astype(dt)
    vh = v.astype(dt)
    for j in builtins.range(m):
        # contribution of v[j]: a shifted so that out[k] += a[k - (m - 1 - j)] * v[j]
        s = m - 1 - j
        out[s:s + n] = out[s:s + n] + ap * vh[j]
    return out


def correlate(a, v, mode="valid"):
    x, y = _asarray(a).ravel(), _asarray(v).ravel()
    if x.size == 0 or y.size == 0:
        raise ValueError("v cannot be empty" if y.size == 0 else "a cannot be empty")
    full = _corr_full(x, y)
    return _mode(full, x.size, y.size, mode, swapped=y.size > x.size)


def convolve(a, v, mode="full"):
    x, y = _asarray(a).ravel(), _asarray(v).ravel()
    if x.size == 0 or y.size == 0:
        raise ValueError("v cannot be empty" if y.size == 0 else "a cannot be empty")
    if y.size > x.size:
        x, y = y, x
    full = _corr_full(x, y[::-1].copy())
    return _mode(full, x.size, y.size, mode)


def _mode(full, n, m, mode, swapped=False):
    """Slice of the full correlation for NumPy's modes.  NumPy correlates
    with the longer operand first and reverses the result when it swapped
    them, so an odd excess is trimmed from the other end then."""
    if mode == "full":
        return full
    if mode == "same":
        L = builtins.max(n, m)
        start = (full.size - L + (1 if swapped else 0)) // 2
        return full[start:start + L].copy()
    if mode == "valid":
        L = builtins.max(n, m) - builtins.min(n, m) + 1
        start = builtins.min(n, m) - 1
        return full[start:start + L].copy()
    raise ValueError(f"mode must be one of 'valid', 'same', or 'full' (got {mode!r})")


# ------------------------------------------------------ index / creation
def identity(n, dtype=None):
    from .creation import eye
    return eye(n, dtype=dtype)


def tri(N, M=None, k=0, dtype=None):
    """Ones at and below diagonal k (creation.py:199-201); the default
    dtype is the library's default float, as for eye."""
    from .manipulation import _tri_mask
    from ._dtypes import resolve_dtype
    M = N if M is None else M
    return _tri_mask((N, M), k, True).astype(resolve_dtype(dtype))


def logspace(start, stop, num=50, endpoint=True, base=10.0, dtype=None, axis=0):
    return _asarray(np.logspace(start, stop, num, endpoint=endpoint, base=base, dtype=dtype,
                                axis=axis))


def geomspace(start, stop, num=50, endpoint=True, dtype=None, axis=0):
    return _asarray(np.geomspace(start, stop, num, endpoint=endpoint, dtype=dtype, axis=axis))


def vander(x, N=None, increasing=False):
    """Powers of x, column by column (x**k by repeated multiplication, as
    NumPy's multiply.accumulate)."""
    from .creation import ones
    a = _asarray(x).ravel()
    N = a.size if N is None else N
    dt = np.promote_types(a.dtype, np.int_)
    a = a.astype(dt)
    out = ones((a.size, N), dtype=dt)
    cols = builtins.range(N) if increasing else builtins.range(N - 1, -1, -1)
    p = None
    for i, c in enumerate(cols):
        if i == 0:
            continue
        p = a if p is None else p * a
        out[:, c] = p
    return out


def indices(dimensions, dtype=int, sparse=False):
    from .creation import arange
    dims = tuple(dimensions)
    nd = len(dims)
    res = []
    for i, d in enumerate(dims):
        shp = [1] * nd
        shp[i] = d
        r = arange(d, dtype=dtype).reshape(tuple(shp))
        res.append(r if sparse else r * _ones(dims, dtype))
    if sparse:
        return tuple(res)
    from .manipulation import stack
    return stack(res, axis=0)


def _ones(dims, dtype):
    from .creation import ones
    return ones(tuple(dims), dtype=dtype)


def ix_(*args):
    out = []
    nd = len(args)
    for k, new in enumerate(args):
        a = _asarray(new)
        if a.ndim != 1:
            raise ValueError("Cross index must be 1 dimensional")
        if a.dtype == np.bool_:
            from .indexing import flatnonzero
            a = flatnonzero(a)
        out.append(a.reshape((1,) * k + (a.size,) + (1,) * (nd - k - 1)))
    return tuple(out)


def fill_diagonal(a, val, wrap=False):
    """Writes through the diagonal view (every ncols + 1 elements of a 2-D
    array; wrap continues past the square part of a tall array)."""
    from .manipulation import diagonal, _view
    if a.ndim < 2:
        raise ValueError("array must be at least 2-d")
    a._materialize_if_lazy()
    a._ensure_gpu()
    if a.ndim == 2:
        r, c = a.shape
        if wrap and r > c:
            if a._strides != (c, 1):
                raise NotImplementedError("fill_diagonal(wrap=True) needs a C-contiguous array")
            n = (a.size + c) // (c + 1)
            _view(a, (n,), (c + 1,), a._offset)[...] = val
            return None
        diagonal(a)[...] = val
        return None
    if len(set(a.shape)) != 1:
        raise ValueError("All dimensions of input must be of equal length")
    _view(a, (a.shape[0],), (builtins.sum(a._strides),), a._offset)[...] = val
    return None


def diag_indices(n, ndim=2):
    from .creation import arange
    idx = arange(n, dtype=np.int64)
    return (idx,) * ndim


def diag_indices_from(arr):
    if arr.ndim < 2 or len(set(arr.shape)) != 1:
        raise ValueError("input array must be at least 2-d and of equal length")
    return diag_indices(arr.shape[0], arr.ndim)


def tril_indices(n, k=0, m=None):
    from .indexing import nonzero
    return nonzero(tri(n, m, k, dtype=bool))


def triu_indices(n, k=0, m=None):
    from .indexing import nonzero
    return nonzero(ew.unary("logical_not_op", tri(n, m, k - 1, dtype=bool)))


def tril_indices_from(arr, k=0):
    return tril_indices(arr.shape[-2], k=k, m=arr.shape[-1])


def triu_indices_from(arr, k=0):
    return triu_indices(arr.shape[-2], k=k, m=arr.shape[-1])


def ravel_multi_index(multi_index, dims, mode="raise", order="C"):
    from . import reductions
    if order != "C":
        raise NotImplementedError("ravel_multi_index(order='F') is not supported")
    dims = tuple(int(d) for d in dims)
    if len(multi_index) != len(dims):
        raise ValueError("parameter multi_index must be a sequence of length " + str(len(dims)))
    r = None
    for idx, d in zip(multi_index, dims):
        i = _asarray(idx).astype(np.int64)
        if mode == "raise" and i.size:
            if int(reductions.min(i)) < 0 or int(reductions.max(i)) >= d:
                raise ValueError("invalid entry in coordinates array")
        elif mode == "wrap":
            i = i % d
        elif mode == "clip":
            i = ew.where(i < 0, 0, ew.where(i >= d, d - 1, i))
        r = i if r is None else r * d + i
    return r


def unravel_index(indices, shape, order="C"):
    from .indexing import _unravel
    from . import reductions
    if order != "C":
        raise NotImplementedError("unravel_index(order='F') is not supported")
    shp = (int(shape),) if isinstance(shape, (int, np.integer)) else tuple(int(s) for s in shape)
    idx = _asarray(indices).astype(np.int64)
    n = _prod(shp)
    if idx.size and (int(reductions.min(idx)) < 0 or int(reductions.max(idx)) >= n):
        raise ValueError(f"index {int(reductions.max(idx))} is out of bounds for array with "
                         f"size {n}")
    return tuple(c.reshape(tuple(idx.shape)) if hasattr(c, "reshape") else c
                 for c in _unravel(idx.ravel(), shp))


def cumulative_sum(x, /, *, axis=None, dtype=None, out=None, include_initial=False):
    from .reductions import cumsum
    from .manipulation import concatenate
    a = _asarray(x)
    if axis is None:
        if a.ndim > 1:
            raise ValueError("axis must be specified for arrays with more than one dimension")
        axis = 0
    r = cumsum(a, axis=axis, dtype=dtype)
    if include_initial:
        ax = _normalize_axis(axis, a.ndim)
        shp = list(r.shape)
        shp[ax] = 1
        from .creation import zeros
        r = concatenate([zeros(tuple(shp), dtype=r.dtype), r], axis=ax)
    if out is not None:
        out[...] = r
        return out
    return r


def cumulative_prod(x, /, *, axis=None, dtype=None, out=None, include_initial=False):
    from .reductions import cumprod
    from .manipulation import concatenate
    a = _asarray(x)
    if axis is None:
        if a.ndim > 1:
            raise ValueError("axis must be specified for arrays with more than one dimension")
        axis = 0
    r = cumprod(a, axis=axis, dtype=dtype)
    if include_initial:
        ax = _normalize_axis(axis, a.ndim)
        shp = list(r.shape)
        shp[ax] = 1
        from .creation import ones
        r = concatenate([ones(tuple(shp), dtype=r.dtype), r], axis=ax)
    if out is not None:
        out[...] = r
        return out
    return r
