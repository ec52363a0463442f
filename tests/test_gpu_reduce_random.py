"""Seeded random reductions and scans over N-D shapes, axes and views.

The reference reduces along one axis or the whole array
(ndarray._reduce / _reduce_axis, ndarray.py:1895-2066; reductions.py:74-418)
and scans with ndarray._prefix_scan (ndarray.py:2068-2152), all checked
against NumPy in its tests (tests/test_reductions.py:29-60, 472-494).  Here
each case draws a 1-4-D shape with odd extents, a dtype, a view (axis
permutation, stepped or reversed slice), an op and its axis argument (None,
an int, a negative int or a tuple; keepdims), and compares with NumPy on the
same view:

* integer and bool results, max / min / argmax / argmin / any / all:
  bit for bit, with NumPy's result dtype and shape;
* float sums, means and scans (accumulated in float64): within one unit in
  the last place of the float64-accumulated result, plus float64 rounding
  over the terms;
* var / std: within 1e-5 relative of the float64 evaluation (plus the same
  rounding allowance)."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu

EXTENTS = [1, 2, 3, 5, 17, 64, 129, 257, 1000]
DTYPES = [np.float32, np.float32, np.float64, np.float16, np.int32, np.int64, np.int16,
          np.uint16, np.bool_]
OPS = ["sum", "sum", "mean", "max", "min", "argmax", "argmin", "any", "all", "prod",
       "cumsum", "cumsum", "var", "std"]


def _draw(rng, shape, dtype, op):
    if dtype == np.bool_:
        return rng.random(shape) < 0.5
    if op == "prod":                      # keep products representable
        if np.dtype(dtype).kind == "f":
            return rng.uniform(0.9, 1.1, shape).astype(dtype)
        vals = [1, 1, 3] if dtype == np.uint16 else [-1, 1, 1]   # unsigned products wrap
        return rng.choice(np.array(vals, dtype=dtype), shape)
    if np.dtype(dtype).kind == "f":
        return rng.standard_normal(shape).astype(dtype)
    if dtype == np.uint16:
        return rng.integers(0, 60000, shape, dtype=np.uint16)
    return rng.integers(-1000, 1000, shape).astype(dtype)


def _case(seed):
    rng = np.random.default_rng(7000 + seed)
    while True:
        ndim = int(rng.integers(1, 5))
        shape = tuple(int(rng.choice(EXTENTS)) for _ in range(ndim))
        if np.prod(shape) <= 1_500_000:
            break
    dtype = DTYPES[int(rng.integers(len(DTYPES)))]
    op = OPS[int(rng.integers(len(OPS)))]
    base = _draw(rng, shape, dtype, op)
    # the view: a permutation of the axes, then a stepped or reversed slice
    views = []
    if ndim > 1 and rng.random() < 0.4:
        views.append(("transpose", tuple(int(i) for i in rng.permutation(ndim))))
    if rng.random() < 0.4:
        ax = int(rng.integers(ndim))
        views.append(("slice", ax, int(rng.choice([2, 3, -1, -2]))))
    # the axis argument
    r = rng.random()
    if op in ("argmax", "argmin", "cumsum") or ndim == 1:
        axis = None if r < 0.3 else int(rng.integers(-ndim, ndim))
    elif r < 0.25:
        axis = None
    elif r < 0.75:
        axis = int(rng.integers(-ndim, ndim))
    else:
        k = int(rng.integers(2, ndim + 1))
        axis = tuple(int(i) for i in rng.choice(ndim, k, replace=False))
    keepdims = op != "cumsum" and rng.random() < 0.3
    return base, views, op, axis, keepdims


def _view(m, x, views):
    for v in views:
        if v[0] == "transpose":
            x = x.transpose(v[1])
        else:
            _, ax, step = v
            idx = [slice(None)] * x.ndim
            idx[ax] = slice(None, None, step)
            x = x[tuple(idx)]
    return x


def _run(m, x, op, axis, keepdims):
    if op == "cumsum":
        return m.cumsum(x, axis=axis)
    if op in ("argmax", "argmin"):
        return getattr(m, op)(x, axis=axis, keepdims=keepdims)
    return getattr(m, op)(x, axis=axis, keepdims=keepdims)


@pytest.mark.parametrize("seed", range(160))
def test_random_reduction(seed):
    base, views, op, axis, keepdims = _case(seed)
    h = _view(np, base, views)
    d = _view(cp, cp.array(base), views)
    if h.size == 0:
        pytest.skip("empty view")
    with np.errstate(all="ignore"):
        want = np.asarray(_run(np, h, op, axis, keepdims))
    got = _run(cp, d, op, axis, keepdims)
    got = np.asarray(got.get() if isinstance(got, cp.ndarray) else got)
    assert got.shape == want.shape, (op, axis, keepdims, got.shape, want.shape)
    assert got.dtype == want.dtype, (op, axis, got.dtype, want.dtype)
    if want.dtype.kind != "f" or op in ("max", "min"):
        np.testing.assert_array_equal(got, want)
        return
    # float results: the float64-accumulated value of the same view
    h64 = h.astype(np.float64)
    with np.errstate(all="ignore"):
        ref = np.asarray(_run(np, h64, op, axis, keepdims))
        if op == "cumsum":
            mag = np.cumsum(np.abs(h64), axis=axis)
        elif op in ("var", "std"):
            mag = np.asarray(np.sum(h64 * h64, axis=axis, keepdims=keepdims))
        elif op == "prod":
            mag = np.abs(ref)
        else:
            mag = np.asarray(np.sum(np.abs(h64), axis=axis, keepdims=keepdims))
    tol = np.spacing(np.abs(ref).astype(want.dtype)).astype(np.float64) + 1e-12 * mag
    if op in ("var", "std"):
        tol = tol + 1e-5 * np.abs(ref)
    if op == "prod":
        tol = tol + 1e-6 * np.abs(ref) * (1 if want.dtype == np.float64 else 4)
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= tol), (op, axis, float(np.max(err - tol)))


KW_OPS = ["sum", "prod", "mean", "max", "min", "var", "std", "cumsum", "cumprod"]
NAN_OPS = ["nansum", "nanmean", "nanmax", "nanmin", "nanargmax", "nanargmin", "nanvar",
           "nanstd", "nanprod", "nancumsum"]


def _kw_case(seed):
    """Reductions with keyword arguments: dtype=, ddof=, initial=, where=."""
    rng = np.random.default_rng(25000 + seed)
    ndim = int(rng.integers(1, 4))
    shape = tuple(int(rng.choice([1, 3, 17, 64, 129])) for _ in range(ndim))
    dtype = [np.float32, np.float64, np.int16, np.int32, np.uint16, np.float16][int(rng.integers(6))]
    op = KW_OPS[int(rng.integers(len(KW_OPS)))]
    x = _draw(rng, shape, dtype, "prod" if op in ("prod", "cumprod") else op)
    axis = None if rng.random() < 0.3 else int(rng.integers(-ndim, ndim))
    kw = {}
    if op in ("sum", "prod", "mean", "cumsum", "cumprod") and rng.random() < 0.5:
        kw["dtype"] = [np.float64, np.int64, np.float32, np.int32][int(rng.integers(4))]
        if op in ("cumsum", "cumprod", "prod") and np.dtype(kw["dtype"]).kind == "f" and np.dtype(dtype).kind in "iu":
            kw["dtype"] = np.float64
    if op in ("var", "std"):
        kw["ddof"] = int(rng.integers(0, 2))
    if op in ("sum", "prod", "max", "min") and rng.random() < 0.4:
        kw["initial"] = [0, 1, -5, 3][int(rng.integers(4))] if np.dtype(dtype).kind != "u" else 3
    int_mean = op == "mean" and np.dtype(kw.get("dtype", np.float64)).kind in "iu"
    if op in ("sum", "prod", "max", "min", "mean") and rng.random() < 0.4 and not int_mean:
        # (an integer mean of an empty selection converts NaN to an integer,
        # which NumPy leaves to the platform)
        kw["where"] = rng.random(shape[-1:] if rng.random() < 0.5 else shape) < 0.7
        if op in ("max", "min") and "initial" not in kw:
            kw["initial"] = 3
    if op not in ("cumsum", "cumprod") and rng.random() < 0.3:
        kw["keepdims"] = True
    return x, op, axis, kw


@pytest.mark.parametrize("seed", range(120))
def test_random_reduction_kwargs(seed):
    x, op, axis, kw = _kw_case(seed)
    dkw = dict(kw)
    if "where" in dkw:
        dkw["where"] = cp.array(kw["where"])
    with np.errstate(all="ignore"):
        want = np.asarray(getattr(np, op)(x, axis=axis, **kw))
    want = want.astype(cp_dtype(want.dtype), copy=False)
    got = getattr(cp, op)(cp.array(x), axis=axis, **dkw)
    got = np.asarray(got.get() if isinstance(got, cp.ndarray) else got)
    assert got.shape == want.shape and got.dtype == want.dtype, (op, kw, got.dtype, want.dtype)
    if want.dtype.kind != "f" or op in ("max", "min"):
        np.testing.assert_array_equal(got, want)
        return
    # the elements are first converted to the requested dtype, as NumPy does
    x64 = (x.astype(kw["dtype"]) if "dtype" in kw else x).astype(np.float64)
    kw64 = {k: v for k, v in kw.items() if k != "dtype"}
    with np.errstate(all="ignore"):
        ref = np.asarray(getattr(np, op)(x64, axis=axis, **kw64), dtype=np.float64)
        mag = np.asarray(np.sum(np.abs(x64) ** (2 if op in ("var", "std") else 1), axis=axis,
                                keepdims=kw.get("keepdims", False))) if op not in ("cumsum", "cumprod") else np.abs(ref)
    rel = 1e-5 if op in ("var", "std", "prod", "cumprod") else 0
    tol = (np.spacing(np.abs(ref).astype(want.dtype)).astype(np.float64) + 1e-12 * mag
           + rel * np.abs(ref))
    if want.dtype == np.float16:
        tol = tol + 1e-3 * np.abs(ref)
    g64 = got.astype(np.float64)
    with np.errstate(invalid="ignore"):
        ok = (g64 == ref) | (np.isnan(g64) & np.isnan(ref)) | (np.abs(g64 - ref) <= tol)
    assert np.all(ok), (op, kw)              # (ddof = n gives inf / NaN, as in NumPy)


def cp_dtype(dt):
    from macmetalpy_amd._dtypes import resolve_dtype
    return resolve_dtype(dt)


@pytest.mark.parametrize("seed", range(120))
def test_random_nan_reduction(seed):
    """NaN-ignoring reductions (reference nan_ops.py:60-100) on float data
    with NaN runs, all-NaN slices included."""
    rng = np.random.default_rng(27000 + seed)
    ndim = int(rng.integers(1, 4))
    shape = tuple(int(rng.choice([1, 2, 5, 17, 64, 129])) for _ in range(ndim))
    dtype = [np.float32, np.float64, np.float16][int(rng.integers(3))]
    op = NAN_OPS[int(rng.integers(len(NAN_OPS)))]
    x = rng.standard_normal(shape).astype(dtype)
    x[rng.random(shape) < rng.choice([0.1, 0.5, 0.95])] = np.nan
    if rng.random() < 0.3 and ndim > 1:                     # an all-NaN slice
        idx = [slice(None)] * ndim
        idx[0] = 0
        x[tuple(idx)] = np.nan
    axis = None if rng.random() < 0.3 else int(rng.integers(-ndim, ndim))
    d = cp.array(x)
    try:
        with np.errstate(all="ignore"), np.testing.suppress_warnings() as sup:
            sup.filter(RuntimeWarning)
            want = np.asarray(getattr(np, op)(x, axis=axis))
        err = None
    except ValueError as e:                                  # all-NaN arg-reductions
        err = e
    if err is not None:
        with pytest.raises(ValueError):
            getattr(cp, op)(d, axis=axis).get()
        return
    with np.testing.suppress_warnings() as sup:
        sup.filter(RuntimeWarning)
        got = getattr(cp, op)(d, axis=axis)
        got = np.asarray(got.get() if isinstance(got, cp.ndarray) else got)
    assert got.shape == want.shape and got.dtype == want.dtype, (op, got.dtype, want.dtype)
    if want.dtype.kind != "f" or op in ("nanmax", "nanmin"):
        np.testing.assert_array_equal(got, want)
        return
    x64 = x.astype(np.float64)
    with np.errstate(all="ignore"), np.testing.suppress_warnings() as sup:
        sup.filter(RuntimeWarning)
        ref = np.asarray(getattr(np, op)(x64, axis=axis), dtype=np.float64)
        mag = np.asarray(np.nansum(np.abs(x64) ** (2 if op in ("nanvar", "nanstd") else 1),
                                   axis=axis)) if op != "nancumsum" else np.nancumsum(np.abs(x64), axis=axis)
    rel = 1e-5 if op in ("nanvar", "nanstd", "nanprod") else 0
    tol = (np.spacing(np.abs(np.nan_to_num(ref)).astype(want.dtype)).astype(np.float64)
           + 1e-12 * np.nan_to_num(mag) + rel * np.abs(np.nan_to_num(ref)))
    if want.dtype == np.float16:
        tol = tol + 1e-3 * np.abs(np.nan_to_num(ref))
    g64 = got.astype(np.float64)
    with np.errstate(invalid="ignore"):
        ok = (g64 == ref) | (np.isnan(g64) & np.isnan(ref)) | (np.abs(g64 - ref) <= tol)
    assert np.all(ok), op
