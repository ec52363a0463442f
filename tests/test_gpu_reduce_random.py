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
