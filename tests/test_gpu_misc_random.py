"""Seeded random casts, where / clip, and sorts against NumPy.

* astype (reference ndarray.astype, ndarray.py:2155-2197, and the cast
  kernels of _kernel_cache.py:44-189): every pair of the ten device dtypes
  on contiguous and strided views, values with the source dtype's edge
  cases; float sources are kept inside the target's range for integer
  targets (NumPy leaves out-of-range float -> int conversion to the
  platform).  Bit for bit, NaN == NaN.
* where / clip (reference math_ops.py:106-155, ndarray.py:1809-1893):
  broadcast condition and branches of mixed dtypes and Python scalars;
  clip with array or scalar bounds, one side None.  Bit for bit.
* sort / argsort (stable) / searchsorted (reference sorting.py:60-263):
  random dtypes, N-D shapes, axes, NaNs and signed zeros; sort with
  kind="stable" and argsort give NumPy's values / indices bit for bit, the
  default sort equal values (its order among -0.0 / +0.0 and among NaNs is
  not fixed, in NumPy either)."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd._dtypes import resolve_dtype

pytestmark = pytest.mark.gpu

DTYPES = [np.bool_, np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64,
          np.float16, np.float32, np.float64]


def _same(got, want):
    got = np.ascontiguousarray(got)
    want = np.ascontiguousarray(want)
    assert got.shape == want.shape and got.dtype == want.dtype, (got.shape, want.shape,
                                                                 got.dtype, want.dtype)
    gn = np.isnan(got) if got.dtype.kind == "f" else False
    wn = np.isnan(want) if want.dtype.kind == "f" else False
    same = (got.view(np.uint8).reshape(got.shape + (-1,))
            == want.view(np.uint8).reshape(want.shape + (-1,))).all(-1)
    bad = ~(same | (gn & wn))
    assert not np.any(bad), (got[bad][:4], want[bad][:4])


def _values(rng, shape, dt, target=None):
    dt = np.dtype(dt)
    if dt == np.bool_:
        return rng.random(shape) < 0.5
    if dt.kind in "iu":
        info = np.iinfo(dt)
        v = rng.integers(info.min, info.max, shape, dtype=dt, endpoint=True)
        flat = v.reshape(-1)
        k = min(flat.size, 4)
        flat[rng.integers(0, flat.size, k)] = rng.choice(np.array([0, info.min, info.max, 1], dt), k)
        return v
    tgt = np.dtype(target) if target is not None else None
    if tgt is not None and tgt.kind in "iu":
        info = np.iinfo(tgt)
        lo = max(float(info.min), -6e4 if dt == np.float16 else -1e15)
        hi = min(float(info.max), 6e4 if dt == np.float16 else 1e15)
        v = rng.uniform(lo, hi, shape)
        v = np.where(rng.random(shape) < 0.5, np.trunc(v), v)
        v = v.astype(dt)
        # rounding to dt can leave the target range at its top end
        return np.clip(v, np.array(lo, dt), np.nextafter(np.array(hi, dt), np.array(0, dt)))
    v = (rng.standard_normal(shape) * 1e3).astype(dt)
    flat = v.reshape(-1)
    k = min(flat.size, 8)
    sp = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 1e-7, -1e30], np.float64)
    with np.errstate(all="ignore"):
        flat[rng.integers(0, flat.size, k)] = rng.choice(sp, k).astype(dt)
    return v


@pytest.mark.parametrize("seed", range(120))
def test_random_astype(seed):
    rng = np.random.default_rng(17000 + seed)
    src = DTYPES[int(rng.integers(len(DTYPES)))]
    dst = DTYPES[int(rng.integers(len(DTYPES)))]
    shape = [(1000,), (33, 65), (4, 7, 9)][int(rng.integers(3))]
    strided = rng.random() < 0.4
    base = _values(rng, (2 * shape[0],) + shape[1:] if strided else shape, src, dst)
    h = base[::2] if strided else base
    d = cp.array(base)[::2] if strided else cp.array(base)
    with np.errstate(all="ignore"):
        want = h.astype(dst)
    _same(d.astype(dst).get(), want)


@pytest.mark.parametrize("seed", range(80))
def test_random_where_clip(seed):
    rng = np.random.default_rng(19000 + seed)
    shapes = [((7, 33), (7, 33), (7, 33)), ((7, 1), (1, 33), (33,)), ((33,), (7, 33), (7, 1))]
    sc, sx, sy = shapes[int(rng.integers(len(shapes)))]
    cond = rng.random(sc) < 0.5
    ops = []
    for s in (sx, sy):
        r = rng.random()
        if r < 0.2:
            ops.append(float(rng.choice([2.5, -0.0, 7.0])) if rng.random() < 0.5
                       else int(rng.integers(-5, 5)))
        else:
            dt = DTYPES[1 + int(rng.integers(len(DTYPES) - 1))]
            ops.append(_values(rng, s, dt))
    want = np.where(cond, *ops)
    want = want.astype(resolve_dtype(want.dtype), copy=False)
    got = cp.where(cp.array(cond), *[cp.array(o) if isinstance(o, np.ndarray) else o for o in ops])
    _same(got.get(), want)
    # clip: bounds as arrays or scalars, one side may be None
    dt = DTYPES[1 + int(rng.integers(len(DTYPES) - 1))]
    x = _values(rng, (7, 33), dt)
    if np.dtype(dt).kind == "f":
        lo, hi = -100.0, 250.0
    else:
        info = np.iinfo(dt)
        lo, hi = int(max(info.min, -1000)), int(min(info.max, 30000))
    lo_a = np.full((1, 33), lo).astype(dt)
    kind = int(rng.integers(4))
    args = [(lo, hi), (None, hi), (lo, None), (lo_a, hi)][kind]
    with np.errstate(all="ignore"):
        want = np.clip(x, *args)
    got = cp.clip(cp.array(x), *[cp.array(a) if isinstance(a, np.ndarray) else a for a in args])
    _same(got.get(), want)


@pytest.mark.parametrize("seed", range(80))
def test_random_sort_argsort_searchsorted(seed):
    rng = np.random.default_rng(21000 + seed)
    dt = DTYPES[1 + int(rng.integers(len(DTYPES) - 1))]
    shape = [(5000,), (17, 300), (3, 40, 9), (1,), (257, 64)][int(rng.integers(5))]
    x = _values(rng, shape, dt)
    if np.dtype(dt).kind in "iu" and rng.random() < 0.5:    # many ties
        x = (x % 7).astype(dt)
    axis = int(rng.integers(-len(shape), len(shape))) if rng.random() < 0.8 else -1
    d = cp.array(x)
    # the default sort's order among equal keys (-0.0 and +0.0, NaNs) is not
    # fixed, in NumPy either: equal values; kind="stable" keeps input order,
    # so it is bit for bit
    got, want = cp.sort(d, axis=axis).get(), np.sort(x, axis=axis)
    assert got.dtype == want.dtype and got.shape == want.shape
    assert np.array_equal(got, want, equal_nan=want.dtype.kind == "f")
    _same(cp.sort(d, axis=axis, kind="stable").get(), np.sort(x, axis=axis, kind="stable"))
    _same(cp.argsort(d, axis=axis, kind="stable").get(), np.argsort(x, axis=axis, kind="stable"))
    # searchsorted of random values (and of the sorted values themselves) in a sorted 1-D array
    s = np.sort(x.reshape(-1))
    q = np.concatenate([_values(rng, (500,), dt), s[:: max(1, s.size // 50)]])
    side = "left" if rng.random() < 0.5 else "right"
    _same(cp.searchsorted(cp.array(s), cp.array(q), side=side).get(),
          np.searchsorted(s, q, side=side))


def test_clip_python_int_bounds_beyond_dtype():
    """NumPy's clip ignores a Python int bound beyond the dtype on its own
    side and raises OverflowError for one beyond the other side."""
    for dt, lo, hi in ((np.uint16, -5, 5), (np.uint16, -5, None), (np.uint16, 0, 70000),
                       (np.int16, -40000, 2), (np.int16, -2, 40000),
                       (np.uint16, 70000, 80000), (np.uint16, None, -5), (np.int16, 40000, 50000)):
        x = np.array([1, 2, 600, 0], dt)
        try:
            want = np.clip(x, lo, hi)
        except OverflowError:
            with pytest.raises(OverflowError):
                cp.clip(cp.array(x), lo, hi).get()
            continue
        _same(cp.clip(cp.array(x), lo, hi).get(), want)
        _same(cp.array(x).clip(lo, hi).get(), want)
