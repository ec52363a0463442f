"""Seeded random indexing keys: reads and assignments against NumPy.

The reference indexes device arrays through ndarray.__getitem__ /
__setitem__ (ndarray.py:893-957), following NumPy's rules.  Each case here
draws a 1-4-D array (optionally a strided view of a larger one) and a key
made of per-axis items -- integers (negative too), slices with any start,
stop and step, integer arrays sharing one broadcast shape, or one boolean
mask -- with None inserted, an Ellipsis replacing a run of whole-axis
slices, and trailing items dropped.  Reads must match NumPy's result
(shape, dtype, values); assignments of a Python scalar, a same-shaped array
or an array broadcast along the last dimension must leave the same array as
NumPy's.  Keys with an out-of-range integer array raise IndexError, as in
NumPy.  Assignment keys never repeat an element (which write lands would be
unspecified)."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu

EXTENTS = [1, 2, 3, 5, 8, 13, 64]
DTYPES = [np.float32, np.int32, np.float64, np.int16, np.bool_, np.float16]


def _data(rng, shape, dtype):
    if dtype == np.bool_:
        return rng.random(shape) < 0.5
    return (rng.standard_normal(shape) * 100).astype(dtype)


def _key(rng, shape, for_set):
    """A valid key for ``shape`` (no repeated elements when ``for_set``)."""
    ndim = len(shape)
    use_mask = rng.random() < 0.2
    adv_shape = [(3,), (2, 3), (1,), (0,), (4,)][int(rng.integers(5))]
    n_adv = int(np.prod(adv_shape))
    items = []
    mask_done = False
    for d, n in enumerate(shape):
        r = rng.random()
        if use_mask and not mask_done and r < 0.35:
            items.append(("mask", rng.random(n) < 0.5))
            mask_done = True
        elif not use_mask and r < 0.3 and (not for_set or n >= n_adv):
            if for_set:                                     # distinct positions
                v = rng.permutation(n)[:n_adv]
            else:
                v = rng.integers(0, n, n_adv) if n else np.zeros(n_adv, np.int64)
            v = np.where(rng.random(n_adv) < 0.3, v - n, v)  # negative forms
            items.append(("arr", v.reshape(adv_shape).astype(np.int64)))
        elif r < 0.5 and n > 0:
            items.append(("int", int(rng.integers(-n, n))))
        elif r < 0.85:
            step = [None, 1, 2, 3, -1, -2][int(rng.integers(6))]
            lo = None if rng.random() < 0.4 else int(rng.integers(-n - 2, n + 3))
            hi = None if rng.random() < 0.4 else int(rng.integers(-n - 2, n + 3))
            items.append(("slice", slice(lo, hi, step)))
        else:
            items.append(("all", slice(None)))
    # put an Ellipsis over a run of whole-axis items, or drop trailing ones
    # (not both: after an Ellipsis the items align with the last axes)
    runs = [i for i, it in enumerate(items) if it[0] == "all"]
    if runs and rng.random() < 0.4:
        i = runs[int(rng.integers(len(runs)))]
        j = i
        while j + 1 < len(items) and items[j + 1][0] == "all":
            j += 1
        items[i:j + 1] = [("ell", Ellipsis)]
    else:
        while items and items[-1][0] == "all" and rng.random() < 0.5:
            items.pop()
    # newaxis
    if rng.random() < 0.25:
        items.insert(int(rng.integers(len(items) + 1)), ("none", None))
    return tuple(v for _, v in items)


def _to_dev(key):
    return tuple(cp.array(k) if isinstance(k, np.ndarray) else k for k in key)


def _case(seed):
    rng = np.random.default_rng(11000 + seed)
    ndim = int(rng.integers(1, 5))
    shape = tuple(int(rng.choice(EXTENTS)) for _ in range(ndim))
    dtype = DTYPES[int(rng.integers(len(DTYPES)))]
    strided = rng.random() < 0.35
    if strided:                                            # a view with offset and steps
        big = _data(rng, tuple(2 * n + 1 for n in shape), dtype)
        sl = tuple(slice(1, 1 + 2 * n, 2) for n in shape)
    else:
        big = _data(rng, shape, dtype)
        sl = tuple(slice(None) for _ in shape)
    return rng, shape, dtype, big, sl


@pytest.mark.parametrize("seed", range(120))
def test_random_getitem(seed):
    rng, shape, dtype, big, sl = _case(seed)
    h = big[sl]
    g = cp.array(big)[sl]
    for _ in range(6):
        key = _key(rng, shape, for_set=False)
        want = h[key]
        got = g[_to_dev(key)]
        got = got.get() if isinstance(got, cp.ndarray) else np.asarray(got)
        want = np.asarray(want)
        assert got.shape == want.shape and got.dtype == want.dtype, (key, got.shape, want.shape)
        assert np.array_equal(got, want, equal_nan=want.dtype.kind == "f"), key


@pytest.mark.parametrize("seed", range(120))
def test_random_setitem(seed):
    rng, shape, dtype, big, sl = _case(seed)
    hb = big.copy()
    gb = cp.array(big)
    h, g = hb[sl], gb[sl]
    for _ in range(4):
        key = _key(rng, shape, for_set=True)
        sel = h[key].shape
        r = rng.random()
        if r < 0.3:
            value = True if dtype == np.bool_ else (3 if np.dtype(dtype).kind == "i" else 2.5)
            dev_value = value
        elif r < 0.7 or not sel:
            value = _data(rng, sel, dtype); dev_value = cp.array(value)
        else:
            value = _data(rng, sel[-1:], dtype); dev_value = cp.array(value)
        h[key] = value
        g[_to_dev(key)] = dev_value
        got = gb.get()
        assert np.array_equal(got, hb, equal_nan=hb.dtype.kind == "f"), key


@pytest.mark.parametrize("seed", range(16))
def test_random_out_of_range_raises(seed):
    rng, shape, dtype, big, sl = _case(seed)
    g = cp.array(big)[sl]
    h = big[sl]
    d = int(rng.integers(len(shape)))
    n = shape[d]
    bad = np.array([0, n if rng.random() < 0.5 else -n - 1], np.int64)
    key = tuple(bad if i == d else slice(None) for i in range(len(shape)))
    with pytest.raises(IndexError):
        h[key]
    with pytest.raises(IndexError):
        g[_to_dev(key)]
    with pytest.raises(IndexError):
        g[_to_dev(key)] = 0
