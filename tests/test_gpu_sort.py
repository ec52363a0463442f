"""sort / argsort / searchsorted on the GPU against the oracle (NumPy).
Bars: argsort equal to NumPy's stable argsort; sort(kind='stable') bit for
bit; default sort equal in value (NaN positions equal, -0.0 == +0.0);
searchsorted exact."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

DTYPES = [np.float32, np.float64, np.float16, np.int32, np.uint32, np.int64, np.uint64,
          np.int16, np.uint16, np.bool_]
SIZES = [0, 1, 2, 255, 4095, 4096, 4097, 100003]


def _data(n, dtype, seed):
    rng = np.random.default_rng(seed)
    dt = np.dtype(dtype)
    if dt.kind == "f":
        x = (rng.standard_normal(n) * 4).astype(dtype)
        x[rng.random(n) < 0.3] = 0.0  # ties
        k = min(n, 9)
        x[:k] = np.array([np.nan, -0.0, 0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 0.0],
                         dtype)[:k]
        if n > 20:
            x[rng.integers(0, n, n // 10)] = np.nan
            x[rng.integers(0, n, n // 10)] = -0.0
        return rng.permutation(x)
    if dt.kind == "b":
        return rng.random(n) < 0.5
    info = np.iinfo(dtype)
    x = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
    if n > 10:
        x[rng.integers(0, n, n // 3)] = x[0]  # many ties
        x[:3] = [info.min, info.max, 0]
    return x


def _value_equal(got, want):
    assert got.dtype == want.dtype and got.shape == want.shape
    assert np.array_equal(got, want, equal_nan=want.dtype.kind == "f")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", SIZES)
def test_sort_argsort_1d(dtype, n):
    x = _data(n, dtype, n + 1)
    cx = cp.array(x)
    idx = cp.argsort(cx).get()
    assert idx.dtype == np.int64
    assert np.array_equal(idx, ref.argsort_stable(x))
    _value_equal(cp.sort(cx).get(), ref.sort(x))
    got = cp.sort(cx, kind="stable").get()
    want = ref.sort(x, kind="stable")
    assert np.array_equal(got.view(f"u{got.itemsize}") if got.dtype.kind == "f" else got,
                          want.view(f"u{want.itemsize}") if want.dtype.kind == "f" else want)


@pytest.mark.parametrize("shape,axis", [((37, 1001), -1), ((37, 1001), 0), ((37, 1001), None),
                                        ((5, 7, 300), 1), ((20000, 3), -1), ((3, 70000), 1),
                                        ((4, 5, 6), 0)])
@pytest.mark.parametrize("dtype", [np.float32, np.int64, np.float16])
def test_sort_argsort_nd(shape, axis, dtype):
    x = _data(int(np.prod(shape)), dtype, 7).reshape(shape)
    cx = cp.array(x)
    assert np.array_equal(cp.argsort(cx, axis=axis).get(), ref.argsort_stable(x, axis=axis))
    _value_equal(cp.sort(cx, axis=axis).get(), ref.sort(x, axis=axis))
    y = x.copy()
    cy = cp.array(y) + 0
    if axis is not None:
        cy.sort(axis=axis)
        y.sort(axis=axis, kind="stable")
        _value_equal(cy.get(), y)


@pytest.mark.parametrize("shape,dtype,lo,hi", [((300, 4096), np.int32, 0, 200),
                                                ((1000, 37), np.int64, -3, 3),
                                                ((64, 4096), np.uint16, 7, 7),
                                                ((17, 2049), np.int32, -(2 ** 31), 2 ** 31 - 1)])
def test_sort_tile_rows_uniform_digits(shape, dtype, lo, hi):
    """Rows of at most one tile, whose keys share most digit bytes (passes
    with one digit for the whole row are skipped) or are all equal: stable
    argsort, sort and kind='stable' equal NumPy's along the last axis."""
    rng = np.random.default_rng(shape[0])
    x = rng.integers(lo, hi, shape, dtype=np.int64, endpoint=True).astype(dtype)
    cx = cp.array(x)
    assert np.array_equal(cp.argsort(cx, axis=-1).get(), ref.argsort_stable(x, axis=-1))
    _value_equal(cp.sort(cx, axis=-1).get(), ref.sort(x, axis=-1))
    f = np.full(shape, 1.5, np.float32)
    assert np.array_equal(cp.argsort(cp.array(f), axis=-1).get(), ref.argsort_stable(f, axis=-1))


@pytest.mark.parametrize("length", [1, 2, 3, 15, 16, 17, 100, 257, 1000, 2048, 2049, 4096])
@pytest.mark.parametrize("dtype", [np.float32, np.int16, np.float64])
def test_sort_rows_packed_per_tile(length, dtype):
    """Whole rows packed into one 4096-key tile (min(256, 4096 // length)
    rows, the last tile partly filled): stable argsort and sort along the
    last axis equal NumPy's for every row length around the packing steps."""
    rows = 1000 + 7 * length % 13
    x = _data(rows * length, dtype, length).reshape(rows, length)
    cx = cp.array(x)
    assert np.array_equal(cp.argsort(cx, axis=-1).get(), ref.argsort_stable(x, axis=-1))
    _value_equal(cp.sort(cx, axis=-1).get(), ref.sort(x, axis=-1))
    got = cp.sort(cx, axis=-1, kind="stable").get()
    want = ref.sort(x, axis=-1, kind="stable")
    if got.dtype.kind == "f":
        got, want = got.view(f"u{got.itemsize}"), want.view(f"u{want.itemsize}")
    assert np.array_equal(got, want)


def test_sort_more_rows_than_workgroups():
    """(2^20 + 5) rows of 2, and 2^28 + 300 rows of 1 (2^20 + 2 tiles of 256
    rows: more tiles than the one-tile kernel's 2^20 workgroups, so the
    last two are taken grid-stride)."""
    x = np.random.default_rng(11).standard_normal(((1 << 20) + 5, 2)).astype(np.float32)
    cx = cp.array(x)
    assert np.array_equal(cp.argsort(cx, axis=-1).get(), ref.argsort_stable(x, axis=-1))
    _value_equal(cp.sort(cx, axis=-1).get(), ref.sort(x, axis=-1))
    y = np.random.default_rng(12).integers(-30000, 30000, ((1 << 28) + 300, 1), dtype=np.int16)
    got = cp.sort(cp.array(y), axis=-1).get()
    assert np.array_equal(got, y)  # rows of one key are already sorted


def test_sort_large_properties():
    """2^24 float32: the output is nondecreasing (NaN last), a permutation
    of the input (same multiset), and argsort reorders the input into it."""
    n = 1 << 24
    x = np.random.default_rng(8).standard_normal(n).astype(np.float32)
    x[::1000] = np.nan
    cx = cp.array(x)
    s = cp.sort(cx).get()
    want = np.sort(x)
    _value_equal(s, want)
    idx = cp.argsort(cx).get()
    assert np.array_equal(idx, np.argsort(x, kind="stable"))


@pytest.mark.parametrize("dtype", [np.float32, np.int32, np.float64, np.uint16])
def test_searchsorted(dtype):
    rng = np.random.default_rng(9)
    a = np.sort(_data(5001, dtype, 10))
    if np.dtype(dtype).kind == "f":
        v = np.concatenate([a[::7], np.array([np.nan, np.inf, -np.inf, -0.0, 0.0], dtype),
                            (rng.standard_normal(300) * 4).astype(dtype)])
    else:
        v = np.concatenate([a[::7], _data(300, dtype, 11)])
    ca = cp.array(a)
    for side in ("left", "right"):
        got = cp.searchsorted(ca, cp.array(v), side=side).get()
        assert got.dtype == np.int64
        assert np.array_equal(got, ref.searchsorted(a, v, side=side))
    # sorter, 2-D values, scalar, mixed dtypes
    perm = rng.permutation(a.size)
    un = a[perm]
    srt = np.argsort(un, kind="stable")
    assert np.array_equal(cp.searchsorted(cp.array(un), cp.array(v), sorter=cp.array(srt)).get(),
                          ref.searchsorted(un, v, sorter=srt))
    v2 = v[:300].reshape(20, 15)
    assert np.array_equal(cp.searchsorted(ca, cp.array(v2)).get(), ref.searchsorted(a, v2))
    assert int(cp.searchsorted(ca, a[10]).get()) == ref.searchsorted(a, a[10])
    assert np.array_equal(cp.searchsorted(ca, cp.array(v.astype(np.float64) + 0.5)).get(),
                          ref.searchsorted(a, v.astype(np.float64) + 0.5))


def test_take_and_errors():
    a = cp.array(np.arange(10, dtype=np.float32))
    with pytest.raises(IndexError):
        cp.searchsorted(a, cp.array(np.array([1.0], np.float32)),
                        sorter=cp.array(np.array([0, 1, 2, 3, 4, 5, 6, 7, 8, 10])))
    with pytest.raises(ValueError):
        cp.searchsorted(cp.array(np.zeros((2, 2))), 1.0)
    with pytest.raises(NotImplementedError):
        cp.sort(a, order="x")
