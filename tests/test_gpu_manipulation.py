"""Array manipulation routines and order statistics on the device against
NumPy, bit-exact with NumPy's dtypes (data movement; NumPy's interpolation
arithmetic for quantiles): concatenate / stack family, splits, tile,
repeat, flips, roll, broadcasts, axis moves, diagonal / diag / trace,
tril / triu, diff, outer, meshgrid, cross, kron, tensordot, average,
unique; median / quantile / percentile and their NaN-aware forms over
dtypes, q forms (Python scalar, list), methods, axes and NaN content."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu


def _same(got, want):
    if isinstance(want, (tuple, list)):
        assert len(got) == len(want)
        for g, w in zip(got, want):
            _same(g, w)
        return
    got = got.get() if hasattr(got, "get") else np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    if want.dtype.kind == "f":
        assert np.array_equal(got, want, equal_nan=True)
        assert np.array_equal(np.signbit(got), np.signbit(want))
    else:
        assert np.array_equal(got, want)


def _x(shape, dtype=np.float32, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * 10).astype(dtype)


def test_joining_and_splitting():
    a, b = _x((3, 4)), _x((2, 4), seed=1)
    c = _x((3, 5), np.int32, 2)
    _same(cp.concatenate([cp.array(a), cp.array(b)]), np.concatenate([a, b]))
    _same(cp.concatenate([cp.array(a), cp.array(c)], axis=1), np.concatenate([a, c], axis=1))
    _same(cp.concatenate([cp.array(a), cp.array(b)], axis=None), np.concatenate([a, b], axis=None))
    _same(cp.stack([cp.array(a), cp.array(a * 2)], axis=1), np.stack([a, a * 2], axis=1))
    _same(cp.vstack([cp.array(a), cp.array(b)]), np.vstack([a, b]))
    _same(cp.hstack([cp.array(a), cp.array(c)]), np.hstack([a, c]))
    _same(cp.dstack([cp.array(a), cp.array(a)]), np.dstack([a, a]))
    _same(cp.column_stack([cp.array(a[:, 0]), cp.array(a)]), np.column_stack([a[:, 0], a]))
    _same(cp.append(cp.array(a), cp.array(b), axis=0), np.append(a, b, axis=0))
    _same(cp.append(cp.array(a), cp.array(b)), np.append(a, b))
    x = _x((10, 6))
    _same(cp.split(cp.array(x), 5), np.split(x, 5))
    _same(cp.array_split(cp.array(x), 3, axis=1), np.array_split(x, 3, axis=1))
    _same(cp.split(cp.array(x), [2, 7]), np.split(x, [2, 7]))
    _same(cp.hsplit(cp.array(x), 2), np.hsplit(x, 2))
    _same(cp.vsplit(cp.array(x), [3]), np.vsplit(x, [3]))
    _same(cp.unstack(cp.array(x), axis=1), np.unstack(x, axis=1))
    with pytest.raises(ValueError):
        cp.split(cp.array(x), 3)
    with pytest.raises(ValueError):
        cp.concatenate([cp.array(a), cp.array(c)])


def test_tile_repeat_flip_roll():
    a = _x((3, 4), np.int16)
    for reps in (2, (2, 3), (2, 1, 2), (0, 2)):
        _same(cp.tile(cp.array(a), reps), np.tile(a, reps))
    _same(cp.repeat(cp.array(a), 3), np.repeat(a, 3))
    _same(cp.repeat(cp.array(a), 2, axis=1), np.repeat(a, 2, axis=1))
    r = np.array([1, 0, 3])
    _same(cp.repeat(cp.array(a), cp.array(r), axis=0), np.repeat(a, r, axis=0))
    _same(cp.repeat(cp.array(a), [2, 0, 1, 1], axis=1), np.repeat(a, [2, 0, 1, 1], axis=1))
    for ax in (None, 0, 1, (0, 1)):
        _same(cp.flip(cp.array(a), ax), np.flip(a, ax))
    _same(cp.fliplr(cp.array(a)), np.fliplr(a))
    _same(cp.flipud(cp.array(a)), np.flipud(a))
    for k in (1, 2, 3, -1):
        _same(cp.rot90(cp.array(a), k), np.rot90(a, k))
    for sh, ax in ((2, None), (-1, 0), (5, 1), ((1, -2), (0, 1)), (3, (1, 1))):
        _same(cp.roll(cp.array(a), sh, ax), np.roll(a, sh, ax))


def test_views_and_axes():
    a = _x((2, 3, 4))
    g = cp.array(a)
    _same(cp.broadcast_to(cp.array(a[0, 0]), (5, 4)), np.broadcast_to(a[0, 0], (5, 4)))
    _same(cp.broadcast_arrays(cp.array(a[:, :1]), cp.array(a[0])), np.broadcast_arrays(a[:, :1], a[0]))
    _same(cp.moveaxis(g, 0, -1), np.moveaxis(a, 0, -1))
    _same(cp.moveaxis(g, [0, 1], [2, 0]), np.moveaxis(a, [0, 1], [2, 0]))
    _same(cp.rollaxis(g, 2), np.rollaxis(a, 2))
    _same(cp.swapaxes(g, 0, 2), np.swapaxes(a, 0, 2))
    _same(cp.expand_dims(g, (0, 3)), np.expand_dims(a, (0, 3)))
    _same(cp.squeeze(cp.array(a[:1, :, :1])), np.squeeze(a[:1, :, :1]))
    _same(cp.atleast_3d(cp.array(a[0, 0])), np.atleast_3d(a[0, 0]))
    _same(cp.atleast_2d(cp.array(np.float32(3))), np.atleast_2d(np.float32(3)))
    _same(cp.matrix_transpose(g), np.matrix_transpose(a))
    m = _x((5, 7))
    for off in (0, 2, -3, 9):
        _same(cp.diagonal(cp.array(m), off), np.diagonal(m, off))
    _same(cp.diagonal(g, 1, 1, 2), np.diagonal(a, 1, 1, 2))
    _same(cp.diag(cp.array(m), -1), np.diag(m, -1))
    _same(cp.diag(cp.array(m[0]), 2), np.diag(m[0], 2))
    np.testing.assert_allclose(cp.trace(cp.array(m)).get(), np.trace(m.astype(np.float64)), rtol=1e-6)
    for k in (-1, 0, 2):
        _same(cp.tril(cp.array(m), k), np.tril(m, k))
        _same(cp.triu(cp.array(m), k), np.triu(m, k))
    _same(cp.tril(g), np.tril(a))
    # writes through a broadcast / diagonal view reach the base
    z = np.zeros((4, 4), np.float32)
    gz = cp.array(z) + 0
    cp.diagonal(gz)[...] = 7
    np.fill_diagonal(z, 7)
    _same(gz, z)


@pytest.mark.filterwarnings("ignore:Arrays of 2-dimensional vectors are deprecated")
def test_small_arithmetic():
    a = _x((6, 5))
    g = cp.array(a)
    _same(cp.ptp(g, axis=0), np.ptp(a, axis=0))
    _same(cp.diff(g), np.diff(a))
    _same(cp.diff(g, n=2, axis=0), np.diff(a, n=2, axis=0))
    _same(cp.diff(g, prepend=0, append=1), np.diff(a, prepend=0, append=1))
    bb = a > 0
    _same(cp.diff(cp.array(bb)), np.diff(bb))
    _same(cp.outer(cp.array(a[0]), cp.array(a[1])), np.outer(a[0], a[1]))
    for ind in ("xy", "ij"):
        _same(cp.meshgrid(cp.array(a[0]), cp.array(a[:, 0]), indexing=ind),
              np.meshgrid(a[0], a[:, 0], indexing=ind))
        _same(cp.meshgrid(cp.array(a[0]), cp.array(a[:, 0]), cp.array(a[1, :3]), indexing=ind,
                          sparse=True),
              np.meshgrid(a[0], a[:, 0], a[1, :3], indexing=ind, sparse=True))
    v3, w3 = _x((4, 3)), _x((4, 3), seed=5)
    _same(cp.cross(cp.array(v3), cp.array(w3)), np.cross(v3, w3))
    _same(cp.cross(cp.array(v3[:, :2]), cp.array(w3[:, :2])), np.cross(v3[:, :2], w3[:, :2]))
    k1, k2 = _x((2, 3), np.int32), _x((3, 2), np.int32, 3)
    _same(cp.kron(cp.array(k1), cp.array(k2)), np.kron(k1, k2))
    t1, t2 = _x((3, 4, 5)), _x((4, 5, 2), seed=4)
    np.testing.assert_allclose(cp.tensordot(cp.array(t1), cp.array(t2)).get(),
                               np.tensordot(t1.astype(np.float64), t2.astype(np.float64)),
                               rtol=1e-4, atol=1e-3)
    np.testing.assert_allclose(cp.tensordot(cp.array(t1), cp.array(t2), axes=([1], [0])).get(),
                               np.tensordot(t1.astype(np.float64), t2.astype(np.float64),
                                            axes=([1], [0])), rtol=1e-4, atol=1e-3)
    w = np.abs(_x((5,), seed=6)) + 1
    np.testing.assert_allclose(cp.average(g, axis=1, weights=cp.array(w)).get(),
                               np.average(a, axis=1, weights=w), rtol=1e-6)
    np.testing.assert_allclose(cp.average(g).get(), np.average(a), rtol=1e-6)


def test_unique():
    rng = np.random.default_rng(7)
    x = rng.integers(0, 20, (30, 7)).astype(np.int32)
    _same(cp.unique(cp.array(x)), np.unique(x))
    got = cp.unique(cp.array(x), return_index=True, return_inverse=True, return_counts=True)
    want = np.unique(x, return_index=True, return_inverse=True, return_counts=True)
    _same(got, want)
    f = rng.standard_normal(500).astype(np.float32).round(1)
    f[::50] = np.nan
    f[1::37] = -0.0
    _same(cp.unique(cp.array(f)), np.unique(f))
    _same(cp.unique(cp.array(np.array([], np.float32))), np.unique(np.array([], np.float32)))


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.float16, np.int32, np.int64])
def test_order_statistics(dtype):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((9, 40)) * 5).astype(dtype)
    g = cp.array(x)
    for axis in (None, 0, 1, -1):
        _same(cp.median(g, axis=axis), np.median(x, axis=axis))
        for q in (0.0, 0.3, 0.5, 1.0, [0.25, 0.75], [0.0, 0.1, 1.0]):
            for method in ("linear", "lower", "higher", "nearest", "midpoint"):
                _same(cp.quantile(g, q, axis=axis, method=method),
                      np.quantile(x, q, axis=axis, method=method))
        _same(cp.percentile(g, 37.5, axis=axis), np.percentile(x, 37.5, axis=axis))
        _same(cp.percentile(g, [10, 90], axis=axis, keepdims=True),
              np.percentile(x, [10, 90], axis=axis, keepdims=True))
    _same(cp.median(cp.array(x[:, :39]), axis=1), np.median(x[:, :39], axis=1))
    _same(cp.median(g, axis=(0, 1)), np.median(x, axis=(0, 1)))
    if np.dtype(dtype).kind == "f":
        xn = x.copy()
        xn[2, ::3] = np.nan
        xn[5, :] = np.nan
        xn[7, 1] = np.nan
        gn = cp.array(xn)
        with np.errstate(all="ignore"):
            import warnings
            with warnings.catch_warnings():
                warnings.simplefilter("ignore")
                _same(cp.median(gn, axis=1), np.median(xn, axis=1))
                _same(cp.nanmedian(gn, axis=1), np.nanmedian(xn, axis=1))
                _same(cp.nanmedian(gn), np.nanmedian(xn))
                for q in (0.3, [0.5, 0.9]):
                    for method in ("linear", "lower", "midpoint", "nearest"):
                        _same(cp.nanquantile(gn, q, axis=1, method=method),
                              np.nanquantile(xn, q, axis=1, method=method))
                _same(cp.nanpercentile(gn, 80, axis=0), np.nanpercentile(xn, 80, axis=0))
    with pytest.raises(ValueError):
        cp.quantile(g, 1.5)
