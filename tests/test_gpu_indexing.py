"""Advanced indexing and the indexing routines on the device, against
NumPy: integer and boolean array keys mixed with slices, integers, None and
Ellipsis (NumPy's adjacency rule for where the index dimensions go), on
contiguous arrays and on strided, offset and transposed views; assignment
through the same keys; take / put / nonzero / flatnonzero / argwhere /
compress / extract / putmask / place / take_along_axis / put_along_axis.
Bar: bit-exact (data movement only).  Duplicate indices in assignments
are avoided: which write lands is unspecified (as in NumPy)."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu


def _data(shape, dtype, seed=0):
    rng = np.random.default_rng(seed)
    if np.dtype(dtype) == np.bool_:
        return rng.random(shape) < 0.5
    return (rng.standard_normal(shape) * 100).astype(dtype)


def _same(got, want):
    got = got.get() if hasattr(got, "get") else np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    assert np.array_equal(got, want, equal_nan=want.dtype.kind == "f")


def _keys(rng):
    i5 = np.array([4, 0, -1, 2])
    i3 = np.array([[1, 0], [2, 2]])
    m7 = rng.random(7) < 0.5
    m57 = rng.random((5, 7)) < 0.4
    return [
        i5, [0, 3, 1], i3, np.array([], np.int64), np.int64(2) * np.ones(3, np.int64),
        m57, np.zeros((5, 7), bool), np.ones((5, 7), bool), m57[:, 0],
        (slice(None), [6, 0, 3]), (i5, slice(1, 6, 2)), (slice(1, 4), [0, 2]),
        (i5, 3), (2, slice(None), [0, 4]), (i5, [1, 2, 3, 4]),
        (i5[:, None], np.array([0, 6])), (i5, slice(None), np.array([1, 0, 4, 2])),
        (Ellipsis, [1, 4]), (None, i5), (i5, None), (slice(None), m7),
        (m57[:, 0], slice(2, 5)), (i5, Ellipsis, 0), (slice(None, None, -1), [1, 1]),
    ]


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.int64, np.bool_, np.uint16])
@pytest.mark.parametrize("layout", ["contig", "strided", "transposed"])
def test_getitem_keys(dtype, layout):
    rng = np.random.default_rng(1)
    base = _data((10, 14, 6), dtype)
    if layout == "contig":
        x = base[:5, :7, :5].copy()
        g = cp.array(x)
    elif layout == "strided":
        x = base[1:10:2, 3:10, 1:]                 # (5, 7, 5) view with offset
        g = cp.array(base)[1:10:2, 3:10, 1:]
    else:
        x = base[:7, :5, 2].T.copy()[:, :, None].repeat(5, 2)
        g = cp.array(x.transpose(1, 0, 2).copy()).transpose(1, 0, 2)
    for key in _keys(rng):
        want = x[key]
        got = g[tuple(cp.array(k) if isinstance(k, np.ndarray) else k for k in key)
                if isinstance(key, tuple) else (cp.array(key) if isinstance(key, np.ndarray) else key)]
        _same(got, want)


@pytest.mark.parametrize("dtype", [np.float32, np.int16, np.float64])
def test_setitem_keys(dtype):
    rng = np.random.default_rng(2)
    keys = [np.array([4, 0, 2]), [1, 3], rng.random((5, 7)) < 0.4, (slice(None), [6, 0, 3]),
            (np.array([0, 3]), slice(1, 6, 2)), (2, slice(None), [0, 2]),
            (np.array([1, 4]), slice(None), np.array([1, 0])), (Ellipsis, [1, 2]),
            (np.array([[0], [2]]), np.array([1, 5]))]
    for key in keys:
        x = _data((5, 7, 3), dtype, 3)
        want_shape = x[key].shape
        for value in (7, _data(want_shape, dtype, 4), _data(want_shape[-1:], dtype, 5)):
            y = x.copy()
            y[key] = value
            g = cp.array(x)
            g[key] = cp.array(value) if isinstance(value, np.ndarray) else value
            _same(g, y)
    # through a strided view of a larger array
    big = _data((12, 9), dtype, 6)
    yb = big.copy()
    yb[2:12:3, 1:8][np.array([0, 2, 3]), 4] = 99
    gb = cp.array(big)
    view = gb[2:12:3, 1:8]
    view[np.array([0, 2, 3]), 4] = 99
    _same(gb, yb)
    # boolean mask assignment with a scalar and with the selected count of values
    x = _data((64, 33), dtype, 7)
    m = x > 0
    y = x.copy()
    y[m] = 0
    g = cp.array(x)
    g[g > 0] = 0
    _same(g, y)
    y2 = x.copy()
    vals = _data((int(m.sum()),), dtype, 8)
    y2[m] = vals
    g2 = cp.array(x)
    g2[cp.array(m)] = cp.array(vals)
    _same(g2, y2)


def test_large_gathers_and_rows():
    """2-D row gathers (16-byte words), a 2^22-element mask and a 2^20
    index gather."""
    rng = np.random.default_rng(9)
    a = rng.standard_normal((4096, 256)).astype(np.float32)
    idx = rng.integers(-4096, 4096, 5000)
    _same(cp.array(a)[cp.array(idx)], a[idx])
    v = rng.standard_normal(1 << 22).astype(np.float32)
    _same(cp.array(v)[cp.array(v) > 0.5], v[v > 0.5])
    j = rng.integers(0, 1 << 22, 1 << 20)
    _same(cp.array(v)[cp.array(j)], v[j])
    h = rng.standard_normal((3000, 7)).astype(np.float16)     # 14-byte rows: 2-byte words
    _same(cp.array(h)[cp.array(idx[:100] % 3000)], h[idx[:100] % 3000])


def test_index_errors():
    g = cp.array(np.arange(20, dtype=np.float32).reshape(4, 5))
    with pytest.raises(IndexError):
        g[cp.array(np.array([0, 4]))]
    with pytest.raises(IndexError):
        g[np.array([-5])]
    with pytest.raises(IndexError):
        g[:, [5]]
    with pytest.raises(IndexError):
        g[np.ones(5, bool)]
    with pytest.raises(IndexError):
        g[np.array([0.5])]
    with pytest.raises(ValueError):
        g[[0, 1]] = np.ones((3, 5), np.float32)


def test_routines():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((6, 8)).astype(np.float32)
    x[x < -0.5] = 0
    g = cp.array(x)
    for gi, wi in zip(cp.nonzero(g), np.nonzero(x)):
        _same(gi, wi)
    for gi, wi in zip(g.nonzero(), x.nonzero()):
        _same(gi, wi)
    _same(cp.flatnonzero(g), np.flatnonzero(x))
    _same(cp.argwhere(g), np.argwhere(x))
    _same(cp.nonzero(cp.array(np.zeros(5, np.int32)))[0], np.nonzero(np.zeros(5, np.int32))[0])
    idx = np.array([3, -1, 0, 7, 2])
    _same(cp.take(g, cp.array(idx)), np.take(x, idx))
    _same(cp.take(g, idx, axis=1), np.take(x, idx, axis=1))
    _same(cp.take(g, [[1, 2], [0, 5]], axis=0), np.take(x, [[1, 2], [0, 5]], axis=0))
    _same(cp.take(g, np.array([9, -20, 4]), axis=1, mode="clip"),
          np.take(x, np.array([9, -20, 4]), axis=1, mode="clip"))
    _same(cp.take(g, np.array([9, -20, 4]), axis=0, mode="wrap"),
          np.take(x, np.array([9, -20, 4]), axis=0, mode="wrap"))
    _same(g.take(idx), x.take(idx))
    with pytest.raises(IndexError):
        cp.take(g, [100])
    y = x.copy()
    np.put(y, [0, 13, -1], [1.5, 2.5, 3.5])
    gy = cp.array(x)
    cp.put(gy, [0, 13, -1], [1.5, 2.5, 3.5])
    _same(gy, y)
    y = x.copy()
    np.put(y, [1, 2, 3, 4], [7.0, 8.0])                 # values repeat
    gy = cp.array(x)
    gy.put([1, 2, 3, 4], [7.0, 8.0])
    _same(gy, y)
    c = np.array([True, False, True, True])
    _same(cp.compress(c, g, axis=0), np.compress(c, x, axis=0))
    _same(cp.compress(c, g, axis=1), np.compress(c, x, axis=1))
    _same(cp.compress(c, g), np.compress(c, x))
    _same(cp.extract(g > 0, g), np.extract(x > 0, x))
    y = x.copy()
    np.putmask(y, y > 0, np.array([10.0, 20.0, 30.0], np.float32))
    gy = cp.array(x)
    cp.putmask(gy, gy > 0, cp.array(np.array([10.0, 20.0, 30.0], np.float32)))
    _same(gy, y)
    y = x.copy()
    np.place(y, y > 0, [-1.0, -2.0])
    gy = cp.array(x)
    cp.place(gy, gy > 0, [-1.0, -2.0])
    _same(gy, y)
    ai = np.argsort(x, axis=1)
    _same(cp.take_along_axis(g, cp.array(ai), axis=1), np.take_along_axis(x, ai, axis=1))
    ai0 = np.argsort(x, axis=0)[:2]
    _same(cp.take_along_axis(g, cp.array(ai0), axis=0), np.take_along_axis(x, ai0, axis=0))
    y = x.copy()
    first = np.argmax(x, axis=1)[:, None]
    np.put_along_axis(y, first, -7.0, axis=1)
    gy = cp.array(x)
    cp.put_along_axis(gy, cp.array(first), -7.0, axis=1)
    _same(gy, y)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.float16, np.int16, np.int64, np.bool_])
@pytest.mark.parametrize("n", [1, 4095, 4096, 4097, (1 << 20) + 3])
def test_full_shape_mask_compaction(dt, n):
    """a[mask] for a mask of a's shape packs the selected elements on the
    device straight from the mask (tiles of 4096: counts, their scan, then
    each tile writes from its offset); nonzero / flatnonzero use the same
    tile counts.  Tile boundaries, every density, views and element sizes
    against NumPy bit for bit."""
    rng = np.random.default_rng(44000 + n)
    x = (rng.standard_normal(n) * 50).astype(dt) if dt != np.bool_ else rng.random(n) < 0.5
    gx = cp.array(x)
    for density in (0.0, 0.01, 0.5, 1.0):
        m = rng.random(n) < density
        gm = cp.array(m)
        got = gx[gm].get()
        assert got.dtype == x.dtype and np.array_equal(got.view(np.uint8), x[m].view(np.uint8))
        assert np.array_equal(cp.flatnonzero(gm).get(), np.flatnonzero(m))
    # 2-D, a mask view one element into its buffer (unaligned) and a transposed source
    if n >= 4096:
        r = 64
        c = n // r
        x2 = x[: r * c].reshape(r, c)
        mb = rng.random(r * c + 1) < 0.3
        gm2 = cp.array(mb)[1:].reshape(r, c)
        want = x2[mb[1:].reshape(r, c)]
        got = cp.array(x2)[gm2].get()
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
        mt = rng.random((c, r)) < 0.3
        got = cp.array(x2).T[cp.array(mt)].get()
        assert np.array_equal(got.view(np.uint8), x2.T[mt].view(np.uint8))


def test_full_shape_mask_empty():
    a = cp.zeros((0, 3), dtype=np.float32)
    assert cp.zeros((0, 3), dtype=np.float32)[a > 0].get().shape == (0,)
