"""Comparison, rounding, set, binning, selection, sorting-variant, pair
statistics, calculus and index-helper routines on the device against NumPy:
bit-exact where NumPy's arithmetic is elementwise or integer; summations
(cov, trapezoid, float correlate, weighted bincount / histogram) within
the tolerance written at each check, since their order differs from
NumPy's BLAS / sequential loops."""
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
        assert np.array_equal(got, want, equal_nan=True), (got, want)
        assert np.array_equal(np.signbit(got), np.signbit(want))
    else:
        assert np.array_equal(got, want), (got, want)


def _close(got, want, rtol, atol=0.0):
    got = got.get() if hasattr(got, "get") else np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol)


def _h(a):
    return a.get() if hasattr(a, "get") else np.asarray(a)


def _x(shape, dtype=np.float32, seed=0, scale=10):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(shape) * scale).astype(dtype)


def test_isclose_allclose_equal():
    a = _x((1000,))
    b = a + _x((1000,), seed=1, scale=1e-4)
    b[:5] = [np.nan, np.inf, -np.inf, 0.0, a[4]]
    a[:5] = [np.nan, np.inf, np.inf, 1e-9, a[4]]
    for eqn in (False, True):
        _same(cp.isclose(cp.array(a), cp.array(b), equal_nan=eqn), np.isclose(a, b, equal_nan=eqn))
        _same(cp.isclose(cp.array(a), cp.array(b), rtol=1e-3, atol=1e-2, equal_nan=eqn),
              np.isclose(a, b, rtol=1e-3, atol=1e-2, equal_nan=eqn))
    d = a.astype(np.float64)
    _same(cp.isclose(cp.array(d), cp.array(d * (1 + 1e-9))), np.isclose(d, d * (1 + 1e-9)))
    assert cp.allclose(cp.array(a[5:]), cp.array(b[5:]), atol=1e-3) == np.allclose(a[5:], b[5:], atol=1e-3)
    assert cp.allclose(cp.array(a[5:]), cp.array(b[5:])) == np.allclose(a[5:], b[5:])
    i = np.arange(12, dtype=np.int32).reshape(3, 4)
    assert cp.array_equal(cp.array(i), cp.array(i.copy()))
    assert not cp.array_equal(cp.array(i), cp.array(i[:, :3]))
    assert not cp.array_equal(cp.array(a), cp.array(a))          # NaN != NaN
    assert cp.array_equal(cp.array(a), cp.array(a), equal_nan=True)
    assert cp.array_equiv(cp.array(i), cp.array(i[1:2] * 0 + i[0:1])) == np.array_equiv(i, i[0:1])
    assert cp.array_equiv(cp.array(np.ones((3, 4))), cp.array(np.ones(4)))
    assert not cp.array_equiv(cp.array(np.ones((3, 4))), cp.array(np.ones(3)))


def test_round_fix_nan_to_num_sinc():
    a = _x((4096,), scale=1000)
    a[:6] = [0.5, 1.5, 2.5, -0.5, -2.5, 1.005]
    for dt in (np.float32, np.float64, np.float16):
        x = a.astype(dt)
        for d in (0, 1, 2, 3, -1, -2):
            _same(cp.round(cp.array(x), d), np.round(x, d))
        _same(cp.around(cp.array(x), 2), np.around(x, 2))
        _same(cp.fix(cp.array(x)), np.fix(x))
    i = np.array([1234, 1250, -1250, -1251, 7, 0], dtype=np.int64)
    for d in (0, 2, -1, -2, -3):
        _same(cp.round(cp.array(i), d), np.round(i, d))
    _same(cp.fix(cp.array(i.astype(np.int32))), np.fix(i.astype(np.int32)))
    z = np.array([np.nan, np.inf, -np.inf, 1.5, -0.0], dtype=np.float32)
    _same(cp.nan_to_num(cp.array(z)), np.nan_to_num(z))
    _same(cp.nan_to_num(cp.array(z), nan=-1.0, posinf=9.0, neginf=-9.0),
          np.nan_to_num(z, nan=-1.0, posinf=9.0, neginf=-9.0))
    _same(cp.nan_to_num(cp.array(z.astype(np.float64))), np.nan_to_num(z.astype(np.float64)))
    _same(cp.nan_to_num(cp.array(i)), np.nan_to_num(i))
    s = np.linspace(-4, 4, 101).astype(np.float64)
    _close(cp.sinc(cp.array(s)), np.sinc(s), rtol=1e-14, atol=1e-16)
    _close(cp.sinc(cp.array(s.astype(np.float32))), np.sinc(s.astype(np.float32)), rtol=1e-6, atol=1e-7)
    _same(cp.angle(cp.array(z[3:])), np.angle(z[3:]))
    _same(cp.real(cp.array(z)), np.real(z))
    _same(cp.imag(cp.array(z)), np.imag(z))
    _same(cp.isreal(cp.array(z)), np.isreal(z))
    _same(cp.iscomplex(cp.array(z)), np.iscomplex(z))


def test_set_operations():
    rng = np.random.default_rng(3)
    for dt in (np.int32, np.int64, np.float32, np.uint16):
        a = rng.integers(0, 50, 300).astype(dt)
        b = rng.integers(20, 90, 200).astype(dt)
        _same(cp.isin(cp.array(a), cp.array(b)), np.isin(a, b))
        _same(cp.isin(cp.array(a), cp.array(b), invert=True), np.isin(a, b, invert=True))
        _same(cp.isin(cp.array(a.reshape(15, 20)), cp.array(b)), np.isin(a.reshape(15, 20), b))
        _same(cp.in1d(cp.array(a), cp.array(b)), np.isin(a.ravel(), b))
        _same(cp.intersect1d(cp.array(a), cp.array(b)), np.intersect1d(a, b))
        _same(cp.union1d(cp.array(a), cp.array(b)), np.union1d(a, b))
        _same(cp.setdiff1d(cp.array(a), cp.array(b)), np.setdiff1d(a, b))
        _same(cp.setxor1d(cp.array(a), cp.array(b)), np.setxor1d(a, b))
    f = np.array([1.0, np.nan, 2.0, 3.0], dtype=np.float32)
    _same(cp.isin(cp.array(f), cp.array(np.array([2.0, np.nan], np.float32))),
          np.isin(f, np.array([2.0, np.nan], np.float32)))
    _same(cp.isin(cp.array(f), cp.array(np.array([], np.float32))),
          np.isin(f, np.array([], np.float32)))
    e = np.array([], dtype=np.int32)
    _same(cp.setxor1d(cp.array(e), cp.array(e)), np.setxor1d(e, e))
    _same(cp.intersect1d(cp.array(e), cp.array(np.array([1], np.int32))),
          np.intersect1d(e, np.array([1], np.int32)))


def test_bincount_digitize_histogram():
    rng = np.random.default_rng(4)
    x = rng.integers(0, 40, 5000).astype(np.int32)
    _same(cp.bincount(cp.array(x)), np.bincount(x))
    _same(cp.bincount(cp.array(x), minlength=64), np.bincount(x, minlength=64))
    _same(cp.bincount(cp.array(np.array([3, 3, 0], np.int64))), np.bincount(np.array([3, 3, 0])))
    w = rng.standard_normal(5000)
    # float64 prefix-sum differences: error below 1e-13 of the total |w|
    _close(cp.bincount(cp.array(x), weights=cp.array(w)), np.bincount(x, weights=w),
           rtol=0, atol=1e-13 * np.abs(w).sum())
    with pytest.raises(ValueError):
        cp.bincount(cp.array(np.array([1, -1], np.int32)))
    for dt in (np.int16, np.uint16, np.uint32, np.int64, np.bool_):
        xs = (x % 2).astype(dt) if dt == np.bool_ else x.astype(dt)
        _same(cp.bincount(cp.array(xs)), np.bincount(xs))
    big = np.random.default_rng(5).integers(0, 20000, 50000).astype(np.int32)   # global-atomic path
    _same(cp.bincount(cp.array(big)), np.bincount(big))
    _same(cp.bincount(cp.array(big), minlength=30000), np.bincount(big, minlength=30000))
    _same(cp.bincount(cp.array(np.array([1, 2, 2], np.uint64))), np.bincount(np.array([1, 2, 2], np.uint64)))
    with pytest.raises(ValueError):
        cp.bincount(cp.array(np.array([2 ** 63 + 5], np.uint64)))
    v = rng.standard_normal(3000).astype(np.float32) * 3
    bins = np.array([-2.0, -1.0, 0.0, 0.5, 1.0, 3.0], dtype=np.float32)
    for right in (False, True):
        _same(cp.digitize(cp.array(v), cp.array(bins), right=right), np.digitize(v, bins, right=right))
        _same(cp.digitize(cp.array(v), cp.array(bins[::-1].copy()), right=right),
              np.digitize(v, bins[::-1], right=right))
    v[:4] = [bins[0], bins[-1], bins[2], np.nan]
    for kw in ({}, {"bins": 7}, {"bins": 20, "range": (-1.0, 2.0)}, {"bins": bins}):
        kb = dict(kw)
        want = np.histogram(v[~np.isnan(v)], **kb)
        kb2 = dict(kw)
        if "bins" in kb2 and isinstance(kb2["bins"], np.ndarray):
            kb2["bins"] = cp.array(kb2["bins"])
        got = cp.histogram(cp.array(v[~np.isnan(v)]), **kb2)
        _same(got[0], want[0])
        _same(got[1], want[1])
    vv = v[~np.isnan(v)]
    d_got = cp.histogram(cp.array(vv), bins=9, density=True)
    d_want = np.histogram(vv, bins=9, density=True)
    _close(d_got[0], d_want[0], rtol=1e-14)
    hw = rng.standard_normal(vv.size).astype(np.float32)
    got = cp.histogram(cp.array(vv), bins=8, weights=cp.array(hw))
    want = np.histogram(vv, bins=8, weights=hw)
    _close(got[0], want[0], rtol=0, atol=1e-5 * np.abs(hw).sum())
    iw = rng.integers(0, 5, vv.size).astype(np.int32)
    _same(cp.histogram(cp.array(vv), bins=8, weights=cp.array(iw))[0],
          np.histogram(vv, bins=8, weights=iw)[0])
    _same(cp.histogram(cp.array(x), bins=10)[0], np.histogram(x, bins=10)[0])
    for dt in (np.float16, np.float64, np.int16, np.uint32):
        vd = (vv * 10).astype(dt)
        for kb in (5, 64, np.array([-20.0, -3.5, 0.0, 0.0, 2.0, 7.0, 20.0])):
            _same(cp.histogram(cp.array(vd), bins=kb)[0], np.histogram(vd, bins=kb)[0])
    many = np.linspace(-3, 3, 6001)                                   # global-atomic path
    _same(cp.histogram(cp.array(vv), bins=cp.array(many))[0], np.histogram(vv, bins=many)[0])
    _same(cp.histogram(cp.array(vv), bins=5000)[0], np.histogram(vv, bins=5000)[0])
    _same(cp.histogram(cp.array(np.array([], np.float32)), bins=4)[0],
          np.histogram(np.array([], np.float32), bins=4)[0])
    _same(cp.histogram(cp.array(x), bins=10)[1], np.histogram(x, bins=10)[1])


def test_interp():
    xp = np.sort(_x((50,), np.float64, 5))
    fp = _x((50,), np.float64, 6)
    x = _x((2000,), np.float64, 7, scale=15)
    x[:6] = [xp[0], xp[-1], xp[10], np.nan, -1e9, 1e9]
    _same(cp.interp(cp.array(x), cp.array(xp), cp.array(fp)), np.interp(x, xp, fp))
    _same(cp.interp(cp.array(x), cp.array(xp), cp.array(fp), left=-7.0, right=7.5),
          np.interp(x, xp, fp, left=-7.0, right=7.5))
    _same(cp.interp(cp.array(x.astype(np.float32)), cp.array(xp), cp.array(fp.astype(np.float32))),
          np.interp(x.astype(np.float32), xp, fp.astype(np.float32)))
    _same(cp.interp(cp.array(x), cp.array(xp[:1]), cp.array(fp[:1])), np.interp(x, xp[:1], fp[:1]))
    xd = np.array([0.0, 1.0, 1.0, 2.0])
    fd = np.array([0.0, 1.0, 5.0, 6.0])
    q = np.array([0.5, 1.0, 1.5, 2.0])
    _same(cp.interp(cp.array(q), cp.array(xd), cp.array(fd)), np.interp(q, xd, fd))


def test_lexsort_partition():
    rng = np.random.default_rng(8)
    k1 = rng.integers(0, 5, 1000).astype(np.int32)
    k2 = rng.standard_normal(1000).astype(np.float32)
    k3 = rng.integers(0, 3, 1000).astype(np.int64)
    _same(cp.lexsort((cp.array(k2), cp.array(k1))), np.lexsort((k2, k1)))
    _same(cp.lexsort([cp.array(k2), cp.array(k1), cp.array(k3)]), np.lexsort([k2, k1, k3]))
    a = _x((40, 33), seed=9)
    for kth in (0, 5, 32, -1):
        p = _h(cp.partition(cp.array(a), kth))
        s = np.sort(a, axis=-1)
        assert np.array_equal(p[:, kth], s[:, kth])
        assert np.all(p[:, :kth % 33] <= p[:, kth % 33][:, None])
        assert np.all(p[:, kth % 33 + 1:] >= p[:, kth % 33][:, None])
        ap = _h(cp.argpartition(cp.array(a), kth))
        assert np.array_equal(np.take_along_axis(a, ap, axis=-1)[:, kth], s[:, kth])
    p0 = _h(cp.partition(cp.array(a), 3, axis=0))
    assert np.array_equal(p0[3], np.sort(a, axis=0)[3])
    with pytest.raises(ValueError):
        cp.partition(cp.array(a), 33)


def test_cov_corrcoef():
    m = _x((5, 300), np.float64, 10)
    for kw in ({}, {"bias": True}, {"ddof": 3}, {"rowvar": False}):
        src = m if kw.get("rowvar", True) else m.T.copy()
        _close(cp.cov(cp.array(src), **kw), np.cov(src, **kw), rtol=1e-12, atol=1e-12)
    _close(cp.cov(cp.array(m[0]), cp.array(m[1])), np.cov(m[0], m[1]), rtol=1e-12, atol=1e-12)
    _close(cp.cov(cp.array(m[0])), np.cov(m[0]), rtol=1e-12)
    f = m.astype(np.float32)
    _close(cp.cov(cp.array(f)), np.cov(f), rtol=1e-5, atol=1e-4)
    _close(cp.corrcoef(cp.array(m)), np.corrcoef(m), rtol=1e-12, atol=1e-13)
    _close(cp.corrcoef(cp.array(m[0]), cp.array(m[2])), np.corrcoef(m[0], m[2]), rtol=1e-12, atol=1e-13)


def test_select_choose_piecewise():
    x = _x((500,), seed=11)
    c1, c2 = x < -3, x > 4
    _same(cp.select([cp.array(c1), cp.array(c2)], [cp.array(x * 2), cp.array(x - 1)]),
          np.select([c1, c2], [x * 2, x - 1]))
    _same(cp.select([cp.array(c1), cp.array(c2)], [cp.array(x * 2), cp.array(x - 1)], default=-5.5),
          np.select([c1, c2], [x * 2, x - 1], default=-5.5))
    i32 = np.arange(500, dtype=np.int32)
    _same(cp.select([cp.array(c1)], [cp.array(i32)]), np.select([c1], [i32]))
    idx = (np.arange(500) % 3).astype(np.int64)
    ch = [x, x * 10, -x]
    _same(cp.choose(cp.array(idx), [cp.array(c) for c in ch]), np.choose(idx, ch))
    _same(cp.choose(cp.array(idx + 2), [cp.array(c) for c in ch], mode="wrap"),
          np.choose(idx + 2, ch, mode="wrap"))
    _same(cp.choose(cp.array(idx + 1), [cp.array(c) for c in ch], mode="clip"),
          np.choose(idx + 1, ch, mode="clip"))
    with pytest.raises(ValueError):
        cp.choose(cp.array(idx + 1), [cp.array(c) for c in ch])
    _same(cp.piecewise(cp.array(x), [cp.array(c1), cp.array(c2)], [lambda v: v * 3, 7.0, lambda v: -v]),
          np.piecewise(x, [c1, c2], [lambda v: v * 3, 7.0, lambda v: -v]))


def test_gradient_trapezoid():
    y = _x((30, 40), np.float64, 12)
    _same(cp.gradient(cp.array(y)), np.gradient(y))
    _same(cp.gradient(cp.array(y), 0.5, axis=1), np.gradient(y, 0.5, axis=1))
    _same(cp.gradient(cp.array(y[0].astype(np.float32)), 2.0), np.gradient(y[0].astype(np.float32), 2.0))
    _same(cp.gradient(cp.array(np.arange(10, dtype=np.int32) ** 2)),
          np.gradient(np.arange(10, dtype=np.int32) ** 2))
    xs = np.sort(_x((40,), np.float64, 13))
    _close(cp.trapezoid(cp.array(y)), np.trapezoid(y), rtol=1e-13, atol=1e-12)
    _close(cp.trapezoid(cp.array(y), dx=0.1, axis=0), np.trapezoid(y, dx=0.1, axis=0), rtol=1e-13, atol=1e-12)
    _close(cp.trapezoid(cp.array(y), x=cp.array(xs)), np.trapezoid(y, x=xs), rtol=1e-12, atol=1e-11)


def test_convolve_correlate():
    rng = np.random.default_rng(14)
    for n, m in ((10, 3), (3, 10), (7, 7), (1, 5), (12, 4), (4, 12)):
        a = rng.integers(-9, 9, n).astype(np.int64)
        v = rng.integers(-9, 9, m).astype(np.int64)
        for mode in ("full", "same", "valid"):
            _same(cp.convolve(cp.array(a), cp.array(v), mode), np.convolve(a, v, mode))
            _same(cp.correlate(cp.array(a), cp.array(v), mode), np.correlate(a, v, mode))
    a = _x((257,), np.float64, 15)
    v = _x((9,), np.float64, 16)
    _close(cp.convolve(cp.array(a), cp.array(v)), np.convolve(a, v), rtol=1e-12, atol=1e-12)
    _close(cp.correlate(cp.array(a), cp.array(v), "same"), np.correlate(a, v, "same"), rtol=1e-12, atol=1e-12)


def test_creation_and_index_helpers():
    # the library's default float is float32 (eye / identity / tri)
    _same(cp.identity(4), np.identity(4, dtype=np.float32))
    _same(cp.identity(3, dtype=np.int32), np.identity(3, dtype=np.int32))
    _same(cp.tri(4, 6, 1), np.tri(4, 6, 1, dtype=np.float32))
    _same(cp.tri(5, k=-1, dtype=np.int32), np.tri(5, k=-1, dtype=np.int32))
    _same(cp.logspace(0, 3, 7), np.logspace(0, 3, 7))
    _same(cp.geomspace(1, 1000, 4), np.geomspace(1, 1000, 4))
    xv = np.array([1.5, -2.0, 3.0, 0.5], dtype=np.float32)
    _same(cp.vander(cp.array(xv)), np.vander(xv))
    _same(cp.vander(cp.array(xv), 6, increasing=True), np.vander(xv, 6, increasing=True))
    _same(cp.vander(cp.array(np.array([2, 3], np.int32)), 4), np.vander(np.array([2, 3], np.int32), 4))
    _same(cp.indices((3, 4)), np.indices((3, 4)))
    _same(cp.indices((2, 3), sparse=True), np.indices((2, 3), sparse=True))
    a = np.arange(20, dtype=np.float32).reshape(4, 5)
    ix = np.ix_([0, 2], [1, 3, 4])
    got = cp.ix_(cp.array(np.array([0, 2])), cp.array(np.array([1, 3, 4])))
    _same(got, ix)
    _same(cp.array(a)[got], a[ix])
    _same(cp.ix_(cp.array(np.array([True, False, True, True]))), np.ix_(np.array([True, False, True, True])))
    for shape, wrap in (((4, 4), False), ((6, 3), False), ((7, 3), True), ((3, 5), False)):
        h = np.zeros(shape, np.float32)
        d = cp.array(h)
        np.fill_diagonal(h, 5.0, wrap=wrap)
        cp.fill_diagonal(d, 5.0, wrap=wrap)
        _same(d, h)
    h3 = np.zeros((3, 3, 3), np.int32)
    d3 = cp.array(h3)
    np.fill_diagonal(h3, 2)
    cp.fill_diagonal(d3, 2)
    _same(d3, h3)
    _same(cp.diag_indices(4), np.diag_indices(4))
    _same(cp.diag_indices_from(cp.array(np.zeros((3, 3, 3)))), np.diag_indices_from(np.zeros((3, 3, 3))))
    for k in (-1, 0, 2):
        _same(cp.tril_indices(5, k), np.tril_indices(5, k))
        _same(cp.triu_indices(5, k, 7), np.triu_indices(5, k, 7))
    _same(cp.tril_indices_from(cp.array(a)), np.tril_indices_from(a))
    _same(cp.triu_indices_from(cp.array(a), 1), np.triu_indices_from(a, 1))
    r, c = np.array([0, 3, 2, 1]), np.array([4, 0, 2, 1])
    _same(cp.ravel_multi_index((cp.array(r), cp.array(c)), (4, 5)), np.ravel_multi_index((r, c), (4, 5)))
    _same(cp.ravel_multi_index((cp.array(r + 3), cp.array(c)), (4, 5), mode="wrap"),
          np.ravel_multi_index((r + 3, c), (4, 5), mode="wrap"))
    _same(cp.ravel_multi_index((cp.array(r + 3), cp.array(c - 2)), (4, 5), mode="clip"),
          np.ravel_multi_index((r + 3, c - 2), (4, 5), mode="clip"))
    with pytest.raises(ValueError):
        cp.ravel_multi_index((cp.array(r + 3), cp.array(c)), (4, 5))
    flat = np.array([0, 7, 19, 13])
    _same(cp.unravel_index(cp.array(flat), (4, 5)), np.unravel_index(flat, (4, 5)))
    _same(cp.unravel_index(cp.array(flat.reshape(2, 2)), (4, 5)), np.unravel_index(flat.reshape(2, 2), (4, 5)))
    with pytest.raises(ValueError):
        cp.unravel_index(cp.array(np.array([20])), (4, 5))


def test_cumulative_include_initial_and_dtype_helpers():
    x = _x((6, 7), np.float64, 17)
    i = np.arange(1, 9, dtype=np.int32)
    _same(cp.cumulative_sum(cp.array(i)), np.cumulative_sum(i))
    _same(cp.cumulative_sum(cp.array(i), include_initial=True), np.cumulative_sum(i, include_initial=True))
    _same(cp.cumulative_prod(cp.array(i), include_initial=True), np.cumulative_prod(i, include_initial=True))
    _close(cp.cumulative_sum(cp.array(x), axis=1, include_initial=True),
           np.cumulative_sum(x, axis=1, include_initial=True), rtol=1e-14, atol=1e-13)
    with pytest.raises(ValueError):
        cp.cumulative_sum(cp.array(x))
    a = cp.array(np.zeros(3, np.float32))
    assert cp.result_type(a, np.int64) == np.result_type(np.float32, np.int64)
    assert cp.can_cast(a, np.float64) and not cp.can_cast(a, np.int32)
    assert cp.promote_types(np.int32, np.float32) == np.float64
    assert cp.finfo(np.float32).eps == np.finfo(np.float32).eps
    assert cp.iinfo(np.int16).max == 32767
    assert cp.ndim(a) == 1 and cp.shape(a) == (3,) and cp.size(a) == 3
    assert cp.isscalar(3.0) and not cp.isscalar(a)
    assert isinstance(cp.asnumpy(a), np.ndarray)
    assert cp.get_array_module(a) is cp
