"""einsum, pad, insert / delete, multi-dimensional histograms, bit
packing, polynomials, window functions, i0, unwrap, the unique family,
index tricks, block, apply_along_axis and the host-side names (I/O,
printing, vectorize) against NumPy.  Data movement and integer work are
bit-exact; float contractions and transcendental windows are held to the
tolerance written at each check (summation order and libm rounding)."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu


def _h(a):
    return a.get() if hasattr(a, "get") else np.asarray(a)


def _same(got, want):
    if isinstance(want, (tuple, list)):
        assert len(got) == len(want)
        for g, w in zip(got, want):
            _same(g, w)
        return
    got, want = _h(got), np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    if want.dtype.kind == "f":
        assert np.array_equal(got, want, equal_nan=True), (got, want)
    else:
        assert np.array_equal(got, want), (got, want)


def _close(got, want, rtol, atol=0.0):
    got, want = _h(got), np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol)


def _x(shape, dtype=np.float32, seed=0, scale=1.0):
    rng = np.random.default_rng(seed)
    if np.dtype(dtype).kind in "iu":
        return rng.integers(-20 if np.dtype(dtype).kind == "i" else 0, 20, shape).astype(dtype)
    return (rng.standard_normal(shape) * scale).astype(dtype)


EINSUM_CASES = [
    ("ij,jk->ik", [(5, 7), (7, 3)]),
    ("ij,jk", [(5, 7), (7, 3)]),
    ("bij,bjk->bik", [(4, 5, 6), (4, 6, 3)]),
    ("ij->ji", [(4, 6)]),
    ("ii->i", [(5, 5)]),
    ("ii", [(5, 5)]),
    ("ij->", [(4, 6)]),
    ("ij->j", [(4, 6)]),
    ("i,j->ij", [(4,), (6,)]),
    ("i,i->", [(9,), (9,)]),
    ("i,i", [(9,), (9,)]),
    ("ij,ij->ij", [(4, 6), (4, 6)]),
    ("ij,ji->", [(4, 6), (6, 4)]),
    ("...ij,...jk->...ik", [(2, 3, 4, 5), (2, 3, 5, 2)]),
    ("...ij,jk", [(3, 4, 5), (5, 2)]),
    ("i...->...", [(3, 4, 5)]),
    ("ijk,kl,lm->im", [(3, 4, 5), (5, 6), (6, 2)]),
    ("abc,cd,b->ad", [(3, 4, 5), (5, 2), (4,)]),
    ("ij,j->i", [(6, 8), (8,)]),
    ("iij,jk->ik", [(4, 4, 3), (3, 5)]),
    ("ijk->kji", [(2, 3, 4)]),
    ("ij,kl->ijkl", [(2, 3), (4, 5)]),
]


@pytest.mark.parametrize("sub,shapes", EINSUM_CASES)
def test_einsum(sub, shapes):
    for dt, tol in ((np.float64, 1e-12), (np.float32, 2e-5), (np.int32, None), (np.int64, None)):
        ops = [_x(s, dt, seed=i) for i, s in enumerate(shapes)]
        got = cp.einsum(sub, *[cp.array(o) for o in ops])
        want = np.einsum(sub, *ops)
        if tol is None:
            _same(got, want)
        else:
            _close(got, want, rtol=tol, atol=tol * 10)


def test_einsum_mixed_and_path():
    a, b = _x((4, 5), np.int32), _x((5, 3), np.float32, 1)
    _close(cp.einsum("ij,jk->ik", cp.array(a), cp.array(b)), np.einsum("ij,jk->ik", a, b), rtol=1e-12)
    _close(cp.einsum("ij,jk->ik", cp.array(a), cp.array(b), dtype=np.float64),
           np.einsum("ij,jk->ik", a, b, dtype=np.float64), rtol=1e-12)
    c = _x((3, 6), np.float64, 2)
    p = cp.einsum_path("ij,jk,kl->il", cp.array(a), cp.array(b), cp.array(c))
    assert p[0] == np.einsum_path("ij,jk,kl->il", a, b, c)[0]
    with pytest.raises(ValueError):
        cp.einsum("ij,jk->ik", cp.array(a), cp.array(a))


PAD_MODES = ["constant", "edge", "reflect", "symmetric", "wrap", "maximum", "minimum", "mean",
             "linear_ramp"]


@pytest.mark.parametrize("mode", PAD_MODES)
def test_pad(mode):
    for dt in (np.float32, np.int32, np.float64):
        a = _x((5, 7), dt, 3, scale=10)
        for pw in (2, (1, 3), ((0, 2), (3, 1)), ((6, 9), (8, 4))):
            if mode in ("maximum", "minimum", "mean", "linear_ramp") and pw == ((6, 9), (8, 4)):
                pw = ((2, 3), (4, 1))
            kw = {}
            if mode == "constant":
                kw = {"constant_values": ((1, 2), (3, 4))}
            if mode == "linear_ramp":
                kw = {"end_values": ((5, -3), (2, 7))}
            want = np.pad(a, pw, mode=mode, **kw)
            got = cp.pad(cp.array(a), pw, mode=mode, **kw)
            if mode == "mean" and dt != np.int32:
                _close(got, want, rtol=1e-6)
            else:
                _same(got, want)
    b = _x((3, 4, 5), np.int64, 4)
    _same(cp.pad(cp.array(b), ((1, 0), (0, 2), (3, 3)), mode="reflect"),
          np.pad(b, ((1, 0), (0, 2), (3, 3)), mode="reflect"))
    _same(cp.pad(cp.array(b), 1), np.pad(b, 1))
    _same(cp.pad(cp.array(b[0, 0]), (2, 3), mode="maximum", stat_length=2),
          np.pad(b[0, 0], (2, 3), mode="maximum", stat_length=2))
    f = _x((6,), np.float32, 5)
    _same(cp.pad(cp.array(f), (4, 2), mode="linear_ramp"), np.pad(f, (4, 2), mode="linear_ramp"))


def test_insert_delete():
    a = _x((4, 6), np.int32, 6)
    for obj, ax in ((1, 0), (-1, 1), ([0, 2, 2], 1), (slice(1, 5, 2), 1), ([True, False, True, False], 0),
                    (3, None), ([0, 5, 23], None)):
        if isinstance(obj, list) and isinstance(obj[0], bool):
            _same(cp.delete(cp.array(a), cp.array(np.array(obj)), axis=ax), np.delete(a, np.array(obj), axis=ax))
        else:
            _same(cp.delete(cp.array(a), obj, axis=ax), np.delete(a, obj, axis=ax))
    with pytest.raises(IndexError):
        cp.delete(cp.array(a), 9, axis=0)
    for obj, vals, ax in ((1, 99, 0), (2, [7, 8, 9, 10], 1), ([1, 1, 4], [5, 6, 7], 1), (6, 3, 1),
                          (0, [[1], [2], [3], [4]], 1), ([0, 3], 42, 0), (5, [1, 2], None),
                          (slice(0, 3), -1, 1), (-2, 11, 1)):
        _same(cp.insert(cp.array(a), obj, vals, axis=ax), np.insert(a, obj, vals, axis=ax))
    f = _x((5,), np.float32, 7)
    _same(cp.insert(cp.array(f), [1, 3], [2.5, -1.5]), np.insert(f, [1, 3], [2.5, -1.5]))
    _same(cp.diagflat(cp.array(f)), np.diagflat(f))
    _same(cp.diagflat(cp.array(f.reshape(1, 5)), -2), np.diagflat(f.reshape(1, 5), -2))
    _same(cp.ediff1d(cp.array(f)), np.ediff1d(f))
    _same(cp.ediff1d(cp.array(a), to_begin=[-1, -2], to_end=5), np.ediff1d(a, to_begin=[-1, -2], to_end=5))
    with pytest.raises(TypeError):
        cp.ediff1d(cp.array(a), to_end=2.5)


def test_histogramdd_2d():
    rng = np.random.default_rng(8)
    s = rng.standard_normal((2000, 3)).astype(np.float32)
    for kw in ({}, {"bins": 4}, {"bins": (3, 5, 2)}, {"bins": 4, "range": [(-1, 1), (-2, 2), (0, 3)]},
               {"bins": [np.array([-2.0, 0.0, 2.0]), 3, np.linspace(-1, 1, 5)]}):
        kd = dict(kw)
        if "bins" in kd and isinstance(kd["bins"], list):
            kd["bins"] = [cp.array(b) if isinstance(b, np.ndarray) else b for b in kd["bins"]]
        got = cp.histogramdd(cp.array(s), **kd)
        want = np.histogramdd(s, **kw)
        _same(got[0], want[0])
        _same(got[1], want[1])
    w = rng.standard_normal(2000)
    g = cp.histogramdd(cp.array(s), bins=3, weights=cp.array(w))
    wn = np.histogramdd(s, bins=3, weights=w)
    _close(g[0], wn[0], rtol=0, atol=1e-12 * np.abs(w).sum())
    g = cp.histogramdd(cp.array(s), bins=3, density=True)
    _close(g[0], np.histogramdd(s, bins=3, density=True)[0], rtol=1e-13)
    x, y = s[:, 0], s[:, 1]
    got = cp.histogram2d(cp.array(x), cp.array(y), bins=(5, 4))
    want = np.histogram2d(x, y, bins=(5, 4))
    for gv, wv in zip(got, want):
        _same(gv, wv)
    _same(cp.histogram_bin_edges(cp.array(x), bins=7), np.histogram_bin_edges(x, bins=7))


def test_packbits():
    # bytes come back as uint16 (the device type holding uint8 data), as in
    # the reference (bitwise_ops.py:100-109); elements count by their low byte
    rng = np.random.default_rng(9)
    b = rng.integers(0, 2, (5, 19)).astype(np.bool_)
    for ax in (None, 0, 1, -1):
        for order in ("big", "little"):
            _same(cp.packbits(cp.array(b), axis=ax, bitorder=order),
                  np.packbits(b, axis=ax, bitorder=order).astype(np.uint16))
    u = rng.integers(0, 256, (4, 6)).astype(np.uint8)
    for ax in (None, 0, 1):
        for order in ("big", "little"):
            _same(cp.unpackbits(cp.array(u), axis=ax, bitorder=order),
                  np.unpackbits(u, axis=ax, bitorder=order).astype(np.uint16))
    for count in (5, 48, 50, -3):
        _same(cp.unpackbits(cp.array(u), axis=1, count=count),
              np.unpackbits(u, axis=1, count=count).astype(np.uint16))
    i = np.array([-3, 0, 256, 1, 255, 512, 7, 0, 3], dtype=np.int32)
    _same(cp.packbits(cp.array(i)), np.packbits(i.astype(np.uint8)).astype(np.uint16))
    _same(cp.unpackbits(cp.array(i)), np.unpackbits(i.astype(np.uint8)).astype(np.uint16))


def test_polynomials():
    p = np.array([2.0, -3.0, 0.5, 4.0])
    q = np.array([1.0, 2.0])
    x = _x((100,), np.float64, 10, scale=3)
    _same(cp.polyval(cp.array(p), cp.array(x)), np.polyval(p, x))
    _same(cp.polyval(cp.array(p.astype(np.float32)), cp.array(x.astype(np.float32))),
          np.polyval(p.astype(np.float32), x.astype(np.float32)))
    _same(cp.polyval(cp.array(np.array([3, 0, -2])), cp.array(np.arange(-5, 5))),
          np.polyval(np.array([3, 0, -2]), np.arange(-5, 5)))
    _same(cp.polyadd(cp.array(p), cp.array(q)), np.polyadd(p, q))
    _same(cp.polysub(cp.array(q), cp.array(p)), np.polysub(q, p))
    _same(cp.polymul(cp.array(p), cp.array(q)), np.polymul(p, q))
    gq, gr = cp.polydiv(cp.array(p), cp.array(q))
    wq, wr = np.polydiv(p, q)
    _close(gq, wq, rtol=1e-15)
    _close(gr, wr, rtol=1e-15, atol=1e-15)
    _same(cp.polyder(cp.array(p)), np.polyder(p))
    _same(cp.polyder(cp.array(p), 2), np.polyder(p, 2))
    _same(cp.polyint(cp.array(p)), np.polyint(p))
    _same(cp.polyint(cp.array(p), 2, [1.0, -1.0]), np.polyint(p, 2, [1.0, -1.0]))
    _same(cp.poly(cp.array(np.array([1.0, -2.0, 3.0]))), np.poly(np.array([1.0, -2.0, 3.0])))
    P = cp.poly1d([1.0, -3.0, 2.0])
    N = np.poly1d([1.0, -3.0, 2.0])
    _same(P(cp.array(x)), N(x))
    assert P.order == N.order
    _same((P * 2 + cp.poly1d([1.0, 1.0])).coeffs, (N * 2 + np.poly1d([1.0, 1.0])).coeffs)
    _same(P.deriv().coeffs, N.deriv().coeffs)
    _same((P ** 2).coeffs, (N ** 2).coeffs)


def test_windows_i0_unwrap():
    for M in (0, 1, 2, 7, 64):
        for name in ("bartlett", "blackman", "hamming", "hanning"):
            _close(getattr(cp, name)(M), getattr(np, name)(M), rtol=0, atol=1e-15)
        _close(cp.kaiser(M, 5.0), np.kaiser(M, 5.0), rtol=1e-13, atol=1e-15)
    x = np.concatenate([np.linspace(-30, 30, 301), [0.0, 8.0, -8.0]])
    _close(cp.i0(cp.array(x)), np.i0(x), rtol=1e-14)
    _close(cp.i0(cp.array(x.astype(np.float32))), np.i0(x.astype(np.float32)), rtol=2e-6)
    _close(cp.i0(cp.array(np.arange(5))), np.i0(np.arange(5)), rtol=1e-14)
    rng = np.random.default_rng(11)
    ph = np.cumsum(rng.standard_normal((3, 200)) * 2, axis=1)
    wrapped = np.angle(np.exp(1j * ph))
    _close(cp.unwrap(cp.array(wrapped)), np.unwrap(wrapped), rtol=1e-12, atol=1e-11)
    _close(cp.unwrap(cp.array(wrapped), axis=0), np.unwrap(wrapped, axis=0), rtol=1e-12, atol=1e-11)
    _close(cp.unwrap(cp.array(wrapped), discont=4.0), np.unwrap(wrapped, discont=4.0), rtol=1e-12, atol=1e-11)
    iv = np.array([0, 1, 5, 6, 2, 9, 3], dtype=np.int64)
    _same(cp.unwrap(cp.array(iv), period=6), np.unwrap(iv, period=6))


def test_unique_family():
    rng = np.random.default_rng(12)
    x = rng.integers(0, 9, (6, 7)).astype(np.int32)
    ua, un = cp.unique_all(cp.array(x)), np.unique_all(x)
    for g, w in zip(ua, un):
        _same(g, w)
    for fn in ("unique_counts", "unique_inverse"):
        for g, w in zip(getattr(cp, fn)(cp.array(x)), getattr(np, fn)(x)):
            _same(g, w)
    f = np.array([1.0, np.nan, 2.0, np.nan, 1.0], dtype=np.float32)
    _same(cp.unique_values(cp.array(f)), np.unique_values(f))
    _same(cp.unique_values(cp.array(x)), np.unique_values(x))


def test_index_tricks_block_apply():
    _same(cp.mgrid[0:4, 1:6:2], np.mgrid[0:4, 1:6:2])
    _same(cp.mgrid[0:1:5j], np.mgrid[0:1:5j])
    _same(cp.mgrid[-1:1:3j, 0:3], np.mgrid[-1:1:3j, 0:3])
    _same(cp.ogrid[0:3, 0:4], np.ogrid[0:3, 0:4])
    a = np.array([1, 2, 3], dtype=np.int32)
    _same(cp.r_[cp.array(a), 0, 7:10], np.r_[a, 0, 7:10])
    _same(cp.r_[1:4, 2.5], np.r_[1:4, 2.5])
    _same(cp.r_["0,2", cp.array(a), cp.array(a)], np.r_["0,2", a, a])
    _same(cp.c_[cp.array(a), cp.array(a * 2)], np.c_[a, a * 2])
    assert cp.s_[1:3] == np.s_[1:3] and cp.index_exp[2] == np.index_exp[2]
    A, B = _x((2, 2), np.float32, 13), _x((2, 3), np.float32, 14)
    C, D = _x((1, 2), np.float32, 15), _x((1, 3), np.float32, 16)
    _same(cp.block([[cp.array(A), cp.array(B)], [cp.array(C), cp.array(D)]]), np.block([[A, B], [C, D]]))
    _same(cp.block([cp.array(a), cp.array(a)]), np.block([a, a]))
    _same(cp.block([[cp.array(a)], [cp.array(a)]]), np.block([[a], [a]]))
    m = _x((3, 4, 5), np.float64, 17)
    _same(cp.apply_along_axis(lambda v: v[::-1] * 2, 1, cp.array(m)),
          np.apply_along_axis(lambda v: v[::-1] * 2, 1, m))
    _close(cp.apply_along_axis(lambda v: cp.sum(v), 2, cp.array(m)),
           np.apply_along_axis(np.sum, 2, m), rtol=1e-13)
    _close(cp.apply_over_axes(cp.sum, cp.array(m), [0, 2]), np.apply_over_axes(np.sum, m, [0, 2]), rtol=1e-13)
    _same(cp.resize(cp.array(a), (2, 4)), np.resize(a, (2, 4)))
    _same(cp.resize(cp.array(a), 2), np.resize(a, 2))
    t = np.array([0, 0, 3, 0, 5, 0, 0], dtype=np.int32)
    for trim in ("fb", "f", "b"):
        _same(cp.trim_zeros(cp.array(t), trim), np.trim_zeros(t, trim))
    z = np.array([np.inf, -np.inf, 1.0, np.nan, -0.0], dtype=np.float32)
    _same(cp.isposinf(cp.array(z)), np.isposinf(z))
    _same(cp.isneginf(cp.array(z)), np.isneginf(z))
    _same(cp.mask_indices(4, cp.triu, 1), np.mask_indices(4, np.triu, 1))
    with pytest.raises(ValueError):
        cp.asarray_chkfinite(cp.array(z))
    _same(cp.asarray_chkfinite(cp.array(a)), a)
    _same(cp.fromfunction(lambda i, j: i * 10 + j, (3, 4), dtype=np.int64),
          np.fromfunction(lambda i, j: i * 10 + j, (3, 4), dtype=np.int64))


def test_host_api(tmp_path):
    a = _x((3, 4), np.float32, 18)
    d = cp.array(a)
    f = tmp_path / "a.npy"
    cp.save(f, d)
    _same(cp.load(f), a)
    cp.savez(tmp_path / "z.npz", x=d, y=cp.array(a * 2))
    with cp.load(tmp_path / "z.npz") as z:
        _same(z["y"], a * 2)
    cp.savetxt(tmp_path / "t.txt", d)
    _close(cp.loadtxt(tmp_path / "t.txt"), np.loadtxt(tmp_path / "t.txt"), rtol=0)
    assert cp.array2string(d) == np.array2string(a)
    assert cp.array_str(d) == np.array_str(a)
    v = cp.vectorize(lambda x, y: x + 2 * y if x > 0 else y)
    _same(v(d, cp.array(a * 3)), np.vectorize(lambda x, y: x + 2 * y if x > 0 else y)(a, a * 3))
    assert cp.common_type(cp.array(np.zeros(2, np.int32))) is np.float64
    assert cp.may_share_memory(d, d[1:])
    assert not cp.may_share_memory(d, cp.array(a))
    assert cp.geterrobj()[0] == np.getbufsize()
    assert cp.issubdtype(d.dtype, cp.floating)
