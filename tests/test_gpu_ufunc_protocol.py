"""NumPy's ufunc protocol on device arrays, and the ufuncs added for it,
against NumPy: ``np.<ufunc>(device arrays)`` with ``out=`` / ``dtype=`` /
``where=``, ``ufunc.reduce`` / ``accumulate`` on the device, and
NotImplemented (NumPy's TypeError) for what has no device form, never a
host computation.  spacing / bitwise_count / ldexp / gcd / lcm / frexp /
modf: bit-exact (float16 / float32 / float64 and the integer types)."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu


def _same(got, want):
    got = got.get() if hasattr(got, "get") else np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    if want.dtype.kind == "f":
        assert np.array_equal(got.view(f"u{got.itemsize}"), want.view(f"u{want.itemsize}")) or \
            np.array_equal(got, want, equal_nan=True)
    else:
        assert np.array_equal(got, want)


SPECIAL = [0.0, -0.0, 1.0, -1.0, 1.5, -2.75, 3e-39, -1e-45, 65504.0, 1e30, -3.4e38,
           np.inf, -np.inf, np.nan, 0.1, 1e-5, 123456.789]


@pytest.mark.parametrize("dtype", [np.float16, np.float32, np.float64])
def test_float_ufuncs(dtype):
    rng = np.random.default_rng(3)
    with np.errstate(all="ignore"):
        x = np.concatenate([np.array(SPECIAL).astype(dtype),
                            (rng.standard_normal(2000) * 10.0 ** rng.integers(-8, 8, 2000)).astype(dtype)])
        n = rng.integers(-30, 30, x.size).astype(np.int32)
        g = cp.array(x)
        _same(cp.spacing(g), np.spacing(x))
        m, e = cp.frexp(g)
        wm, we = np.frexp(x)
        _same(m, wm)
        _same(e, we)
        f, i = cp.modf(g)
        wf, wi = np.modf(x)
        _same(f, wf)
        _same(i, wi)
        _same(cp.ldexp(g, cp.array(n)), np.ldexp(x, n))
        _same(cp.conjugate(g), np.conjugate(x))


def test_spacing_every_float16():
    """np.spacing over all 65536 float16 bit patterns (NumPy's half rule:
    the step toward +inf, 65504 -> inf), and float32 edges (the step away
    from zero, +-max -> +-inf, -0 -> +smallest subnormal)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    with np.errstate(all="ignore"):
        _same(cp.spacing(cp.array(h)), np.spacing(h))
        f = np.array([0.0, -0.0, 3.4028235e38, -3.4028235e38, 1e-45, -1e-45, 2.0, -2.0], np.float32)
        _same(cp.spacing(cp.array(f)), np.spacing(f))


@pytest.mark.parametrize("dtype", [np.int16, np.int32, np.int64, np.uint16, np.uint32, np.uint64])
def test_integer_ufuncs(dtype):
    rng = np.random.default_rng(4)
    info = np.iinfo(dtype)
    a = rng.integers(info.min, info.max, 3000, dtype=dtype, endpoint=True)
    b = rng.integers(info.min, info.max, 3000, dtype=dtype, endpoint=True)
    small = rng.integers(-1000 if info.min < 0 else 0, 1000, 3000).astype(dtype)
    a[:6] = np.array([0, 0, 1, info.max, info.min, 12], dtype=dtype)
    b[:6] = np.array([0, 5, 0, info.min, 0, 18], dtype=dtype)
    ga, gb = cp.array(a), cp.array(b)
    _same(cp.gcd(ga, gb), np.gcd(a, b))
    _same(cp.lcm(cp.array(small), cp.array(small[::-1].copy())), np.lcm(small, small[::-1]))
    want = np.bitwise_count(a)
    got = cp.bitwise_count(ga)
    assert np.array_equal(got.get(), want)  # uint8 in NumPy; uint16 on the device
    _same(cp.ldexp(cp.array(small), cp.array(np.full(3000, 3, np.int32))), np.ldexp(small, 3))


def test_protocol_call_out_dtype_where():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((40, 33)).astype(np.float32)
    y = rng.standard_normal((40, 33)).astype(np.float32)
    gx, gy = cp.array(x), cp.array(y)
    r = np.add(gx, gy)
    assert isinstance(r, cp.ndarray)
    _same(r, x + y)
    out = cp.array(np.zeros_like(x)) + 0
    r = np.multiply(gx, gy, out=out)
    assert r is out
    _same(out, x * y)
    np.add(gx, gy, out=gx)                     # in place through the protocol
    _same(gx, x + y)
    r64 = np.sin(cp.array(x), dtype=np.float64)
    assert r64.dtype == np.float64
    np.testing.assert_allclose(r64.get(), np.sin(x, dtype=np.float64), rtol=1e-14, atol=1e-15)
    mask = x > 0
    o = cp.array(np.full_like(x, -7.0)) + 0
    np.sqrt(cp.array(np.abs(x)), out=o, where=cp.array(mask))
    w = np.full_like(x, -7.0)
    np.sqrt(np.abs(x), out=w, where=mask)
    _same(o, w)
    i32 = cp.array(np.zeros((40, 33), np.int32)) + 0
    with pytest.raises(TypeError):
        np.add(gy, gy, out=i32)                # float -> int is not same_kind
    with pytest.raises(TypeError):
        np.add.outer(cp.array(x[0]), cp.array(y[0]))
    for u in (np.gcd, np.spacing, np.frexp, np.ldexp, np.modf, np.vecdot, np.matvec):
        assert _ufunc_has_device(u), u


def _ufunc_has_device(u):
    from macmetalpy_amd import _ufunc_table
    return _ufunc_table.lookup(u) is not None


def test_protocol_reduce_accumulate():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((64, 50)).astype(np.float32)
    gx = cp.array(x)
    s = np.add.reduce(gx)                      # axis 0 by default
    assert isinstance(s, cp.ndarray)
    np.testing.assert_allclose(s.get(), np.add.reduce(x.astype(np.float64)), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(np.add.reduce(gx, axis=1, keepdims=True).get(),
                               np.add.reduce(x.astype(np.float64), axis=1, keepdims=True),
                               rtol=1e-5, atol=1e-5)
    _same(np.maximum.reduce(gx, axis=1), np.maximum.reduce(x, axis=1))
    _same(np.minimum.reduce(gx, axis=None), np.minimum.reduce(x, axis=None))
    _same(np.logical_or.reduce(gx > 2, axis=0), np.logical_or.reduce(x > 2, axis=0))
    np.testing.assert_allclose(np.add.accumulate(gx).get(),
                               np.cumsum(x.astype(np.float64), axis=0), rtol=1e-5, atol=1e-5)
    ints = rng.integers(-5, 5, (10, 7)).astype(np.int32)
    _same(np.multiply.accumulate(cp.array(ints), axis=1), np.multiply.accumulate(ints, axis=1))
    xn = x.copy()
    xn[3, 4] = np.nan
    _same(np.fmax.reduce(cp.array(xn), axis=1), np.fmax.reduce(xn, axis=1))
    with pytest.raises(TypeError):
        np.add.reduceat(gx, [0, 10])


def test_gufunc_style_products():
    rng = np.random.default_rng(7)
    a = rng.standard_normal((5, 6, 7)).astype(np.float32)
    v = rng.standard_normal((5, 7)).astype(np.float32)
    w = rng.standard_normal((5, 6)).astype(np.float32)
    np.testing.assert_allclose(np.matvec(cp.array(a), cp.array(v)).get(), np.matvec(a, v),
                               rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(np.vecmat(cp.array(w), cp.array(a)).get(), np.vecmat(w, a),
                               rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(np.vecdot(cp.array(v), cp.array(v)).get(), np.vecdot(v, v),
                               rtol=1e-5)
