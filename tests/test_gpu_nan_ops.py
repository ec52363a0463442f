"""NaN-aware reductions on the GPU against the oracle (NumPy's nan*
functions, the reference's CPU path).  Bars: nanmax / nanmin / arg ops
exact; sums, products and means within 1e-5 relative of NumPy evaluated
in float64 (the device accumulates in float64); all-NaN slices as NumPy."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu


def _data(shape, dtype, seed, nan_frac=0.1):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(shape).astype(dtype)
    x[rng.random(shape) < nan_frac] = np.nan
    return x


def _close(got, want, rtol=1e-5):
    """Within rtol of ``want``; a float16 result may also be off by its
    subnormal spacing (2^-24), which one rounding of a tiny value allows."""
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    atol = 2.0 ** -24 if got.dtype == np.float16 else 0.0
    assert np.allclose(got[ok].astype(np.float64), want[ok], rtol=rtol, atol=atol)


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.float16])
@pytest.mark.parametrize("axis", [None, 0, 1, -1, (0, 2)])
def test_nan_sum_mean_prod_max_min(dtype, axis):
    x = _data((7, 33, 517), dtype, 1)
    x[2] = np.nan                       # all-NaN slices along axes 1 and 2
    x[3, :, :] = np.where(np.isnan(x[3]), 0.5, x[3])
    cx = cp.array(x)
    x64 = x.astype(np.float64)
    for keep in (False, True):
        kw = dict(axis=axis, keepdims=keep)
        for name in ("nanmax", "nanmin"):
            got = getattr(cp, name)(cx, **kw).get()
            want = ref.nan_reduce(name, x, **kw)
            assert got.dtype == want.dtype
            _close(got, want, rtol=0)
        got = cp.nansum(cx, **kw).get()
        assert got.dtype == ref.nan_reduce("nansum", x, **kw).dtype
        _close(got, ref.nan_reduce("nansum", x64, **kw), rtol=1e-5 if dtype != np.float16 else 2e-3)
        got = cp.nanmean(cx, **kw).get()
        assert got.dtype == ref.nan_reduce("nanmean", x, **kw).dtype
        _close(got, ref.nan_reduce("nanmean", x64, **kw), rtol=1e-5 if dtype != np.float16 else 1e-3)
    xs = (x * 0.01 + 1.0).astype(dtype)  # products of moderate size
    got = cp.nanprod(cp.array(xs), axis=axis).get()
    _close(got, ref.nan_reduce("nanprod", xs.astype(np.float64), axis=axis),
           rtol=1e-5 if dtype != np.float16 else 2e-2)


def test_nan_reductions_full_size_rows():
    """16384 x 16384-class row lengths exercise the split-row (multi
    workgroup) path; all-NaN rows and a row whose only finite value is last."""
    x = _data((6, 1 << 20), np.float32, 2, nan_frac=0.3)
    x[1] = np.nan
    x[4, :-1] = np.nan
    x[4, -1] = 0.25
    cx = cp.array(x)
    for axis in (None, 1):
        _close(cp.nanmax(cx, axis=axis).get(), ref.nan_reduce("nanmax", x, axis=axis), 0)
        _close(cp.nanmin(cx, axis=axis).get(), ref.nan_reduce("nanmin", x, axis=axis), 0)
        _close(cp.nansum(cx, axis=axis).get(),
               ref.nan_reduce("nansum", x.astype(np.float64), axis=axis))
        _close(cp.nanmean(cx, axis=axis).get(),
               ref.nan_reduce("nanmean", x.astype(np.float64), axis=axis))
    ok = np.delete(x, 1, axis=0)
    cok = cp.array(ok)
    for name in ("nanargmax", "nanargmin"):
        assert getattr(cp, name)(cok) == ref.nan_reduce(name, ok)
        assert np.array_equal(getattr(cp, name)(cok, axis=1).get(),
                              ref.nan_reduce(name, ok, axis=1))
        with pytest.raises(ValueError, match="All-NaN"):
            getattr(cp, name)(cx, axis=1)


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.float16])
def test_nanargmax_nanargmin_ties_inf_and_axes(dtype):
    x = _data((9, 40, 301), dtype, 3, nan_frac=0.2)
    x[0, 0, :5] = [np.nan, 3.0, 3.0, np.nan, 3.0]
    x[1, :, :] = -np.inf
    x[1, 5, 7] = np.nan
    cx = cp.array(x)
    for axis in (None, 0, 1, 2):
        for name in ("nanargmax", "nanargmin"):
            got = getattr(cp, name)(cx, axis=axis)
            want = ref.nan_reduce(name, x, axis=axis)
            if axis is None:
                assert got == want
            else:
                assert np.array_equal(got.get(), want)
    z = np.full((3, 4), np.nan, dtype)
    with pytest.raises(ValueError, match="All-NaN"):
        cp.nanargmax(cp.array(z))


@pytest.mark.parametrize("ddof", [0, 1])
def test_nanvar_nanstd(ddof):
    x = _data((12, 4099), np.float32, 4, nan_frac=0.25)
    x[3] = np.nan
    x[5, 1:] = np.nan  # one element: ddof=1 gives NaN
    cx = cp.array(x)
    x64 = x.astype(np.float64)
    for axis in (None, 1, 0):
        for name in ("nanvar", "nanstd"):
            got = getattr(cp, name)(cx, axis=axis, ddof=ddof).get()
            want = ref.nan_reduce(name, x64, axis=axis, ddof=ddof)
            assert got.dtype == np.float32
            _close(got, want, rtol=1e-4)


def test_nancumsum_nancumprod_and_integer_passthrough():
    x = _data((5, 3001), np.float32, 5)
    cx = cp.array(x)
    _close(cp.nancumsum(cx, axis=1).get(), ref.nan_reduce("nancumsum", x.astype(np.float64), axis=1),
           rtol=1e-5)
    xs = (x * 0.001 + 1.0).astype(np.float32)
    _close(cp.nancumprod(cp.array(xs), axis=1).get(),
           ref.nan_reduce("nancumprod", xs.astype(np.float64), axis=1), rtol=1e-5)
    i = np.random.default_rng(6).integers(-50, 50, (4, 999)).astype(np.int32)
    ci = cp.array(i)
    assert cp.nansum(ci).get() == np.nansum(i)
    assert np.array_equal(cp.nanmax(ci, axis=1).get(), np.nanmax(i, axis=1))
    assert cp.nanargmin(ci) == np.nanargmin(i)
    _close(cp.nanmean(ci, axis=0).get(), np.nanmean(i, axis=0))


def test_nan_reductions_empty_and_initial():
    e = np.zeros((3, 0), np.float32)
    ce = cp.array(e)
    assert np.array_equal(cp.nansum(ce, axis=1).get(), np.nansum(e, axis=1))
    assert np.array_equal(cp.nanprod(ce, axis=1).get(), np.nanprod(e, axis=1))
    with pytest.raises(ValueError):
        cp.nanmax(ce, axis=1)
    x = np.array([[np.nan, np.nan], [1.0, np.nan]], np.float32)
    assert np.array_equal(cp.nanmax(cp.array(x), axis=1, initial=3.0).get(),
                          np.nanmax(x, axis=1, initial=3.0))
    assert np.array_equal(cp.nansum(cp.array(x), axis=1, initial=2.0).get(),
                          np.nansum(x, axis=1, initial=2.0))
