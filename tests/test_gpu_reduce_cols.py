"""Reductions over a strided axis (axis=0 of a C-contiguous matrix, or a
middle axis), the layouts the reference reduces with its axis kernels
(reductions.py:74-163, ndarray.py:2015-2152).

Sums, products, max and min over element sizes of 2, 4 and 8 bytes with an
inner extent that is a multiple of the 16-byte vector and an aligned base
take the column-vector kernel (a lane owns 16 bytes of adjacent columns,
the four waves of a workgroup take every fourth row); arg-reductions, bool
(the one one-byte device type), odd inner extents and offset bases take the
column-per-thread kernels.  Both must give NumPy's answer:
integers and max / min / arg-reductions bit for bit (first occurrence on
ties, first NaN), float sums within the rounding bound of a float64 sum.
Shapes cover a partial last column block, a single split (short axis), many
splits, an outer extent above one, and NaNs."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu

SHAPES = [((1000, 260), 0), ((5, 4096), 0), ((3000, 1024), 0), ((65, 12), 0),
          ((7, 300, 520), 1), ((4, 2048, 16), 1), ((20000, 64), 0)]
DTYPES = [np.float32, np.float64, np.float16, np.int16, np.int32, np.int64, np.uint16, np.bool_]


def _data(rng, shape, dt, small=False):
    if dt == np.bool_:
        return rng.random(shape) < 0.5
    if np.dtype(dt).kind == "f":
        x = rng.standard_normal(shape).astype(dt)
        if small:
            x = np.round(x).astype(dt)                  # many ties
        return x
    info = np.iinfo(dt)
    lo, hi = (0, 4) if small else (max(info.min, -1000), min(info.max, 1000))
    return rng.integers(lo, hi, shape).astype(dt)


def _check_sum(got, h, axis):
    want = np.sum(h, axis=axis)
    assert got.dtype == want.dtype and got.shape == want.shape
    if want.dtype.kind == "f":
        ref = np.sum(h.astype(np.float64), axis=axis)
        tol = np.finfo(want.dtype).eps * np.sum(np.abs(h.astype(np.float64)), axis=axis) * 2
        assert np.all(np.abs(got.astype(np.float64) - ref) <= tol + np.finfo(want.dtype).tiny)
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("shape_axis", SHAPES, ids=lambda s: f"{s[0]}-ax{s[1]}")
@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: np.dtype(d).name)
def test_strided_axis_reductions(shape_axis, dt):
    shape, axis = shape_axis
    rng = np.random.default_rng(43000 + len(shape) * 7 + shape[-1])
    h = _data(rng, shape, dt)
    d = cp.array(h)
    _check_sum(cp.sum(d, axis=axis).get(), h, axis)
    for f in ("max", "min", "argmax", "argmin"):
        got, want = getattr(cp, f)(d, axis=axis).get(), getattr(np, f)(h, axis=axis)
        assert got.dtype == want.dtype and np.array_equal(got, want), f
    if np.dtype(dt).kind == "f":
        got = cp.mean(d, axis=axis).get()
        want = np.mean(h.astype(np.float64), axis=axis)
        np.testing.assert_allclose(got.astype(np.float64), want,
                                   rtol=2e-3 if dt == np.float16 else 1e-5, atol=1e-3)


@pytest.mark.parametrize("dt", [np.float32, np.int32, np.float16, np.int64], ids=lambda d: np.dtype(d).name)
def test_strided_axis_ties_first_occurrence(dt):
    rng = np.random.default_rng(43100)
    h = _data(rng, (4099, 520), dt, small=True)            # each column's extreme repeats
    d = cp.array(h)
    for f in ("argmax", "argmin"):
        assert np.array_equal(getattr(cp, f)(d, axis=0).get(), getattr(np, f)(h, axis=0)), f


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.float16], ids=lambda d: np.dtype(d).name)
def test_strided_axis_nans(dt):
    rng = np.random.default_rng(43200)
    h = rng.standard_normal((3001, 264)).astype(dt)
    h[rng.random(h.shape) < 0.002] = np.nan
    h[:, 5] = np.nan                                       # an all-NaN column
    d = cp.array(h)
    for f in ("argmax", "argmin", "max", "min"):
        got, want = getattr(cp, f)(d, axis=0).get(), getattr(np, f)(h, axis=0)
        assert np.array_equal(got, want, equal_nan=want.dtype.kind == "f"), f
    with np.errstate(all="ignore"):
        for f in ("nanmax", "nanargmax"):
            if f == "nanargmax":
                ok = ~np.all(np.isnan(h), axis=0)
                got = cp.nanargmax(d[:, ok], axis=0).get()
                assert np.array_equal(got, np.nanargmax(h[:, ok], axis=0)), f
            else:
                got, want = cp.nanmax(d, axis=0).get(), np.nanmax(h, axis=0)
                assert np.array_equal(got, want, equal_nan=True), f
        got = cp.nansum(d, axis=0).get()
        ref = np.nansum(h.astype(np.float64), axis=0)
        tol = np.finfo(dt).eps * np.nansum(np.abs(h.astype(np.float64)), axis=0) * 2
        assert np.all(np.abs(got.astype(np.float64) - ref) <= tol + np.finfo(dt).tiny)


@pytest.mark.parametrize("dt", [np.float32, np.int16, np.float64], ids=lambda d: np.dtype(d).name)
def test_strided_axis_offset_base(dt):
    """A contiguous view one element into its buffer: the base is not
    16-byte aligned, so the column-per-thread kernels run; same answers."""
    rng = np.random.default_rng(43300)
    flat = _data(rng, (1 + 2000 * 256,), dt)
    h = flat[1:].reshape(2000, 256)
    d = cp.array(flat)[1:].reshape(2000, 256)
    _check_sum(cp.sum(d, axis=0).get(), h, 0)
    assert np.array_equal(cp.argmax(d, axis=0).get(), np.argmax(h, axis=0))
    assert np.array_equal(cp.min(d, axis=0).get(), np.min(h, axis=0))


SCAN_SHAPES = [((1000, 260), 0), ((5, 4096), 0), ((3000, 1024), 0), ((65, 12), 0),
               ((7, 300, 520), 1), ((20000, 64), 0), ((999, 130), 0)]


@pytest.mark.parametrize("shape_axis", SCAN_SHAPES, ids=lambda s: f"{s[0]}-ax{s[1]}")
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.float16, np.int16, np.int32, np.int64,
                                np.uint16, np.bool_], ids=lambda d: np.dtype(d).name)
def test_strided_axis_cumsum(shape_axis, dt):
    """cumsum over a strided axis: 2-, 4- and 8-byte inputs with a
    16-byte-multiple inner extent take the column-vector scan (chunk totals,
    carries, rescan), the rest the column-per-thread scan.  Integers bit for
    bit (64-bit accumulation as NumPy); floats within the float64 running
    sum's rounding bound."""
    shape, axis = shape_axis
    rng = np.random.default_rng(43400 + shape[0] + shape[-1])
    h = _data(rng, shape, dt)
    got = cp.cumsum(cp.array(h), axis=axis).get()
    want = np.cumsum(h, axis=axis)
    assert got.dtype == want.dtype and got.shape == want.shape
    if want.dtype.kind == "f":
        ref = np.cumsum(h.astype(np.float64), axis=axis)
        bound = np.cumsum(np.abs(h.astype(np.float64)), axis=axis)
        tol = np.finfo(want.dtype).eps * (np.abs(ref) + 1e-3 * bound) + np.finfo(want.dtype).tiny
        assert np.all(np.abs(got.astype(np.float64) - ref) <= 2 * tol + 1e-12 * bound)
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("dt", [np.int32, np.float64, np.int16], ids=lambda d: np.dtype(d).name)
def test_strided_axis_cumprod(dt):
    rng = np.random.default_rng(43500)
    h = rng.choice(np.array([-1, 1, 1, 2], dtype=dt), size=(40, 520))
    got = cp.cumprod(cp.array(h), axis=0).get()
    want = np.cumprod(h, axis=0)
    assert got.dtype == want.dtype and np.array_equal(got, want)


def test_strided_axis_cumsum_offset_base():
    """Input one element into its buffer (not 16-byte aligned): the
    column-per-thread scan; same answer."""
    rng = np.random.default_rng(43600)
    flat = rng.integers(-1000, 1000, 1 + 3000 * 256).astype(np.int32)
    h = flat[1:].reshape(3000, 256)
    got = cp.cumsum(cp.array(flat)[1:].reshape(3000, 256), axis=0).get()
    assert np.array_equal(got, np.cumsum(h, axis=0))
