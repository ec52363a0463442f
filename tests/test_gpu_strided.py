"""Strided-axis reductions, arg-reductions and scans, permuted copies and
device-side creation, against the oracle (NumPy).  Bars: integer and
arg results exact, float sums / scans within 1e-5 of float64, copies bit
for bit."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu


def _f32(shape, seed, nan_every=0):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32)
    if nan_every:
        x.reshape(-1)[::nan_every] = np.nan
    return x


@pytest.mark.parametrize("shape", [(4099, 300), (16384, 257), (3, 2048, 130), (200, 64)])
def test_column_arg_reductions_split(shape):
    """The reduced axis is split over workgroups (first index of ties and
    NaN rules survive the combine)."""
    x = _f32(shape, 1)
    x[x > 2.5] = 2.5            # many ties at the maximum
    x[x < -2.5] = -2.5
    xn = x.copy()
    xn.reshape(-1)[::977] = np.nan
    for arr in (x, xn):
        cx = cp.array(arr)
        for ax in range(arr.ndim - 1):
            assert np.array_equal(cp.argmax(cx, axis=ax).get(), np.argmax(arr, axis=ax))
            assert np.array_equal(cp.argmin(cx, axis=ax).get(), np.argmin(arr, axis=ax))
    cx = cp.array(xn)
    for ax in range(xn.ndim - 1):
        for name in ("nanargmax", "nanargmin"):
            assert np.array_equal(getattr(cp, name)(cx, axis=ax).get(),
                                  ref.nan_reduce(name, xn, axis=ax))
    i = np.random.default_rng(2).integers(-5, 5, shape).astype(np.int32)
    ci = cp.array(i)
    assert np.array_equal(cp.argmax(ci, axis=0).get(), np.argmax(i, axis=0))


@pytest.mark.parametrize("shape", [(16384, 300), (5000, 1031), (2, 3000, 65)])
def test_column_reductions(shape):
    x = _f32(shape, 3)
    cx = cp.array(x)
    x64 = x.astype(np.float64)
    for ax in range(len(shape) - 1):
        got = cp.sum(cx, axis=ax).get()
        assert np.allclose(got, x64.sum(axis=ax), rtol=1e-5, atol=1e-4)
        assert np.array_equal(cp.max(cx, axis=ax).get(), x.max(axis=ax))
        assert np.array_equal(cp.min(cx, axis=ax).get(), x.min(axis=ax))
    i = np.random.default_rng(4).integers(-1000, 1000, shape).astype(np.int32)
    assert np.array_equal(cp.sum(cp.array(i), axis=0).get(), i.sum(axis=0))


@pytest.mark.parametrize("shape,ax", [((5000, 700), 0), ((16384, 64), 0), ((3, 4000, 129), 1),
                                      ((130, 3, 50), 0), ((64, 5), 0)])
def test_column_scans_chunked(shape, ax):
    i = np.random.default_rng(5).integers(-100, 100, shape).astype(np.int32)
    got = cp.cumsum(cp.array(i), axis=ax).get()
    assert got.dtype == np.int64 and np.array_equal(got, np.cumsum(i, axis=ax))
    x = _f32(shape, 6)
    gf = cp.cumsum(cp.array(x), axis=ax).get()
    want = np.cumsum(x.astype(np.float64), axis=ax)
    assert gf.dtype == np.float32
    assert np.allclose(gf, want, rtol=1e-5, atol=1e-3)
    p = (1.0 + 0.001 * _f32(shape, 7)).astype(np.float32)
    gp = cp.cumprod(cp.array(p), axis=ax).get()
    assert np.allclose(gp, np.cumprod(p.astype(np.float64), axis=ax), rtol=1e-5)


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.float16, np.int16, np.bool_,
                                   np.int64])
@pytest.mark.parametrize("shape,perm", [((1000, 777), (1, 0)), ((64, 64), (1, 0)),
                                        ((5, 130, 70), (0, 2, 1)), ((70, 5, 130), (2, 1, 0)),
                                        ((33, 17, 3), (1, 0, 2)), ((300, 20), (1, 0)),
                                        ((192, 256), (1, 0)), ((3, 128, 192), (0, 2, 1)),
                                        ((128, 3, 256), (2, 1, 0))])
def test_transpose_copies(dtype, shape, perm):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(shape) * 100).astype(dtype)
    cx = cp.array(x)
    got = cx.transpose(perm).copy().get()
    want = np.ascontiguousarray(x.transpose(perm))
    assert got.dtype == want.dtype and np.array_equal(got.view(np.uint8), want.view(np.uint8))
    # with a cast and a sliced (offset, non-unit) source
    sl = cx[1:, ::2] if len(shape) == 2 else cx[1:]
    nsl = x[1:, ::2] if len(shape) == 2 else x[1:]
    inv = tuple(range(nsl.ndim))[::-1]
    got2 = sl.transpose(inv).astype(np.float32).get()
    assert np.array_equal(got2, np.ascontiguousarray(nsl.transpose(inv)).astype(np.float32))


@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.float16, np.int16, np.int32])
def test_transpose_copies_whole_tiles(dtype):
    """Whole 64 x 64 tiles with 16-byte aligned rows take the vector
    transpose (one 16-byte access per lane on both sides): sliced views whose
    offsets and strides keep that alignment, reversed and stepped views, a
    batch dimension, and a view whose offset breaks it (the element kernel)."""
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((320, 512)) * 100).astype(dtype)
    cx = cp.array(x)
    for sl in ((slice(64, None), slice(128, None)), (slice(None), slice(None, None, 2)),
               (slice(None, None, -1), slice(None)), (slice(1, 257), slice(None)),
               (slice(None), slice(8, 392))):
        got = cx[sl].T.copy().get()
        assert np.array_equal(got.view(np.uint8), np.ascontiguousarray(x[sl].T).view(np.uint8)), sl
    b = (rng.standard_normal((4, 128, 192)) * 100).astype(dtype)
    got = cp.ascontiguousarray(cp.array(b).transpose(2, 0, 1)).get()
    assert np.array_equal(got.view(np.uint8), np.ascontiguousarray(b.transpose(2, 0, 1)).view(np.uint8))


def test_device_creation_large():
    n = 1 << 18
    for dt in (np.float32, np.int64, np.float16, np.bool_):
        z = cp.zeros((n,), dtype=dt)
        o = cp.ones((4, n // 4), dtype=dt)
        assert z._np_data is None and o._np_data is None  # created in HBM
        assert np.array_equal(z.get(), np.zeros(n, dt))
        assert np.array_equal(o.get(), np.ones((4, n // 4), dt))
    f = cp.full((512, 512), 3.25)
    assert f.dtype == np.float64 or f.dtype == np.float32
    assert np.array_equal(f.get(), np.full((512, 512), 3.25, dtype=f.dtype))
    e = cp.empty((1 << 17,), dtype=np.int32)
    e.fill(7)
    assert np.array_equal(e.get(), np.full(1 << 17, 7, np.int32))
    small = cp.zeros((10,))
    assert small._np_data is not None  # small arrays stay on the host until used
    r = cp.zeros((1 << 17,)) + cp.arange(1 << 17, dtype=np.float32)
    assert np.array_equal(r.get(), np.arange(1 << 17, dtype=np.float32))


@pytest.mark.parametrize("src,dst", [(np.float32, np.float16), (np.float16, np.float32),
                                     (np.float32, np.float64), (np.int32, np.int64),
                                     (np.float64, np.int32), (np.bool_, np.float32),
                                     (np.int16, np.uint16), (np.float32, np.float32)])
@pytest.mark.parametrize("n", [1, 1000, 65536 + 7, (1 << 20) + 3])
def test_contiguous_casts(src, dst, n):
    """Vector (16-byte) contiguous cast path and its element-wise tail; an
    offset view takes the unaligned path."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 50).astype(src)
    cx = cp.array(x)
    cx._ensure_gpu()  # device-resident: the cast runs on the device
    with np.errstate(all="ignore"):
        want = x.astype(dst)
    got = cx.astype(dst).get()
    assert got.dtype == want.dtype and np.array_equal(got, want, equal_nan=True)
    if n > 3:
        got2 = cx[3:].astype(dst).get()
        assert np.array_equal(got2, want[3:], equal_nan=True)
