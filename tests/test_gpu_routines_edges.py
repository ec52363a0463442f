"""Edge cases of the composed routines against NumPy: empty inputs,
zero-width pads, size-1 axes, scalar operands and degenerate shapes."""
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
    assert got.shape == want.shape and got.dtype == want.dtype, (got.shape, want.shape, got.dtype, want.dtype)
    assert np.array_equal(got, want, equal_nan=True), (got, want)


def test_empty_and_degenerate():
    e = np.zeros((0,), np.float32)
    _same(cp.isin(cp.array(e), cp.array(np.array([1.0], np.float32))), np.isin(e, np.array([1.0], np.float32)))
    _same(cp.union1d(cp.array(e), cp.array(np.array([3.0, 1.0], np.float32))),
          np.union1d(e, np.array([3.0, 1.0], np.float32)))
    _same(cp.bincount(cp.array(np.zeros(0, np.int32)), minlength=3), np.bincount(np.zeros(0, np.int32), minlength=3))
    _same(cp.histogram(cp.array(e), bins=3)[0], np.histogram(e, bins=3)[0])
    _same(cp.pad(cp.array(np.zeros((0, 3), np.float32)), ((1, 1), (0, 0))),
          np.pad(np.zeros((0, 3), np.float32), ((1, 1), (0, 0))))
    a = np.arange(6, dtype=np.int32).reshape(2, 3)
    _same(cp.pad(cp.array(a), 0), np.pad(a, 0))
    _same(cp.pad(cp.array(a), ((0, 0), (2, 0)), mode="edge"), np.pad(a, ((0, 0), (2, 0)), mode="edge"))
    _same(cp.pad(cp.array(a[:, :1]), 3, mode="reflect"), np.pad(a[:, :1], 3, mode="reflect"))
    _same(cp.delete(cp.array(a), [], axis=1), np.delete(a, [], axis=1))
    _same(cp.insert(cp.array(np.zeros(0, np.int32)), 0, 5), np.insert(np.zeros(0, np.int32), 0, 5))
    _same(cp.einsum("i->", cp.array(np.zeros(0, np.float32))), np.einsum("i->", np.zeros(0, np.float32)))
    _same(cp.einsum("ij,jk->ik", cp.array(np.ones((2, 0))), cp.array(np.ones((0, 3)))),
          np.einsum("ij,jk->ik", np.ones((2, 0)), np.ones((0, 3))))
    _same(cp.trim_zeros(cp.array(np.zeros(4, np.int32))), np.trim_zeros(np.zeros(4, np.int32)))
    _same(cp.unique_values(cp.array(np.zeros(0, np.int32))), np.unique_values(np.zeros(0, np.int32)))
    _same(cp.resize(cp.array(np.zeros(0, np.float32)), (2, 2)), np.resize(np.zeros(0, np.float32), (2, 2)))
    _same(cp.convolve(cp.array(np.array([2.0])), cp.array(np.array([3.0, 4.0]))),
          np.convolve(np.array([2.0]), np.array([3.0, 4.0])))
    _same(cp.interp(cp.array(np.array([0.5, 2.0])), cp.array(np.array([0.0, 1.0])), cp.array(np.array([5.0, 7.0]))),
          np.interp(np.array([0.5, 2.0]), np.array([0.0, 1.0]), np.array([5.0, 7.0])))
    _same(cp.packbits(cp.array(np.zeros(0, np.bool_))), np.packbits(np.zeros(0, np.bool_)).astype(np.uint16))
    _same(cp.digitize(cp.array(np.array([1.0, 5.0])), cp.array(np.array([2.0]))),
          np.digitize(np.array([1.0, 5.0]), np.array([2.0])))


def test_scalars_and_size_one():
    _same(cp.round(cp.array(np.float32(2.5))), np.round(np.float32(2.5)))
    _same(cp.isclose(cp.array(np.array([1.0])), 1.0), np.isclose(np.array([1.0]), 1.0))
    _same(cp.nan_to_num(cp.array(np.array(np.nan, np.float32))), np.nan_to_num(np.array(np.nan, np.float32)))
    x = np.array([[3.0]])
    _same(cp.linalg.inv(cp.array(x)), np.linalg.inv(x))
    # NumPy's det goes through log / exp (2.9999999999999996 here); the
    # device multiplies the pivots
    np.testing.assert_allclose(_h(cp.linalg.det(cp.array(x))), np.linalg.det(x), rtol=1e-15)
    _same(cp.linalg.cholesky(cp.array(x)), np.linalg.cholesky(x))
    _same(cp.linalg.eigvalsh(cp.array(x)), np.linalg.eigvalsh(x))
    _same(cp.linalg.svd(cp.array(x), compute_uv=False), np.linalg.svd(x, compute_uv=False))
    _same(cp.linalg.matrix_power(cp.array(x), 3), np.linalg.matrix_power(x, 3))
    _same(cp.gradient(cp.array(np.array([1.0, 4.0]))), np.gradient(np.array([1.0, 4.0])))
    _same(cp.cumulative_sum(cp.array(np.array([], np.int32)), include_initial=True),
          np.cumulative_sum(np.array([], np.int32), include_initial=True))


def test_unique_counting_path():
    # integer inputs of >= 2^16 elements with a value range < 2^22 are counted
    rng = np.random.default_rng(77)
    for dt, lo, hi in ((np.int32, -500, 500), (np.int64, 10 ** 12, 10 ** 12 + 3000), (np.uint16, 0, 60000),
                       (np.int16, -3, 3), (np.uint32, 7, 8)):
        x = rng.integers(lo, hi, 1 << 17).astype(dt)
        _same(cp.unique(cp.array(x)), np.unique(x))
        g, c = cp.unique(cp.array(x), return_counts=True)
        wv, wc = np.unique(x, return_counts=True)
        _same(g, wv)
        _same(c, wc)
    # full-range int16 (hi - lo > 32767 wraps in int16) and uint64 values
    # above the int64 range in a small window
    full16 = rng.integers(-32768, 32767, 1 << 17, endpoint=True).astype(np.int16)
    big_u64 = (np.uint64(2 ** 64 - 5000) + rng.integers(0, 4000, 1 << 17).astype(np.uint64))
    for x in (full16, big_u64):
        g, c = cp.unique(cp.array(x), return_counts=True)
        wv, wc = np.unique(x, return_counts=True)
        _same(g, wv)
        _same(c, wc)
        _same(cp.unique(cp.array(x)), wv)
    wide = rng.integers(-2 ** 40, 2 ** 40, 1 << 17)               # range too wide: sorted path
    _same(cp.unique(cp.array(wide)), np.unique(wide))
