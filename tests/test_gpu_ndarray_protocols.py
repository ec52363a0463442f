"""NumPy functions on device arrays dispatch to the device library
(__array_function__, as the reference's ndarray.py:2722-2729), and the
remaining ndarray methods (view, byteswap, partition, resize, round,
diagonal, trace, ptp, repeat, choose, itemset, tobytes, copy protocols,
__contains__, @=, reflected divmod, pickling) agree with NumPy's."""
import copy
import pickle

import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu


def _h(a):
    return a.get() if hasattr(a, "get") else np.asarray(a)


def _same(got, want):
    got, want = _h(got), np.asarray(want)
    assert got.shape == want.shape and got.dtype == want.dtype, (got.shape, want.shape, got.dtype, want.dtype)
    assert np.array_equal(got, want, equal_nan=True), (got, want)


def test_array_function_dispatch():
    x = np.arange(24, dtype=np.float32).reshape(4, 6) - 7.5
    d = cp.array(x)
    r = np.concatenate([d, d])
    assert isinstance(r, cp.ndarray)
    _same(r, np.concatenate([x, x]))
    _same(np.sum(d, axis=0), np.sum(x, axis=0))
    _same(np.where(d > 0, d, 0), np.where(x > 0, x, 0))
    _same(np.clip(d, -1, 1), np.clip(x, -1, 1))
    _same(np.sort(d, axis=1), np.sort(x, axis=1))
    _same(np.argmax(d, axis=1), np.argmax(x, axis=1))
    _same(np.unique(d), np.unique(x))
    _same(np.transpose(d), np.transpose(x))
    _same(np.reshape(d, (6, 4)), np.reshape(x, (6, 4)))
    _same(np.einsum("ij->j", d), np.einsum("ij->j", x))
    _same(np.tile(d, (2, 1)), np.tile(x, (2, 1)))
    np.testing.assert_allclose(_h(np.linalg.norm(d)), np.linalg.norm(x), rtol=1e-6)
    assert isinstance(np.linalg.inv(cp.array(np.eye(3))), cp.ndarray)
    with pytest.raises(NotImplementedError):
        np.fft.fft(d)
    _same(np.fft.fftshift(d), np.fft.fftshift(x))


def test_view_byteswap():
    f = np.array([1.5, -2.0, np.inf, 3.25], dtype=np.float32)
    d = cp.array(f)
    _same(d.view(np.int32), f.view(np.int32))
    _same(d.view(np.uint16), f.view(np.uint16))
    i16 = np.arange(8, dtype=np.int16) * 1000 - 3000
    _same(cp.array(i16).view(np.int32), i16.view(np.int32))
    _same(cp.array(i16.reshape(2, 4)).view(np.uint64), i16.reshape(2, 4).view(np.uint64))
    v = d.view()
    v[0] = 9.0
    assert float(d[0]) == 9.0
    for arr in (i16, np.arange(6, dtype=np.int32) * 123457 - 9, np.linspace(-3, 7, 5),
                np.arange(5, dtype=np.uint64) * 0x0102030405060708):
        _same(cp.array(arr).byteswap(), arr.byteswap())
    with pytest.raises(ValueError):
        cp.array(np.zeros((3, 3), np.float32))[:, :2].view(np.float64)


def test_methods():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 6)).astype(np.float32)
    d = cp.array(x)
    p = cp.array(x.copy())
    p.partition(2, axis=1)
    assert np.array_equal(_h(p)[:, 2], np.sort(x, axis=1)[:, 2])
    ap = _h(d.argpartition(3))
    assert np.array_equal(np.take_along_axis(x, ap, axis=-1)[:, 3], np.sort(x, axis=-1)[:, 3])
    _same(d.round(2), x.round(2))
    _same(d.diagonal(1), x.diagonal(1).copy())
    np.testing.assert_allclose(_h(d.trace()), x.trace(), rtol=1e-6)
    _same(d.ptp(axis=0), np.ptp(x, axis=0))
    _same(d.repeat(2, axis=0), x.repeat(2, axis=0))
    idx = cp.array(np.array([0, 1, 0], dtype=np.int64))
    _same(idx.choose([cp.array(x[0, :3]), cp.array(x[1, :3])]), np.array([0, 1, 0]).choose([x[0, :3], x[1, :3]]))
    r = cp.array(x.copy())
    r.resize((3, 12))
    h = x.copy()
    h.resize((3, 10))
    r2 = cp.array(x.copy())
    r2.resize(3, 10)
    _same(r2, h)
    h12 = x.copy()
    h12.resize((3, 12))
    _same(r, h12)
    g = cp.array(np.zeros(8, np.float32))
    g.resize((12,))
    _same(g, np.zeros(12, np.float32))
    s = cp.array(np.zeros((2, 3), np.int32))
    s.itemset(4, 7)
    s.itemset(0, 1, 5)
    _same(s, np.array([[0, 5, 0], [0, 7, 0]], np.int32))
    assert d.tobytes() == x.tobytes()
    assert float(x[2, 3]) in d and 1e9 not in d
    c1, c2 = copy.copy(d), copy.deepcopy(d)
    c1[0, 0] = 100.0
    _same(d, x)
    _same(c2, x)
    with pytest.raises(ValueError):
        del d[0]
    m = cp.array(np.eye(3, dtype=np.float32) * 2)
    m @= cp.array(np.full((3, 3), 0.5, np.float32))
    _same(m, (np.eye(3, dtype=np.float32) * 2) @ np.full((3, 3), 0.5, np.float32))
    qi = cp.array(np.array([3, 4, 5], np.int32))
    q, rr = divmod(17, qi)
    _same(q, 17 // np.array([3, 4, 5], np.int32))
    _same(rr, 17 % np.array([3, 4, 5], np.int32))
    assert isinstance(d.data, int) and d.data != 0
    _same(pickle.loads(pickle.dumps(d)), x)
    assert d.to_device("gpu") is d
    _same(d.conj(), x)


def test_fft_namespace():
    for n, d in ((8, 1.0), (9, 0.1), (1, 2.0)):
        np.testing.assert_array_equal(_h(cp.fft.fftfreq(n, d)), np.fft.fftfreq(n, d))
        np.testing.assert_array_equal(_h(cp.fft.rfftfreq(n, d)), np.fft.rfftfreq(n, d))
    x = np.arange(30, dtype=np.float32).reshape(5, 6)
    for axes in (None, 0, 1, (0, 1)):
        _same(cp.fft.fftshift(cp.array(x), axes=axes), np.fft.fftshift(x, axes=axes))
        _same(cp.fft.ifftshift(cp.array(x), axes=axes), np.fft.ifftshift(x, axes=axes))
    with pytest.raises(NotImplementedError):
        cp.fft.fft(cp.array(x))
