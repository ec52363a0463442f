"""ndarray.get() into page-locked host blocks (the reference's get(),
src/macmetalpy/ndarray.py:576-603, reads unified memory; here results of
32 KiB .. 1 GiB come back by DMA into cached pinned blocks)."""
import gc

import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd._backend import HipBackend, _PINNED_MAX, _PINNED_MIN, _PinnedBlock

pytestmark = pytest.mark.gpu


def _pinned(a):
    b = a
    while b is not None and not isinstance(b, _PinnedBlock):
        b = b.base if isinstance(b, np.ndarray) else None
    return b is not None


@pytest.mark.parametrize("n,dtype", [(1000, np.float32), (1 << 16, np.float32),
                                     (1 << 20, np.float64), ((1 << 20) + 3, np.int16),
                                     (3 << 20, np.int32), (_PINNED_MAX // 8, np.float64),
                                     (_PINNED_MAX // 8 + 1, np.float64)])
def test_get_values_and_backing(n, dtype):
    g = np.random.default_rng(n)
    h = (g.standard_normal(n) * 100).astype(dtype)
    d = cp.array(h)
    d._ensure_gpu()
    out = (d * 1).get()  # a device result (lazy, then materialised)
    assert out.dtype == h.dtype and out.shape == h.shape and out.flags.c_contiguous
    assert out.flags.writeable
    np.testing.assert_array_equal(out, h)
    assert _pinned(out) == (_PINNED_MIN <= h.nbytes <= _PINNED_MAX)
    out[0] = 7  # the caller owns the array
    assert out[0] == 7


def test_pinned_blocks_are_reused_and_outlive_the_device_array():
    d = cp.array(np.arange(1 << 20, dtype=np.float32))
    d._ensure_gpu()
    first = d.get()
    ptr = first.__array_interface__["data"][0]
    del first
    gc.collect()
    again = d.get()                      # the block just released comes back
    assert again.__array_interface__["data"][0] == ptr
    del d
    gc.collect()
    np.testing.assert_array_equal(again, np.arange(1 << 20, dtype=np.float32))
    views = [again[::2], again.reshape(1024, 1024)[3]]
    del again
    gc.collect()                         # views keep the block alive
    assert views[0][5] == 10.0 and views[1][0] == 3 * 1024


def test_strided_and_2d_views_come_back_contiguous():
    h = np.arange(512 * 256, dtype=np.float32).reshape(512, 256)
    d = cp.array(h)
    d._ensure_gpu()
    np.testing.assert_array_equal(d.T.get(), h.T)
    np.testing.assert_array_equal(d[::3, 1::2].get(), h[::3, 1::2])
    assert d.T.get().flags.c_contiguous
