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


@pytest.mark.parametrize("nbytes", [1, 15, 4096, (32 << 10) - 4, 32 << 10, (32 << 10) + 4,
                                    (48 << 10) - 4, 48 << 10, (48 << 10) + 4, 200_000])
@pytest.mark.parametrize("src_off", [0, 4, 3])
def test_d2h_by_size_source_offset_and_destination(nbytes, src_off):
    """mmp_d2h through the C ABI at the sizes where its route changes (the
    polled copy kernel below 32 KiB, and below 48 KiB into pageable
    memory; DMA above), from aligned and unaligned device addresses, into
    pageable and page-locked host memory, twice in a row with new data."""
    be = HipBackend()
    lib = be._lib
    g = np.random.default_rng(nbytes + src_off)
    dev = be.create_buffer(nbytes + 16, np.uint8)
    for rep in range(2):
        h = g.integers(0, 256, nbytes + 16, dtype=np.uint8)
        be.write_buffer(dev, 0, h)
        pageable = np.zeros(nbytes, np.uint8)
        assert lib.mmp_d2h(pageable.ctypes.data, dev.ptr + src_off, nbytes) == 0
        np.testing.assert_array_equal(pageable, h[src_off:src_off + nbytes])
        locked = be.host_empty((nbytes,), np.uint8)
        locked[:] = 0
        assert lib.mmp_d2h(locked.ctypes.data, dev.ptr + src_off, nbytes) == 0
        np.testing.assert_array_equal(locked, h[src_off:src_off + nbytes])
