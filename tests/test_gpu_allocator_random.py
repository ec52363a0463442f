"""Seeded random allocation / release sequences through the caching
allocator.

The reference pools Metal buffers by size and releases them when the
Python wrapper goes away (_metal_backend.py:23-372, _BufferPool).  Here the
device memory comes from a stream-ordered caching allocator (mmp_alloc /
mmp_free, best fit over the cached blocks).  Each case runs a random
sequence of array creations (1 byte to 48 MiB, uploads and device fills),
device writes, releases and re-reads; every live array must keep its own
contents whatever blocks are reused around it, and once everything is
released the in-use byte count must return to where it started."""
import gc

import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd._backend import HipBackend

pytestmark = pytest.mark.gpu

SIZES = [1, 3, 64, 1000, 4096, 65537, 1 << 20, (1 << 20) + 7, 3 << 20, 17 << 20, 48 << 20]


@pytest.mark.parametrize("seed", range(24))
def test_random_alloc_release(seed):
    rng = np.random.default_rng(39000 + seed)
    be = HipBackend()
    gc.collect()
    cp.synchronize()
    base_in_use, _ = be.memory_stats()
    live = {}                                  # name -> (device array, expected host copy)
    for step in range(60):
        r = rng.random()
        if r < 0.45 or not live:
            n = int(rng.choice(SIZES)) // 4 or 1
            if rng.random() < 0.5:
                h = rng.integers(-1000, 1000, n).astype(np.int32)
                d = cp.array(h)
            else:
                v = int(rng.integers(-1000, 1000))
                d = cp.full((n,), v, dtype=np.int32)
                h = np.full(n, v, np.int32)
            live[step] = (d, h)
        elif r < 0.7:                          # release one
            k = list(live)[int(rng.integers(len(live)))]
            del live[k]
            if rng.random() < 0.5:
                gc.collect()
        elif r < 0.85:                         # a device write into one
            k = list(live)[int(rng.integers(len(live)))]
            d, h = live[k]
            d += 3
            live[k] = (d, h + np.int32(3))
        else:                                  # read one back
            k = list(live)[int(rng.integers(len(live)))]
            d, h = live[k]
            np.testing.assert_array_equal(d.get(), h)
    for d, h in live.values():
        np.testing.assert_array_equal(d.get(), h)
    live.clear()
    d = h = None                               # the loop variables held the last array
    gc.collect()
    cp.synchronize()
    in_use, cached = be.memory_stats()
    assert in_use == base_in_use, (in_use, base_in_use)
    if seed % 6 == 5:
        be.empty_cache()
        assert be.memory_stats()[1] == 0
