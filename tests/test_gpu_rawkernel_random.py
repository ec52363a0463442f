"""Seeded random RawKernel grids: exactly the requested threads run.

The reference's RawKernel(src, name)(grid, args) launches ``grid`` threads
in total (Metal dispatchThreads, raw_kernel.py:26-62).  Each case draws a
1-, 2- or 3-D grid (prime extents, extents of one, sizes above and below
one workgroup, large 1-D counts) and runs a kernel in which every thread
adds one to the counter of its own (x, y, z) -- or to an overflow counter
if its index lies outside the grid, so no write leaves the buffers.  Every
counter must be exactly one and the overflow counter zero."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu

SRC = r"""
extern "C" __global__ void cover(int* count, int* extra, int gx, int gy, int gz) {
  const long long x = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long y = (long long)blockIdx.y * blockDim.y + threadIdx.y;
  const long long z = (long long)blockIdx.z * blockDim.z + threadIdx.z;
  if (x >= gx || y >= gy || z >= gz) { atomicAdd(extra, 1); return; }
  atomicAdd(&count[(z * gy + y) * gx + x], 1);
}
"""
EXTENTS = [1, 2, 3, 7, 63, 64, 65, 97, 255, 256, 257, 1000, 1009, 4096, 65537]
_KERNEL = None


def _kernel():
    global _KERNEL
    if _KERNEL is None:
        _KERNEL = cp.RawKernel(SRC, "cover")
    return _KERNEL


def _grid(seed):
    rng = np.random.default_rng(29000 + seed)
    nd = int(rng.integers(1, 4))
    while True:
        g = tuple(int(rng.choice(EXTENTS)) for _ in range(nd))
        if nd == 1 and rng.random() < 0.3:
            g = (int(rng.integers(1, 5_000_000)),)
        if int(np.prod(g)) <= 8_000_000:
            return g


@pytest.mark.parametrize("seed", range(60))
def test_random_grid_runs_each_thread_once(seed):
    g = _grid(seed)
    gx, gy, gz = (g + (1, 1))[:3]
    count = cp.zeros(gx * gy * gz, dtype=np.int32)
    extra = cp.zeros(1, dtype=np.int32)
    grid = g if seed % 3 else (g[0] if len(g) == 1 else g)
    _kernel()(grid, (count, extra, np.int32(gx), np.int32(gy), np.int32(gz)))
    c = count.get()
    assert int(extra.get()[0]) == 0, g
    assert c.min() == 1 and c.max() == 1, (g, int(np.sum(c != 1)))
