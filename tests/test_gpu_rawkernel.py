"""RawKernel on the GPU: the reference's tests/test_rawkernel.py cases with
the kernels written in HIP C++ (the reference's are MSL).  Grid = total
threads, exactly that many run (partial last workgroup)."""
import numpy as np
import numpy.testing as npt
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd import RawKernel

pytestmark = pytest.mark.gpu

DBL_F32 = r'''
extern "C" __global__ void dbl(const float* a, float* out) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  out[i] = a[i] * 2.0f;
}'''
DBL_I32 = r'''
extern "C" __global__ void dbl_int(const int* a, int* out) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  out[i] = a[i] * 2;
}'''
DBL_F16 = r'''
extern "C" __global__ void dbl_half(const _Float16* a, _Float16* out) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  out[i] = a[i] * (_Float16)2.0f;
}'''
DBL_U32 = r'''
extern "C" __global__ void dbl_uint(const unsigned* a, unsigned* out) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  out[i] = a[i] * 2u;
}'''
ADD = r'''
extern "C" __global__ void add_k(const float* a, const float* b, float* out) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  out[i] = a[i] + b[i];
}'''
SUM8 = r'''
extern "C" __global__ void sum8(const float* a, const float* b, const float* c, const float* d,
                                const float* e, const float* f, const float* g, const float* h,
                                float* out) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  out[i] = a[i] + b[i] + c[i] + d[i] + e[i] + f[i] + g[i] + h[i];
}'''
GRID2D = r'''
extern "C" __global__ void fill2d(int* out, int width) {
  unsigned x = blockIdx.x * blockDim.x + threadIdx.x;
  unsigned y = blockIdx.y * blockDim.y + threadIdx.y;
  out[y * width + x] = (int)(y * 1000 + x);
}'''
MANGLED = r'''
__global__ void scale3(float* a) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  a[i] *= 3.0f;
}'''


def test_float32():
    a = cp.array([1, 2, 3], dtype=np.float32)
    out = cp.empty(3, dtype=np.float32)
    RawKernel(DBL_F32, "dbl")(3, (a, out))
    npt.assert_allclose(out.get(), [2, 4, 6])


def test_int32_float16_uint32():
    a = cp.array([1, 2, 3], dtype=np.int32)
    out = cp.empty(3, dtype=np.int32)
    RawKernel(DBL_I32, "dbl_int")(3, (a, out))
    npt.assert_array_equal(out.get(), [2, 4, 6])
    h = cp.array([1, 2, 3], dtype=np.float16)
    oh = cp.empty(3, dtype=np.float16)
    RawKernel(DBL_F16, "dbl_half")(3, (h, oh))
    npt.assert_allclose(oh.get(), [2, 4, 6], rtol=1e-2)
    u = cp.array([1, 2, 3], dtype=np.uint32)
    ou = cp.empty(3, dtype=np.uint32)
    RawKernel(DBL_U32, "dbl_uint")(3, (u, ou))
    npt.assert_array_equal(ou.get(), [2, 4, 6])


@pytest.mark.parametrize("grid", [4, (4,), (4, 1), (4, 1, 1)])
def test_grid_forms(grid):
    a = cp.array([1, 2, 3, 4], dtype=np.float32)
    out = cp.empty(4, dtype=np.float32)
    RawKernel(DBL_F32, "dbl")(grid, (a, out))
    npt.assert_allclose(out.get(), [2, 4, 6, 8])


def test_4_tuple_raises():
    k = RawKernel(DBL_F32, "dbl")
    with pytest.raises(ValueError, match="1-3"):
        k((1, 1, 1, 1), (cp.array([1.0]), cp.empty(1, dtype=np.float32)))


def test_exact_thread_count_leaves_tail_untouched():
    """Exactly `grid` threads run: elements past the grid keep their value."""
    n, pad = 1000, 300
    a = cp.array(np.arange(n + pad, dtype=np.float32))
    out = cp.array(np.full(n + pad, -7.0, np.float32))
    RawKernel(DBL_F32, "dbl")(n, (a, out))
    got = out.get()
    npt.assert_array_equal(got[:n], 2 * np.arange(n, dtype=np.float32))
    assert np.all(got[n:] == -7.0)


BLOCKDIM = r'''
extern "C" __global__ void block_extent(int* out) {
  unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  out[i] = (int)(blockDim.x * 1000 + gridDim.x);
}'''


def test_prime_thread_count_runs_in_full_workgroups():
    """A prime count has no divisor that fills a wave64: it runs in
    256-thread workgroups with a partial last one (blockDim stays 256 there
    too), exactly n threads, and the tail past n is untouched."""
    n, pad = 1_000_003, 512
    a = cp.array(np.arange(n + pad, dtype=np.float32))
    out = cp.array(np.full(n + pad, -7.0, np.float32))
    RawKernel(DBL_F32, "dbl")(n, (a, out))
    got = out.get()
    npt.assert_array_equal(got[:n], 2 * np.arange(n, dtype=np.float32))
    assert np.all(got[n:] == -7.0)
    ext = cp.array(np.full(n + pad, -1, np.int32))
    RawKernel(BLOCKDIM, "block_extent")(n, (ext,))
    got = ext.get()
    assert np.all(got[:n] == 256 * 1000 + (n + 255) // 256)
    assert np.all(got[n:] == -1)


def test_prime_2d_grid():
    w, h = 1009, 7
    o = cp.array(np.full(1024 * 8 + 4096, -1, np.int32))
    RawKernel(GRID2D, "fill2d")((w, h), (o, np.int32(w)))
    got = o.get()
    yy, xx = np.mgrid[0:h, 0:w]
    npt.assert_array_equal(got[:w * h].reshape(h, w), yy * 1000 + xx)
    assert np.all(got[w * h:] == -1)


def test_eight_buffers_reuse_two_kernels():
    bufs = [cp.array([float(i + 1)], dtype=np.float32) for i in range(8)]
    out = cp.empty(1, dtype=np.float32)
    RawKernel(SUM8, "sum8")(1, (*bufs, out))
    npt.assert_allclose(out.get(), [36.0])
    k = RawKernel(DBL_F32, "dbl")
    for v in [1, 5, 10]:
        a = cp.array([v], dtype=np.float32)
        o = cp.empty(1, dtype=np.float32)
        k(1, (a, o))
        npt.assert_allclose(o.get(), [2 * v])
    a = cp.array([1, 2, 3], dtype=np.float32)
    b = cp.array([4, 5, 6], dtype=np.float32)
    o2 = cp.empty(3, dtype=np.float32)
    RawKernel(ADD, "add_k")(3, (a, b, o2))
    npt.assert_allclose(o2.get(), [5, 7, 9])


def test_large_and_2d_grid_and_scalar_arg():
    n = 100_000
    a = cp.array(np.ones(n, dtype=np.float32))
    out = cp.empty(n, dtype=np.float32)
    RawKernel(DBL_F32, "dbl")(n, (a, out))
    npt.assert_allclose(out.get(), np.full(n, 2.0))
    w, h = 37, 23
    # padded so that even whole 16x16 workgroups would stay inside the buffer
    o = cp.array(np.full(48 * 32 + 64, -1, np.int32))
    RawKernel(GRID2D, "fill2d")((w, h), (o, np.int32(w)))
    got = o.get()
    yy, xx = np.mgrid[0:h, 0:w]
    npt.assert_array_equal(got[:w * h].reshape(h, w), yy * 1000 + xx)
    assert np.all(got[w * h:] == -1)


def test_writes_visible_to_lazy_consumers_and_mangled_name():
    a = cp.array(np.ones(64, np.float32))
    before = a + 1.0                      # lazy, must see the old contents
    RawKernel(MANGLED, "scale3")(64, (a,))
    npt.assert_allclose(before.get(), 2.0)
    npt.assert_allclose(a.get(), 3.0)


def test_metal_source_rejected():
    with pytest.raises(TypeError, match="HIP"):
        RawKernel("#include <metal_stdlib>\nkernel void k(device float* a [[buffer(0)]]) {}", "k")
