"""Seeded random matmul shapes, batch broadcasting, 1-D operands and views.

The reference's __matmul__ (ndarray.py:1398-1450) and linalg_top.matmul
(linalg_top.py:94-111) follow np.matmul's shape rules; its tests compare
with NumPy (tests/test_ndarray.py:528-556, tests/test_linalg.py:571-592).
Each case draws M, N, K from odd and power-of-two extents, optional batch
dimensions that broadcast, 1-D operands, transposed views and a dtype, and
compares with NumPy:

* integer results bit for bit (NumPy's integer matmul wraps);
* float results elementwise within the rounding-error bound of any
  summation order, 2 K u (|A| |B|) + u_out |C| (u the unit roundoff of the
  accumulator: float32 for float16 / float32 inputs, float64 for float64;
  u_out that of the output dtype), against the float64 product."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu

EXTENTS = [1, 2, 3, 7, 16, 31, 64, 100, 129, 256, 257, 512, 1000]
DTYPES = [np.float32, np.float32, np.float16, np.float64, np.int32, np.int64]


def _draw(rng, shape, dtype):
    if np.dtype(dtype).kind == "f":
        return rng.standard_normal(shape).astype(dtype)
    return rng.integers(-50, 50, shape).astype(dtype)


def _case(seed):
    rng = np.random.default_rng(9000 + seed)
    while True:
        M, N, K = (int(rng.choice(EXTENTS)) for _ in range(3))
        r = rng.random()
        if r < 0.4:
            ba, bb = (), ()
        elif r < 0.6:
            b = int(rng.integers(1, 5)); ba, bb = (b,), (b,)
        elif r < 0.75:
            b1, b2 = int(rng.integers(1, 4)), int(rng.integers(1, 4)); ba, bb = (b1, 1), (1, b2)
        else:
            b = int(rng.integers(1, 4)); ba, bb = (b,), ()
        batch = int(np.prod(np.broadcast_shapes(ba, bb)))
        if batch * M * N * K <= 3e8:
            break
    dtype = DTYPES[int(rng.integers(len(DTYPES)))]
    a1 = not ba and rng.random() < 0.15           # 1-D operands
    b1 = not bb and rng.random() < 0.15
    ta = rng.random() < 0.3                       # operand given as a transposed view
    tb = rng.random() < 0.3
    a_shape = (K,) if a1 else ba + ((K, M) if ta else (M, K))
    b_shape = (K,) if b1 else bb + ((N, K) if tb else (K, N))
    A = _draw(rng, a_shape, dtype)
    B = _draw(rng, b_shape, dtype)
    return A, B, (not a1) and ta, (not b1) and tb


def _t(x, flag):
    return x.swapaxes(-1, -2) if flag else x


@pytest.mark.parametrize("seed", range(128))
def test_random_matmul(seed):
    A, B, ta, tb = _case(seed)
    ha, hb = _t(A, ta), _t(B, tb)
    want = np.matmul(ha, hb)
    da, db = _t(cp.array(A), ta), _t(cp.array(B), tb)
    got = (da @ db) if seed % 2 else cp.matmul(da, db)
    got = np.asarray(got.get() if hasattr(got, "get") else got)   # 1-D @ 1-D: a scalar
    assert got.shape == want.shape and got.dtype == want.dtype, (got.shape, want.shape,
                                                                 got.dtype, want.dtype)
    if want.dtype.kind != "f":
        np.testing.assert_array_equal(got, want)
        return
    K = ha.shape[-1]
    a64, b64 = ha.astype(np.float64), hb.astype(np.float64)
    exact = np.matmul(a64, b64)
    mag = np.matmul(np.abs(a64), np.abs(b64))
    u_acc = 2.0 ** -53 if want.dtype == np.float64 else 2.0 ** -24
    u_out = float(np.finfo(want.dtype).eps) / 2
    tol = 2 * K * u_acc * mag + u_out * np.abs(exact) + np.finfo(want.dtype).tiny
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= tol), float(np.max(err / tol))
