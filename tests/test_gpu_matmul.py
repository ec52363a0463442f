"""Matmul on the GPU (MFMA) against the oracle.  Bars (normwise, against a
float64 product of the same inputs): 1e-4 for float32, 1e-2 for float16,
1e-12 for float64; integer products bit-exact (wrapping, as NumPy)."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd.workloads import c4_inputs
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

TOL = {np.float32: 1e-4, np.float16: 1e-2, np.float64: 1e-12}


def _check(a, b, got, dtype):
    want = ref.matmul_f64(a, b)
    assert got.dtype == np.dtype(dtype)
    assert got.shape == want.shape
    err = ref.normwise_rel_error(got, want)
    assert err <= TOL[dtype], err
    # elementwise: |C - C_ref| <= tol * (|A| @ |B|)
    bound = np.matmul(np.abs(np.asarray(a, np.float64)), np.abs(np.asarray(b, np.float64)))
    assert np.all(np.abs(got.astype(np.float64) - want) <= TOL[dtype] * bound + 1e-30)


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.float64])
@pytest.mark.parametrize("mnk", [(128, 128, 64), (256, 384, 128), (65, 130, 47), (1, 1, 1),
                                 (300, 5, 700), (7, 257, 3)])
def test_matmul_2d(dtype, mnk):
    m, n, k = mnk
    g = np.random.default_rng(m * 7 + n)
    a = (g.standard_normal((m, k)) / np.sqrt(k)).astype(dtype)
    b = (g.standard_normal((k, n)) / np.sqrt(k)).astype(dtype)
    got = (cp.array(a) @ cp.array(b)).get()
    _check(a, b, got, dtype)


def test_matmul_mfma_layout_known_answer():
    """Integer-valued operands make every product exact in fp32, so the
    MFMA fragment layout (row / column / k mapping) must reproduce NumPy
    exactly."""
    g = np.random.default_rng(0)
    for dtype in (np.float32, np.float16, np.float64):
        a = g.integers(-3, 4, (128, 64)).astype(dtype)
        b = g.integers(-3, 4, (64, 128)).astype(dtype)
        got = (cp.array(a) @ cp.array(b)).get()
        assert np.array_equal(got.astype(np.float64), a.astype(np.float64) @ b.astype(np.float64)), dtype
    e = np.eye(128, dtype=np.float32)
    m = g.standard_normal((128, 128)).astype(np.float32)
    assert np.array_equal((cp.array(m) @ cp.array(e)).get(), m)
    assert np.array_equal((cp.array(e) @ cp.array(m)).get(), m)


@pytest.mark.parametrize("batch,m,n,k", [(1, 2048, 4096, 320), (2, 2048, 2048, 192),
                                         (1, 4096, 2048, 256), (1, 4096, 2048, 64)])
def test_matmul_f16_large_tile_exact(batch, m, n, k):
    """Products with at least 128 tiles of 256 x 256 take the large-tile
    float16 kernel (split A/B loading, swizzled LDS, swapped-operand
    epilogue, XCD tile remap; odd and even numbers of 64-deep slabs, and a
    single slab, through the two-stage pipeline).
    Operands in {-1, 0, 1} make every sum an integer of magnitude <= k, exact
    in fp32 and in the float16 output, so the whole result must equal
    NumPy's."""
    g = np.random.default_rng(k)
    a = g.integers(-1, 2, (batch, m, k)).astype(np.float16)
    b = g.integers(-1, 2, (batch, k, n)).astype(np.float16)
    got = (cp.array(a) @ cp.array(b)).get()
    want = np.matmul(a.astype(np.float32), b.astype(np.float32))
    assert got.dtype == np.float16 and np.array_equal(got.astype(np.float32), want)


def _exact_f32_product(batch, m, n, k, seed):
    g = np.random.default_rng(seed)
    a = g.integers(-3, 4, (batch, m, k)).astype(np.float32)
    b = g.integers(-3, 4, (batch, k, n)).astype(np.float32)
    got = (cp.array(a) @ cp.array(b)).get()
    assert np.array_equal(got, np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("batch,m,n,k", [(1, 128, 128, 32), (2, 256, 128, 96), (1, 384, 256, 160),
                                         (3, 128, 384, 1024), (1, 512, 640, 224), (1, 256, 128, 32),
                                         (2, 256, 256, 64), (1, 768, 128, 320), (300, 256, 128, 64)])
def test_matmul_f32_dma_exact(batch, m, n, k):
    """Float32 products with 128-divisible extents and 32-divisible k whose
    256-row tiles would leave CUs idle take the 128 x 128 global -> LDS copy
    kernel (one to 32 slabs of 32, batches).  Integer-valued operands make
    every product exact, so the result must equal NumPy's."""
    _exact_f32_product(batch, m, n, k, batch * 1000 + k)


# (tiles per CU, tile rows of 256, tile columns of 128, k): the batch is set
# so the 256 x 128 tiles fill whole rounds of the device's CUs.
@pytest.mark.parametrize("rounds,tm,tn,k", [(1, 1, 1, 32), (2, 1, 1, 32), (3, 1, 1, 64), (2, 1, 2, 96),
                                            (2, 2, 2, 160), (3, 3, 4, 320), (3, 6, 4, 96)])
def test_matmul_f32_persistent_exact(rounds, tm, tn, k):
    """Products whose 256 x 128 tiles fill whole rounds of the CUs take the
    persistent three-stage kernel: one workgroup per CU runs `rounds` tiles
    in one slab stream, so tile ends fall at every position of the
    three-slab loop (tiles of 1, 2, 3, 5 and 10 slabs; C stored after every
    slab with 1), tile counts divisible by 8 take the XCD ranges, and the
    four-row tile groups end with a group of two or three rows.
    Integer-valued operands make every product exact, so the result must
    equal NumPy's."""
    from macmetalpy_amd._backend import HipBackend
    cus = HipBackend().device_info()["cu_count"]
    per_b = tm * tn
    if (rounds * cus) % per_b:
        pytest.skip(f"{cus} CUs do not divide into whole products of {per_b} tiles")
    _exact_f32_product(rounds * cus // per_b, 256 * tm, 128 * tn, k, rounds * 100 + k)


# (tiles short of whole rounds, rounds, tile rows of 256, k)
@pytest.mark.parametrize("short,rounds,tm,k", [(6, 1, 1, 96), (2, 2, 1, 32), (8, 2, 1, 64),
                                               (8, 3, 1, 160), (6, 1, 2, 32)])
def test_matmul_f32_persistent_partial_round_exact(short, rounds, tm, k):
    """Tile counts a few short of whole rounds of the CUs (at least 97 % of
    the last round) also take the persistent kernel.  A count not divisible
    by 8 (250, 510 tiles on 256 CUs) is taken grid-stride by workgroup id;
    one divisible by 8 (504, 760) is cut into eight XCD ranges whose
    workgroups run uneven numbers of tiles (2 or 1, 3 or 2).  Integer-valued
    operands make every product exact, so the result must equal NumPy's."""
    from macmetalpy_amd._backend import HipBackend
    cus = HipBackend().device_info()["cu_count"]
    tiles = rounds * cus - short
    if tiles % tm or tiles * 100 < rounds * cus * 97:
        pytest.skip(f"{tiles} tiles on {cus} CUs do not make this case")
    _exact_f32_product(tiles // tm, 256 * tm, 128, k, tiles + k)


@pytest.mark.parametrize("batch,m,n,k,pad", [(1, 256, 128, 96, 32), (2, 512, 256, 128, 4),
                                             (1, 256, 384, 64, 128), (2, 128, 128, 64, 36)])
def test_matmul_f32_dma_row_strides(batch, m, n, k, pad):
    """mmp_matmul with row strides wider than the product (lda = k + pad,
    ldb = n + pad, ldc = n + 4) and batch strides of whole padded matrices:
    the copy kernels address every row from the row stride, not from k or
    n, and leave the padding of C untouched."""
    from macmetalpy_amd._backend import HipBackend
    from macmetalpy_amd._dtypes import dtype_code
    g = np.random.default_rng(m + n + k + pad)
    af = g.integers(-3, 4, (batch, m, k + pad)).astype(np.float32)
    bf = g.integers(-3, 4, (batch, k, n + pad)).astype(np.float32)
    cf = np.full((batch, m, n + 4), 7.0, np.float32)
    da, db, dc = (cp.array(x)._ensure_gpu() for x in (af, bf, cf))  # device-resident
    HipBackend().matmul(dtype_code(np.dtype(np.float32)), batch, m, n, k,
                        da._ptr, k + pad, m * (k + pad), db._ptr, n + pad, k * (n + pad),
                        dc._ptr, n + 4, m * (n + 4))
    got = dc.get()
    want = np.matmul(af[:, :, :k].astype(np.float64), bf[:, :, :n].astype(np.float64))
    assert np.array_equal(got[:, :, :n], want.astype(np.float32))
    assert np.all(got[:, :, n:] == 7.0)

@pytest.mark.parametrize("dtype", [np.int32, np.int64, np.int16, np.uint32])
def test_matmul_integer_exact(dtype):
    g = np.random.default_rng(1)
    a = g.integers(-1000 if np.dtype(dtype).kind == "i" else 0, 1000, (70, 300)).astype(dtype)
    b = g.integers(-1000 if np.dtype(dtype).kind == "i" else 0, 1000, (300, 45)).astype(dtype)
    got = (cp.array(a) @ cp.array(b)).get()
    want = np.matmul(a, b)
    assert got.dtype == want.dtype and np.array_equal(got, want)


def test_matmul_batched_broadcast_and_1d():
    g = np.random.default_rng(2)
    a = g.standard_normal((3, 128, 96)).astype(np.float32)
    b = g.standard_normal((3, 96, 64)).astype(np.float32)
    _check(a, b, cp.matmul(cp.array(a), cp.array(b)).get(), np.float32)
    _check(a, b, (cp.array(a) @ cp.array(b)).get(), np.float32)    # 3-D @ (NumPy semantics)
    b2 = g.standard_normal((96, 64)).astype(np.float32)              # broadcast B
    _check(a, b2, cp.matmul(cp.array(a), cp.array(b2)).get(), np.float32)
    a4 = g.standard_normal((2, 1, 40, 30)).astype(np.float32)
    b4 = g.standard_normal((3, 30, 20)).astype(np.float32)
    got = cp.matmul(cp.array(a4), cp.array(b4)).get()
    assert got.shape == (2, 3, 40, 20)
    assert ref.normwise_rel_error(got, ref.matmul_f64(a4, b4)) <= 1e-4
    v = g.standard_normal(96).astype(np.float32)
    m = g.standard_normal((96, 50)).astype(np.float32)
    assert ref.normwise_rel_error((cp.array(v) @ cp.array(m)).get(), v.astype(np.float64) @ m) <= 1e-5
    assert ref.normwise_rel_error((cp.array(m.T) @ cp.array(v)).get(), m.T.astype(np.float64) @ v) <= 1e-5
    # tests/test_error_handling.py:107-114: 1-D @ 1-D inner product
    x = np.arange(3, dtype=np.float32)
    assert float((cp.array(x) @ cp.array(x)).get()) == 5.0
    assert ref.normwise_rel_error(cp.linalg.matmul(cp.array(m.T), cp.array(m)).get(),
                                  m.T.astype(np.float64) @ m) <= 1e-4
    assert ref.normwise_rel_error(cp.dot(cp.array(m.T), cp.array(m)).get(),
                                  m.T.astype(np.float64) @ m) <= 1e-4


def test_matmul_shape_mismatch_message():
    # tests/test_error_handling.py:100-105
    with pytest.raises(ValueError, match="shape mismatch"):
        cp.zeros((2, 3), dtype=cp.float32) @ cp.zeros((4, 5), dtype=cp.float32)


@pytest.mark.parametrize("kind,dtype", [("f32", np.float32), ("f16", np.float16),
                                        ("batched", np.float32)])
def test_c4_full_size_whole(kind, dtype):
    """The three matmul configurations at full size (float32 4096^2,
    float16 8192^2, batched float32 64 x 1024^2), every element checked:
    normwise error against the float64 product of the same inputs, and each
    element within tol * (|A| @ |B|) of it."""
    print(f"c4 {kind} full size", flush=True)
    a, b = c4_inputs(kind)
    got = (cp.array(a) @ cp.array(b)).get()
    assert got.dtype == np.dtype(dtype) and got.shape == a.shape[:-1] + b.shape[-1:]
    _check(a, b, got, dtype)


def test_c4_f16_full_size_exact():
    """The float16 8192^3 shape with operands in {-1, 0, 1}: every sum is an
    integer of magnitude <= 8192, exact in the fp32 accumulators, so the
    whole 32 x 32 grid of 256 x 256 tiles (XCD tile remap included) must
    equal NumPy's float32 product rounded to float16."""
    print("c4 f16 8192^3 exact", flush=True)
    g = np.random.default_rng(8192)
    a = g.integers(-1, 2, (8192, 8192)).astype(np.float16)
    b = g.integers(-1, 2, (8192, 8192)).astype(np.float16)
    got = (cp.array(a) @ cp.array(b)).get()
    want = np.matmul(a.astype(np.float32), b.astype(np.float32)).astype(np.float16)
    assert got.dtype == np.float16 and np.array_equal(got, want)
