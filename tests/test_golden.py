"""Committed golden vectors (tests/golden/hot_path_vectors.npz, written by
tests/golden/make_golden.py from the oracle).

CPU tests: the oracle still reproduces every stored vector (a NumPy or
oracle change would show here), and the literals taken from the
reference's own tests hold.  GPU tests: the HIP path against the stored
vectors, to the parity bars of each operation (integers bit-exact; float
add, sqrt, abs, neg bit-exact; float32 transcendentals within 2 ULP of
NumPy; float32 sums and scans within 1e-5 of the float64-accumulated
result; matmul normwise 1e-4 float32, 1e-2 float16)."""
import os

import numpy as np
import pytest

from oracle import reference_cpu as ref

HERE = os.path.dirname(os.path.abspath(__file__))
G = np.load(os.path.join(HERE, "golden", "hot_path_vectors.npz"))
RTOL = 1e-5


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.dtype == b.dtype and a.shape == b.shape
    if a.dtype.kind == "f":
        both_nan = np.isnan(a) & np.isnan(b)
        assert np.all((a.view(f"u{a.itemsize}") == b.view(f"u{b.itemsize}")) | both_nan)
    else:
        assert np.array_equal(a, b)


def _rel(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)))


# ------------------------------------------------------------------- CPU
def test_oracle_reproduces_golden_vectors():
    a, b = G["floor_divide_i32/a"], G["floor_divide_i32/b"]
    _same(ref.floor_divide(a, b), G["floor_divide_i32/out"])
    _same(ref.mod(a, b), G["mod_i32/out"])
    x, y = G["f32/x"], G["f32/y"]
    _same(ref.binary("add_op", x, y), G["add_f32/out"])
    for op in ("sin_op", "exp_op", "log1p_op", "tanh_op", "sqrt_op", "abs_op", "neg_op"):
        _same(ref.unary(op, x), G[f"{op}_f32/out"])
    _same(ref.fused_elementwise(G["c1/x"]), G["c1/out"])
    np.testing.assert_allclose(ref.fusion_chain_f64(G["c5/x"], G["c5/r"]), G["c5/out_f64"],
                               rtol=1e-12)
    m = G["c3/m"]
    clean = np.where(np.isnan(m), 0.0, m).astype(np.float32)
    np.testing.assert_allclose(ref.sum_f64(clean, axis=1), G["sum_axis1/out_f64"], rtol=1e-12)
    _same(ref.argmax(m, axis=1).astype(np.int64), G["argmax_axis1/out"])
    _same(ref.cumsum(G["cumsum_i32/x"]), G["cumsum_i32/out"])
    np.testing.assert_allclose(ref.matmul_f64(G["matmul_f32/a"], G["matmul_f32/b"]),
                               G["matmul_f32/out_f64"], rtol=1e-12)


def test_reference_literals_and_invariants():
    # tests/test_math_ops.py:446-453 / tests/test_math_ext.py:302-307
    _same(np.mod(G["lit_mod/a"], G["lit_mod/b"]), G["lit_mod/out"])
    # tests/test_untested_math.py:227-232
    _same(np.floor_divide(G["lit_floordiv_f32/a"], G["lit_floordiv_f32/b"]),
          G["lit_floordiv_f32/out"])
    # floor_divide / mod: a == q*b + r, r has b's sign, |r| < |b| (b != 0)
    a = G["floor_divide_i32/a"].astype(np.int64)
    b = G["floor_divide_i32/b"].astype(np.int64)
    q = G["floor_divide_i32/out"].astype(np.int64)
    r = G["mod_i32/out"].astype(np.int64)
    nz = (b != 0) & ~((a == -2**31) & (b == -1))
    assert np.all(a[nz] == q[nz] * b[nz] + r[nz])
    assert np.all((r[nz] == 0) | (np.sign(r[nz]) == np.sign(b[nz])))
    assert np.all(np.abs(r[nz]) < np.abs(b[nz]))
    assert np.all(q[b == 0] == 0) and np.all(r[b == 0] == 0)
    # argmax: the planted tie (row 3, columns 17 and 400) and NaN (row 7, column 5)
    am = G["argmax_axis1/out"]
    assert am[3] == 17 and am[7] == 5
    # cumsum: last = sum, first differences = input
    ci, co = G["cumsum_i32/x"], G["cumsum_i32/out"]
    assert co.dtype == np.int64 and co[-1] == int(ci.astype(np.int64).sum())
    assert np.array_equal(np.diff(co), ci[1:].astype(np.int64))


# ------------------------------------------------------------------- GPU
@pytest.mark.gpu
def test_gpu_integer_and_exact_float_vectors():
    import macmetalpy_amd as cp
    a, b = cp.array(G["floor_divide_i32/a"]), cp.array(G["floor_divide_i32/b"])
    _same(cp.floor_divide(a, b).get(), G["floor_divide_i32/out"])
    _same(cp.mod(a, b).get(), G["mod_i32/out"])
    _same((a % b).get(), G["mod_i32/out"])
    _same(cp.mod(cp.array(G["lit_mod/a"]), cp.array(G["lit_mod/b"])).get(), G["lit_mod/out"])
    _same(cp.floor_divide(cp.array(G["lit_floordiv_f32/a"]),
                          cp.array(G["lit_floordiv_f32/b"])).get(), G["lit_floordiv_f32/out"])
    x, y = cp.array(G["f32/x"]), cp.array(G["f32/y"])
    _same((x + y).get(), G["add_f32/out"])
    _same(cp.sqrt(x).get(), G["sqrt_op_f32/out"])
    _same(cp.abs(x).get(), G["abs_op_f32/out"])
    _same((-x).get(), G["neg_op_f32/out"])


@pytest.mark.gpu
@pytest.mark.parametrize("name,op", [("sin", "sin_op"), ("exp", "exp_op"),
                                     ("log1p", "log1p_op"), ("tanh", "tanh_op")])
def test_gpu_transcendental_vectors(name, op):
    import macmetalpy_amd as cp
    got = getattr(cp, name)(cp.array(G["f32/x"])).get()
    want = G[f"{op}_f32/out"]
    assert got.dtype == np.float32
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert int(ref.ulp_distance(got, want).max()) <= 2


@pytest.mark.gpu
def test_gpu_fused_vectors():
    import macmetalpy_amd as cp
    x = cp.array(G["c1/x"])
    got = (cp.sqrt(cp.abs(x)) + cp.exp(-(x * x))).get()
    assert int(ref.ulp_distance(got, G["c1/out"]).max()) <= 4
    X, R = cp.array(G["c5/x"]), cp.array(G["c5/r"])
    z = cp.sum(cp.tanh(X * R + 1.0) * cp.exp(-cp.abs(X)) - cp.log1p(X * X), axis=1).get()
    assert _rel(z, G["c5/out_f64"]) <= RTOL


@pytest.mark.gpu
def test_gpu_reduction_and_scan_vectors():
    import macmetalpy_amd as cp
    m = G["c3/m"]
    clean = cp.array(np.where(np.isnan(m), 0.0, m).astype(np.float32))
    assert _rel(float(cp.sum(clean).get()), G["sum_all/out_f64"]) <= RTOL
    assert _rel(cp.sum(clean, axis=1).get(), G["sum_axis1/out_f64"]) <= RTOL
    assert _rel(cp.mean(clean, axis=1).get(), G["mean_axis1/out_f64"]) <= RTOL
    M = cp.array(m)
    _same(cp.argmax(M, axis=1).get().astype(np.int64), G["argmax_axis1/out"])
    assert cp.argmax(M) == int(G["argmax_all/out"])
    ones = cp.ones(int(G["lit_sum_ones/n"]), dtype=cp.float32)   # tests/test_edge_shapes.py:367-378
    assert float(cp.sum(ones).get()) == 1e6
    _same(cp.cumsum(cp.array(G["cumsum_i32/x"])).get(), G["cumsum_i32/out"])
    assert _rel(cp.cumsum(cp.array(G["cumsum_f32/x"])).get(), G["cumsum_f32/out_f64"]) <= RTOL


@pytest.mark.gpu
def test_gpu_matmul_vectors():
    import macmetalpy_amd as cp
    for name, tol in (("f32", 1e-4), ("f16", 1e-2)):
        A, B = G[f"matmul_{name}/a"], G[f"matmul_{name}/b"]
        got = (cp.array(A) @ cp.array(B)).get()
        assert got.dtype == A.dtype
        assert ref.normwise_rel_error(got, G[f"matmul_{name}/out_f64"]) <= tol
    x = cp.array(G["lit_inner/x"])
    assert float((x @ x).get()) == float(G["lit_inner/out"])   # tests/test_error_handling.py:107-114
