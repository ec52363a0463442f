"""Reductions, arg-reductions, scans and fused reductions on the GPU against
the oracle.  Bars: integer results bit-exact; float32 sums / means / scans
within 1e-5 relative of the float64-accumulated reference (the kernels
accumulate in float64); max / min / argmax exact, with NumPy's NaN rules."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd.workloads import c3_matrix, c3_scan_inputs, c5_inputs
from oracle import c_oracle as C
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

RTOL = 1e-5


def _rel_err(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    scale = np.maximum(np.abs(want), np.finfo(np.float32).tiny)
    return float(np.max(np.abs(got - want) / scale)) if got.size else 0.0


SHAPES = [(1,), (7,), (4096,), (4097,), (1 << 20,), (3, 5), (64, 1000), (2, 3, 4097),
          (300, 2, 7), (1, 70000)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("axis", [None, 0, -1])
def test_sum_mean_f32(shape, axis):
    x = np.random.default_rng(0).standard_normal(shape).astype(np.float32)
    X = cp.array(x)
    for fn, r64 in ((cp.sum, ref.sum_f64), (cp.mean, ref.mean_f64)):
        got = fn(X, axis=axis).get()
        assert got.dtype == np.float32
        assert got.shape == np.sum(x, axis=axis).shape
        assert _rel_err(got, r64(x, axis=axis).astype(np.float32)) <= RTOL


@pytest.mark.parametrize("dtype", [np.int32, np.int16, np.int64, np.uint32, np.uint16, np.bool_])
@pytest.mark.parametrize("axis", [None, 0, 1])
def test_integer_reductions_exact(dtype, axis):
    g = np.random.default_rng(1)
    if dtype == np.bool_:
        x = g.random((257, 1031)) < 0.3
    else:
        info = np.iinfo(dtype)
        x = g.integers(max(info.min, -1000), min(info.max, 1000), (257, 1031)).astype(dtype)
    X = cp.array(x)
    for name in ("sum", "max", "min"):
        got = getattr(cp, name)(X, axis=axis).get()
        want = getattr(np, name)(x, axis=axis)
        assert got.dtype == want.dtype and np.array_equal(got, want), name
    got = cp.prod(X[:, :5], axis=axis).get()
    assert np.array_equal(got, np.prod(x[:, :5], axis=axis))
    m = cp.mean(X, axis=axis).get()
    assert m.dtype == np.float64
    assert _rel_err(m, np.mean(x.astype(np.float64), axis=axis)) <= 1e-12


@pytest.mark.parametrize("dtype", [np.float16, np.float64])
def test_float16_float64(dtype):
    x = np.random.default_rng(2).standard_normal((37, 4099)).astype(dtype)
    X = cp.array(x)
    for axis in (None, 0, 1):
        s = cp.sum(X, axis=axis).get()
        assert s.dtype == dtype
        want = ref.sum_f64(x, axis=axis).astype(dtype)
        if dtype == np.float64:
            assert _rel_err(s, want) <= 1e-12
        else:
            assert int(ref.ulp_distance(s, want).max()) <= 1
        assert np.array_equal(cp.max(X, axis=axis).get(), np.max(x, axis=axis))


def test_nan_rules_and_ties():
    x = np.array([1, 5, np.nan, 5, np.nan, -3], np.float32)
    X = cp.array(x)
    assert np.isnan(float(cp.max(X).get())) and np.isnan(float(cp.min(X).get()))
    assert cp.argmax(X) == 2 and cp.argmin(X) == 2
    y = np.array([1, 5, 3, 5, 2, -4, -4], np.float32)
    assert cp.argmax(cp.array(y)) == 1 and cp.argmin(cp.array(y)) == 5
    m = np.random.default_rng(3).integers(0, 4, (123, 777)).astype(np.float32)
    m[5, 100] = np.nan
    m[5, 3] = np.nan
    M = cp.array(m)
    for axis in (0, 1):
        assert np.array_equal(cp.argmax(M, axis=axis).get(), np.argmax(m, axis=axis))
        assert np.array_equal(cp.argmin(M, axis=axis).get(), np.argmin(m, axis=axis))
    assert cp.argmax(M) == np.argmax(m)
    big = np.random.default_rng(4).standard_normal(5_000_003).astype(np.float32)
    big[4_999_999] = 100.0
    big[17] = 100.0
    assert cp.argmax(cp.array(big)) == 17 == C.argmax_f32(big)


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.float64, np.int32, np.int64,
                                   np.uint32, np.int16, np.bool_])
def test_argmax_argmin_extremes_and_first_occurrence(dtype):
    """Rows whose extreme equals the reduction's identity (all -inf / +inf,
    all INT_MIN / INT_MAX, all False) must still report index 0; ties
    between elements that different threads visit resolve to the smaller
    index; the first NaN wins in float rows."""
    g = np.random.default_rng(11)
    rows, cols = 9, 70001
    if np.dtype(dtype).kind == "f":
        m = g.standard_normal((rows, cols)).astype(dtype)
        m[0] = -np.inf
        m[1] = np.inf
        m[2, [50000, 7, 30000]] = np.nan
        m[3, [60000, 1234]] = np.inf
    elif dtype == np.bool_:
        m = g.random((rows, cols)) < 0.5
        m[0] = False
        m[1] = True
    else:
        info = np.iinfo(dtype)
        m = g.integers(info.min // 2 if info.min else 0, info.max // 2, (rows, cols)).astype(dtype)
        m[0] = info.min
        m[1] = info.max
        m[3, [60000, 1234]] = info.max
        m[4, [65000, 4321]] = info.min
    M = cp.array(m)
    for axis in (1, None):
        want_max = np.argmax(m, axis=axis)
        want_min = np.argmin(m, axis=axis)
        got_max = cp.argmax(M, axis=axis)
        got_min = cp.argmin(M, axis=axis)
        if axis is None:
            assert got_max == int(want_max) and got_min == int(want_min)
        else:
            assert np.array_equal(got_max.get(), want_max)
            assert np.array_equal(got_min.get(), want_min)


def test_reference_known_answers():
    # tests/test_edge_shapes.py:367-378: sum of 1M ones
    assert float(cp.sum(cp.ones(1_000_000, dtype=np.float32)).get()) == 1e6
    n = 1 << 22
    assert float(cp.sum(cp.arange(n, dtype=np.float32)).get()) == n * (n - 1) / 2
    assert int(cp.sum(cp.ones(1000, dtype=np.int32)).get()) == 1000


def test_repeated_calls_reuse_scratch():
    """Completion tickets are re-armed: back-to-back split reductions of
    different shapes stay correct."""
    g = np.random.default_rng(5)
    for n in (1 << 22, 3_000_001, 1 << 20, 1 << 23):
        x = g.standard_normal(n).astype(np.float32)
        X = cp.array(x)
        for _ in range(3):
            assert _rel_err(cp.sum(X).get(), ref.sum_f64(x)) <= RTOL
            assert cp.argmax(X) == np.argmax(x)


def test_empty_and_errors():
    e = cp.array(np.zeros((0, 4), np.float32))
    assert np.array_equal(cp.sum(e, axis=0).get(), np.zeros(4, np.float32))
    assert float(cp.sum(e).get()) == 0.0
    with pytest.raises(ValueError):
        cp.max(e)
    with pytest.raises(ValueError):
        cp.argmax(e)


def test_integer_mean_dtype_wraps_like_numpy():
    """mean(x, dtype=<int>): NumPy sums in that dtype (wrapping), divides by
    the count in float64 and truncates back (numpy/_core/_methods.py
    _mean).  Known answers: 1000 x 100 in int16 sums to 100000 = 34464 mod
    2^16 = -31072 as int16, / 1000 -> -31; 1000 x 3e6 in int32 sums to
    3e9 -> -1294967296, / 1000 -> -1294967."""
    print("integer mean dtypes", flush=True)
    assert int(cp.mean(cp.array(np.full(1000, 100, np.int16)), dtype=np.int16)) == -31
    assert int(cp.mean(cp.array(np.full(1000, 3_000_000, np.int32)), dtype=np.int32)) == -1294967
    g = np.random.default_rng(11)
    cases = [(g.integers(20000, 32767, (64, 300)).astype(np.int16), np.int16),
             (g.integers(-2**31, 2**31 - 1, (16, 5000), dtype=np.int64).astype(np.int32), np.int32),
             (g.integers(0, 65535, (8, 4000)).astype(np.uint16), np.uint16),
             (g.integers(-2**62, 2**62, (4, 1000), dtype=np.int64), np.int64),
             (g.integers(0, 2**31, (4, 1000)).astype(np.int32), np.int16)]
    for x, dt in cases:
        X = cp.array(x)
        for axis in (None, 0, 1):
            want = np.mean(x, axis=axis, dtype=dt)
            got = cp.mean(X, axis=axis, dtype=dt)
            assert got.dtype == want.dtype, (dt, axis, got.dtype)
            assert np.array_equal(np.asarray(got.get()), want), (dt, axis)
            nwant = np.nanmean(x, axis=axis, dtype=dt)
            assert np.array_equal(np.asarray(cp.nanmean(X, axis=axis, dtype=dt).get()), nwant)


def test_keepdims_and_var_std():
    x = np.random.default_rng(6).standard_normal((40, 50)).astype(np.float32)
    X = cp.array(x)
    assert cp.sum(X, axis=1, keepdims=True).shape == (40, 1)
    assert cp.mean(X, keepdims=True).shape == (1, 1)
    for axis in (None, 0, 1):
        assert _rel_err(cp.var(X, axis=axis).get(), np.var(x.astype(np.float64), axis=axis)) <= 1e-4
        assert _rel_err(cp.std(X, axis=axis, ddof=1).get(),
                        np.std(x.astype(np.float64), axis=axis, ddof=1)) <= 1e-4


# ------------------------------------------------------------------ scan
@pytest.mark.parametrize("n", [1, 5, 4095, 4096, 4097, 3 * 4096 + 5, 1_000_003])
def test_cumsum_int32_exact_and_float(n):
    g = np.random.default_rng(7)
    xi = g.integers(-100, 100, n, endpoint=True, dtype=np.int32)
    got = cp.cumsum(cp.array(xi)).get()
    assert got.dtype == np.int64 and np.array_equal(got, ref.cumsum(xi))
    assert np.array_equal(got, C.cumsum_i32(xi))
    xf = g.random(n, dtype=np.float32)
    gf = cp.cumsum(cp.array(xf)).get()
    assert gf.dtype == np.float32
    assert _rel_err(gf, ref.cumsum_f64(xf).astype(np.float32)) <= RTOL


@pytest.mark.parametrize("shape,axis", [((33, 5000), 1), ((33, 5000), 0), ((4, 3, 9001), -1),
                                        ((4, 3, 9001), 1), ((7, 4096), None), ((1000, 3), 1)])
def test_cumsum_axes(shape, axis):
    x = np.random.default_rng(8).integers(-50, 50, shape).astype(np.int32)
    got = cp.cumsum(cp.array(x), axis=axis).get()
    assert np.array_equal(got, np.cumsum(x, axis=axis))
    f = np.random.default_rng(8).random(shape, dtype=np.float32)
    gf = cp.cumsum(cp.array(f), axis=axis).get()
    want = np.cumsum(f.astype(np.float64), axis=axis).astype(np.float32)
    assert _rel_err(gf, want) <= RTOL


@pytest.mark.parametrize("dtype", [np.int32, np.int16, np.int64, np.uint32, np.float32,
                                   np.float64, np.bool_])
@pytest.mark.parametrize("shape", [(16384 * 3,), (16384 * 4 + 4000,), (3, 40000), (2, 32768)])
def test_cumsum_whole_tiles_and_tails(dtype, shape):
    """Rows whose byte length is a multiple of 16 take the streaming kernel
    for their whole tiles (16384 elements, 8192 for 8-byte types) and a
    second launch for each row's partial tail, which starts from the
    inclusive prefix the first launch published for the row's last whole
    tile."""
    g = np.random.default_rng(len(shape) * 31 + shape[-1])
    if dtype == np.bool_:
        x = g.random(shape) < 0.5
    elif np.dtype(dtype).kind == "f":
        x = g.random(shape).astype(dtype)
    else:
        x = g.integers(0, 100, shape).astype(dtype)
    got = cp.cumsum(cp.array(x), axis=-1).get()
    if np.dtype(dtype).kind == "f":
        want = np.cumsum(x.astype(np.float64), axis=-1).astype(dtype)
        assert got.dtype == np.dtype(dtype) and _rel_err(got, want) <= RTOL
    else:
        want = np.cumsum(x, axis=-1)
        assert got.dtype == want.dtype and np.array_equal(got, want)


def test_cumprod_small():
    x = np.random.default_rng(9).integers(1, 3, 40).astype(np.int32)
    assert np.array_equal(cp.cumprod(cp.array(x)).get(), np.cumprod(x))
    f = (1 + np.random.default_rng(9).standard_normal(10000).astype(np.float32) * 1e-3)
    assert _rel_err(cp.cumprod(cp.array(f)).get(), np.cumprod(f.astype(np.float64))) <= 1e-5


def test_scan_repeated_generations():
    x = np.arange(50000, dtype=np.int32) % 7 - 3
    X = cp.array(x)
    want = np.cumsum(x)
    for _ in range(5):
        assert np.array_equal(cp.cumsum(X).get(), want)


@pytest.mark.parametrize("dtype,shape,op", [(np.float32, (1 << 24,), "cumsum"),
                                            (np.float32, (3, (1 << 22) + 1000), "cumsum"),
                                            (np.float64, (1 << 23,), "cumsum"),
                                            (np.float16, (1 << 22,), "cumsum"),
                                            (np.float32, (1 << 22,), "cumprod")])
def test_float_scan_bits_repeat(dtype, shape, op):
    """A floating scan's tile prefixes are folded in an order fixed by tile
    position, not by which predecessor happened to publish first, so
    repeated runs over hundreds of tiles give the same bits."""
    g = np.random.default_rng(77)
    x = (g.random(shape) + (0.5 if op == "cumprod" else 0.0))
    if op == "cumprod":
        x = 1.0 + (x - 1.0) * 1e-6
    X = cp.array(x.astype(dtype))
    f = getattr(cp, op)
    first = f(X, axis=-1).get()
    for _ in range(3):
        assert np.array_equal(f(X, axis=-1).get(), first, equal_nan=True)


# ------------------------------------------------------ fused reductions
def test_fused_sum_matches_unfused():
    x_np = np.random.default_rng(10).standard_normal((300, 7001)).astype(np.float32)
    x = cp.array(x_np)
    for axis in (None, -1, 1):
        fused = cp.sum(cp.exp(-cp.abs(x)) * 2.0 - x * x, axis=axis).get()
        cp.set_config(fusion=False)
        unf = cp.sum(cp.exp(-cp.abs(x)) * 2.0 - x * x, axis=axis).get()
        cp.set_config(fusion=True)
        want = ref.sum_f64((np.exp(-np.abs(x_np)) * np.float32(2.0) - x_np * x_np), axis=axis)
        assert _rel_err(fused, want.astype(np.float32)) <= RTOL
        assert _rel_err(unf, want.astype(np.float32)) <= RTOL
    m = cp.mean(cp.sin(x), axis=-1).get()
    assert _rel_err(m, ref.mean_f64(np.sin(x_np), axis=-1).astype(np.float32)) <= 1e-4


def test_c5_fusion_chain_full_size():
    x_np, r_np = c5_inputs()
    x, r = cp.array(x_np), cp.array(r_np)
    z = cp.sum(cp.tanh(x * r + 1.0) * cp.exp(-cp.abs(x)) - cp.log1p(x * x), axis=1)
    got = z.get()
    want = ref.fusion_chain_f64(x_np, r_np)
    assert got.shape == (8192,) and got.dtype == np.float32
    assert _rel_err(got, want) <= RTOL


def test_c3_full_size():
    a = c3_matrix()
    A = cp.array(a)
    s_all = float(cp.sum(A).get())
    assert abs(s_all - float(ref.sum_f64(a))) <= RTOL * abs(float(ref.sum_f64(a)))
    assert _rel_err(cp.mean(A).get(), ref.mean_f64(a)) <= RTOL
    rows = cp.sum(A, axis=1).get()
    assert _rel_err(rows, ref.sum_f64(a, axis=1).astype(np.float32)) <= RTOL
    assert _rel_err(cp.mean(A, axis=1).get(), ref.mean_f64(a, axis=1).astype(np.float32)) <= RTOL
    assert np.array_equal(cp.argmax(A, axis=1).get(), np.argmax(a, axis=1))
    assert cp.argmax(A) == int(np.argmax(a))


def test_c3_scan_full_size():
    ci, cf = c3_scan_inputs()
    got = cp.cumsum(cp.array(ci)).get()
    assert got.dtype == np.int64
    assert np.array_equal(got, np.cumsum(ci))
    del got
    CF = cp.array(cf)
    gf = cp.cumsum(CF).get()
    want = np.cumsum(cf.astype(np.float64))
    assert _rel_err(gf, want) <= RTOL
    assert np.array_equal(cp.cumsum(CF).get(), gf)  # the same bits on a second run
