"""The reference's own test cases for the hot path, run on the device.

Each test restates one case (or one parametrised group) of the reference's
test suite -- same inputs, same operations, same tolerances -- against the
device implementation; the citation names the reference test it follows.
The reference compares against NumPy at run time, so NumPy is the expected
value here too.  Where the device library deliberately differs from the reference
(float64 kept on the device, NumPy integer semantics), the NumPy result is
the one checked.
"""
import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd import linalg_top
from macmetalpy_amd._backend import HipBackend

pytestmark = pytest.mark.gpu

FLOAT_DTYPES = [np.float16, np.float32]
INT_DTYPES = [np.int16, np.int32, np.int64, np.uint16, np.uint32, np.uint64]
NUMERIC_DTYPES = FLOAT_DTYPES + INT_DTYPES
REDUCE_SHAPES = [(5,), (2, 3), (2, 3, 4)]


def _arg(shape, dtype):
    """Deterministic input: 1, 2, 3, ... in row-major order (bool: even
    positions True), the data the reference's tests use
    (tests/conftest.py:114-131)."""
    if not shape:
        return np.array(1, dtype=dtype)
    n = int(np.prod(shape))
    if n == 0:
        return np.zeros(shape, dtype=dtype)
    data = np.arange(1, n + 1, dtype=np.float64).reshape(shape)
    if np.dtype(dtype) == np.bool_:
        return data % 2 == 0
    return data.astype(dtype)


def _tol(dtype, category="default"):
    """Tolerances of the reference's tol_for (tests/conftest.py:67-97)."""
    dt = np.dtype(dtype)
    if category == "arithmetic":
        return dict(rtol=1e-2, atol=1e-2) if dt == np.float16 else dict(rtol=1e-6, atol=1e-4)
    if category == "unary_math":
        return dict(rtol=1e-2, atol=1e-2) if dt == np.float16 else dict(rtol=1e-5, atol=1e-5)
    if dt == np.float16:
        return dict(rtol=1e-2, atol=1e-3)
    if dt == np.float32:
        return dict(rtol=1e-5, atol=1e-6)
    return dict(rtol=0, atol=0)


def _eq(got, want, dtype=None, category="default"):
    """The reference's assert_eq (tests/conftest.py:100-105), plus a dtype
    check against NumPy's result dtype."""
    g = got.get() if hasattr(got, "get") else np.asarray(got)
    w = np.asarray(want)
    assert g.shape == w.shape
    assert g.dtype == w.dtype, (g.dtype, w.dtype)
    np.testing.assert_allclose(g, w, **_tol(dtype or w.dtype, category))


def _randn(seed, n, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


# --------------------------------------------- fusion (tests/test_fusion.py)
def _legacy(n, k=1):
    """The reference's inputs: np.random.seed(42) then k draws of randn(n)
    as float32 (tests/test_fusion.py:14-17)."""
    rs = np.random.RandomState(42)
    out = [rs.randn(n).astype(np.float32) for _ in range(k)]
    return out if k > 1 else out[0]


def test_fusion_chains():
    """tests/test_fusion.py:12-60: five fused chains at rtol 1e-5.
    sin(cos(exp(a))) is held to the float64 evaluation of the chain instead:
    one ulp of exp moves the result by up to ~5e-7, so two correct float32
    chains differ by far more than rtol 1e-5 wherever cos(exp(a)) nears a
    zero (NumPy's own float32 chain is 5.6e-7 from the float64 one).  The
    reference's test passes at rtol 1e-5 because at 100,000 elements its
    transcendentals run on NumPy (ndarray.py:41-44), i.e. it compares NumPy
    with itself.  The bar: at most twice NumPy's largest error."""
    a, b, c = _legacy(100_000, 3)
    ga, gb, gc = cp.array(a), cp.array(b), cp.array(c)
    np.testing.assert_allclose((cp.sin(ga) + cp.cos(gb) * gc).get(),
                               np.sin(a) + np.cos(b) * c, rtol=1e-5, atol=1e-6)
    h = _legacy(100_000) * np.float32(0.5)
    got = cp.sin(cp.cos(cp.exp(cp.array(h)))).get().astype(np.float64)
    want32 = np.sin(np.cos(np.exp(h))).astype(np.float64)
    truth = np.sin(np.cos(np.exp(h.astype(np.float64))))
    assert np.abs(got - truth).max() <= 2 * np.abs(want32 - truth).max()
    pa, pb = np.abs(a) + np.float32(0.1), np.abs(b) + np.float32(0.1)
    np.testing.assert_allclose((cp.exp(cp.array(pa) * 0.1) + cp.log(cp.array(pb))).get(),
                               np.exp(pa * np.float32(0.1)) + np.log(pb), rtol=1e-5, atol=1e-6)
    a3, b3 = np.abs(_randn(45, 300_000)) + np.float32(0.01), _randn(46, 300_000)
    np.testing.assert_allclose((cp.sqrt(cp.array(a3)) + cp.array(b3) * cp.array(b3)).get(),
                               np.sqrt(a3) + b3 * b3, rtol=1e-5)
    a4, b4 = _randn(47, 300_000), _randn(48, 300_000)
    np.testing.assert_allclose(((-cp.array(a4)) + cp.abs(cp.array(b4))).get(),
                               (-a4) + np.abs(b4), rtol=1e-5, atol=1e-7)


def test_fusion_materialisation_points():
    """tests/test_fusion.py:66-101: get(), a reduction, indexing and repr of
    lazy arrays."""
    ones = np.ones(100_000, np.float32)
    g = cp.array(ones)
    np.testing.assert_allclose((cp.sin(g) + cp.cos(g)).get(), np.sin(ones) + np.cos(ones),
                               rtol=1e-5)
    twos = ones * 2
    s = cp.sin(cp.array(twos)).sum()
    np.testing.assert_allclose(float(s), float(np.sin(twos).astype(np.float64).sum()), rtol=1e-4)
    ar = np.arange(100_000, dtype=np.float32)
    lazy = cp.exp(cp.array(ar) * 0.0001)
    np.testing.assert_allclose(float(lazy[0]), float(np.exp(ar[0] * np.float32(0.0001))), rtol=1e-5)
    np.testing.assert_allclose(float(lazy[99_999]), float(np.exp(ar[99_999] * np.float32(0.0001))),
                               rtol=1e-5)
    assert len(repr(cp.sin(g))) > 0


def test_fusion_edge_cases():
    """tests/test_fusion.py:105-174: shared subexpression, a chain past the
    depth cap, tiny and empty arrays, in-place update from a lazy operand,
    float16."""
    a = _legacy(100_000)
    t = cp.sin(cp.array(a))
    np.testing.assert_allclose((t + t).get(), np.sin(a) + np.sin(a), rtol=1e-5)
    half = np.full(100_000, 0.5, np.float32)
    r, e = cp.array(half), half.copy()
    for _ in range(20):
        r = r + r * 0.001
        e = e + e * np.float32(0.001)
    np.testing.assert_allclose(r.get(), e, rtol=1e-4)
    small = np.array([1.0, 2.0, 3.0], np.float32)
    gs = cp.array(small)
    np.testing.assert_allclose((cp.sin(gs) + cp.cos(gs)).get(), np.sin(small) + np.cos(small),
                               rtol=1e-5)
    assert cp.sin(cp.array(np.array([], np.float32))).size == 0
    b = _randn(43, 100_000)
    ga = cp.array(a.copy())
    ga += cp.sin(cp.array(b))
    np.testing.assert_allclose(ga.get(), a + np.sin(b), rtol=1e-5, atol=1e-7)
    h1 = np.random.default_rng(1).standard_normal(100_000).astype(np.float16)
    h2 = np.random.default_rng(2).standard_normal(100_000).astype(np.float16)
    got = (cp.array(h1) + cp.array(h2)).get()
    assert got.dtype == np.float16
    np.testing.assert_array_equal(got, h1 + h2)  # one rounding: bit-exact


def test_fusion_ops():
    """tests/test_fusion.py:177-209: tanh(sin), floor + ceil, log(exp),
    unary -> binary and unary chain -> multiply."""
    a = _randn(42, 100_000, 5.0)
    np.testing.assert_allclose(cp.tanh(cp.sin(cp.array(a))).get(), np.tanh(np.sin(a)),
                               rtol=1e-5, atol=1e-7)
    a10 = _randn(3, 100_000, 10.0)
    g10 = cp.array(a10)
    np.testing.assert_array_equal((cp.floor(g10) + cp.ceil(g10)).get(), np.floor(a10) + np.ceil(a10))
    p = np.abs(_randn(4, 100_000)) + np.float32(0.1)
    np.testing.assert_allclose(cp.log(cp.exp(cp.array(p))).get(), p, rtol=1e-4, atol=1e-5)
    b = np.abs(_randn(5, 100_000)) + np.float32(0.1)
    np.testing.assert_allclose((cp.sin(cp.array(a)) + cp.array(b)).get(), np.sin(a) + b,
                               rtol=1e-5, atol=1e-7)
    c, d = _randn(6, 100_000), _randn(7, 100_000)
    np.testing.assert_allclose((cp.sin(cp.cos(cp.array(c))) * cp.sin(cp.array(d))).get(),
                               np.sin(np.cos(c)) * np.sin(d), rtol=1e-5, atol=1e-7)


# -------------------------------------- synchronize (tests/test_synchronize.py)
def test_synchronize_semantics():
    """tests/test_synchronize.py:19-92 (the two cases that read the Metal
    backend's private _has_pending flag have no counterpart: the HIP stream
    is synchronised, there is no pending-command-buffer state)."""
    be = HipBackend()
    be.synchronize()
    be.synchronize()
    np.testing.assert_allclose(cp.sqrt(cp.array([1.0, 2.0, 3.0], dtype=np.float32)).get(),
                               np.sqrt(np.array([1.0, 2.0, 3.0], np.float32)), rtol=1e-5)
    np.testing.assert_allclose(cp.sqrt(cp.exp(cp.array([0.0, 1.0, 2.0], dtype=np.float32))).get(),
                               np.sqrt(np.exp(np.array([0.0, 1.0, 2.0], np.float32))), rtol=1e-5)
    a = cp.array([2.0, 4.0, 6.0], dtype=np.float32)
    np.testing.assert_array_equal((a + a).get(), [4.0, 8.0, 12.0])
    e = cp.empty(3, dtype=np.float32)
    e.set(np.array([10.0, 20.0, 30.0], np.float32))
    np.testing.assert_array_equal(e.get(), [10.0, 20.0, 30.0])
    x = cp.array([1.0, 2.0], dtype=np.float32)
    y = cp.array([3.0, 4.0], dtype=np.float32)
    c, d = x + y, x * y
    cp.synchronize()
    np.testing.assert_array_equal(c.get(), [4.0, 6.0])
    np.testing.assert_array_equal(d.get(), [3.0, 8.0])
    s = cp.sqrt(cp.array([1.0, 4.0, 9.0], dtype=np.float32))
    cp.synchronize()
    cp.synchronize()
    np.testing.assert_array_equal(s.get(), [1.0, 2.0, 3.0])


# ----------------------------------------- reductions (tests/test_reductions.py)
@pytest.mark.parametrize("dtype", NUMERIC_DTYPES)
def test_sum_axes(dtype):
    """tests/test_reductions.py:29-60: sum over axis None / 0 / 1 / -1 and
    keepdims, NumPy's result dtype (int16 -> int64, ...)."""
    for shape in REDUCE_SHAPES:
        a = _arg(shape, dtype)
        g = cp.array(a)
        _eq(cp.sum(g), np.sum(a), dtype)
        _eq(cp.sum(g, axis=-1), np.sum(a, axis=-1), dtype)
        if len(shape) > 1:
            _eq(cp.sum(g, axis=0), np.sum(a, axis=0), dtype)
            _eq(cp.sum(g, axis=1), np.sum(a, axis=1), dtype)
            _eq(cp.sum(g, axis=0, keepdims=True), np.sum(a, axis=0, keepdims=True), dtype)


@pytest.mark.parametrize("dtype", NUMERIC_DTYPES)
def test_cumsum_cumprod_axes(dtype):
    """tests/test_reductions.py:472-494 and tests/test_ndarray.py:875-915:
    cumsum over axis None / 0 / -1 and the cumsum / cumprod methods (cumprod
    on 2s, as there)."""
    for shape in [(5,), (2, 3)]:
        a = _arg(shape, dtype)
        _eq(cp.cumsum(cp.array(a)), np.cumsum(a), dtype)
    a = _arg((2, 3), dtype)
    _eq(cp.cumsum(cp.array(a), axis=0), np.cumsum(a, axis=0), dtype)
    _eq(cp.cumsum(cp.array(a), axis=-1), np.cumsum(a, axis=-1), dtype)
    for shape in REDUCE_SHAPES:
        a = _arg(shape, dtype)
        g = cp.array(a)
        _eq(g.cumsum(), a.cumsum(), category="arithmetic")
        twos = np.ones(shape, dtype) * 2
        if not (np.dtype(dtype).itemsize <= 2 and twos.size > 16):
            _eq(cp.array(twos).cumprod(), twos.cumprod(), category="arithmetic")
        if len(shape) > 1:
            for ax in (0, -1):
                _eq(g.cumsum(axis=ax), a.cumsum(axis=ax), category="arithmetic")
                _eq(cp.array(twos).cumprod(axis=ax), twos.cumprod(axis=ax), category="arithmetic")


# ------------------------------- matmul (tests/test_ndarray.py, tests/test_linalg.py)
@pytest.mark.parametrize("dtype", FLOAT_DTYPES)
def test_matmul_small_cases(dtype):
    """tests/test_ndarray.py:528-556 (basic, square, shape error) and
    tests/test_linalg.py:571-592 (matrix, vector-matrix, square through
    linalg_top.matmul)."""
    a, b = _arg((2, 3), dtype), _arg((3, 4), dtype)
    _eq(cp.array(a) @ cp.array(b), a @ b, dtype, "arithmetic")
    s = _arg((3, 3), dtype)
    _eq(cp.array(s) @ cp.array(s), s @ s, dtype, "arithmetic")
    with pytest.raises(ValueError):
        cp.array(_arg((2, 3), dtype)) @ cp.array(_arg((4, 5), dtype))
    a = np.arange(6, dtype=dtype).reshape(2, 3)
    b = np.arange(12, dtype=dtype).reshape(3, 4)
    np.testing.assert_allclose(linalg_top.matmul(cp.array(a), cp.array(b)).get(),
                               np.matmul(a, b), rtol=1e-3, atol=1e-3)
    v = np.array([1, 2, 3], dtype=dtype)
    np.testing.assert_allclose(linalg_top.matmul(cp.array(v), cp.array(b)).get(),
                               np.matmul(v, b), rtol=1e-3, atol=1e-3)
    q = np.arange(9, dtype=dtype).reshape(3, 3)
    np.testing.assert_allclose(linalg_top.matmul(cp.array(q), cp.array(q)).get(),
                               np.matmul(q, q), rtol=1e-2, atol=1e-2)


# --------------------------------- numeric edges (tests/test_numeric_edges.py)
SPECIALS = [np.nan, np.inf, -np.inf, 0.0, -0.0]
UNARY = ["sqrt", "exp", "log", "sin", "cos", "tan", "arcsin", "arccos", "arctan", "sinh", "cosh",
         "tanh", "log2", "log10", "square", "negative", "abs", "sign", "floor", "ceil"]


@pytest.mark.parametrize("name", UNARY)
def test_unary_specials(name):
    """tests/test_numeric_edges.py:17-88: NaN, +-inf, +-0 through 20 unary
    ops (here also the sign of zeros and infinities must match)."""
    x = np.array(SPECIALS, np.float32)
    with np.errstate(all="ignore"):
        want = getattr(np, name)(x)
    got = getattr(cp, name)(cp.array(x)).get()
    assert got.dtype == want.dtype
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    np.testing.assert_allclose(got[ok], want[ok], **_tol(np.float32, "unary_math"))
    np.testing.assert_array_equal(np.signbit(got[ok]), np.signbit(want[ok]))


BIN_COMBOS = [(np.nan, 1.0), (1.0, np.nan), (np.inf, 1.0), (1.0, np.inf), (np.nan, np.inf),
              (np.inf, -np.inf), (0.0, 0.0), (-0.0, 0.0)]


@pytest.mark.parametrize("name", ["add", "subtract", "multiply", "divide", "power"])
def test_binary_specials(name):
    """tests/test_numeric_edges.py:94-148: special pairs through five
    binary ops."""
    a = np.array([l for l, _ in BIN_COMBOS], np.float32)
    b = np.array([r for _, r in BIN_COMBOS], np.float32)
    with np.errstate(all="ignore"):
        want = getattr(np, name)(a, b)
    got = getattr(cp, name)(cp.array(a), cp.array(b)).get()
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_allclose(got, want, **_tol(np.float32, "arithmetic"), equal_nan=True)


def test_float16_precision_and_integer_wrap():
    """tests/test_numeric_edges.py:153-240: float16 epsilon, overflow to
    inf, underflow and subnormal round trips; int32 / int16 wrap-around."""
    eps = np.finfo(np.float16).eps
    one = np.array([1.0], np.float16)
    np.testing.assert_array_equal((cp.array(one) + cp.array(np.array([eps], np.float16))).get(),
                                  one + np.array([eps], np.float16))
    a, b = np.array([1.001], np.float16), np.array([1.0], np.float16)
    np.testing.assert_array_equal((cp.array(a) - cp.array(b)).get(), a - b)
    big = np.array([65504.0], np.float16)
    assert np.isinf((cp.array(big) + cp.array(np.array([100.0], np.float16))).get()[0])
    m = np.array([256.0], np.float16)
    np.testing.assert_array_equal((cp.array(m) * cp.array(m)).get(), m * m)
    for v in (np.finfo(np.float16).tiny / np.float16(100.0), np.finfo(np.float16).smallest_subnormal):
        h = np.array([v], np.float16)
        np.testing.assert_array_equal(cp.array(h).get(), h)
        np.testing.assert_array_equal((cp.array(h) + 0).get(), h + np.float16(0))
    for dt in (np.int32, np.int16):
        info = np.iinfo(dt)
        hi, lo, one_i = np.array([info.max], dt), np.array([info.min], dt), np.array([1], dt)
        np.testing.assert_array_equal((cp.array(hi) + cp.array(one_i)).get(), hi + one_i)
        np.testing.assert_array_equal((cp.array(lo) - cp.array(one_i)).get(), lo - one_i)


def test_nan_in_add_sum_max():
    """tests/test_numeric_edges.py:585-608: NaN propagates through add, sum
    and max."""
    a = np.array([1.0, np.nan, 3.0], np.float32)
    b = np.array([4.0, 5.0, 6.0], np.float32)
    got = (cp.array(a) + cp.array(b)).get()
    assert got[0] == 5.0 and np.isnan(got[1]) and got[2] == 9.0
    assert np.isnan(float(cp.sum(cp.array(a))))
    assert np.isnan(float(cp.max(cp.array(a))))
    big = np.ones(1 << 20, np.float32)
    big[123_457] = np.nan
    assert np.isnan(float(cp.sum(cp.array(big))))
    assert np.isnan(float(cp.max(cp.array(big))))
    assert int(cp.argmax(cp.array(big))) == 123_457
