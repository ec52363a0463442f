"""Pin the oracle (CPU): every function is checked against mathematics or
known answers that a plausible mistake (truncating division, wrong
remainder sign, int32 cumsum, last-index argmax, fmod for mod, a dropped
term in a fused expression) would violate."""
import math

import numpy as np
import pytest

from oracle import c_oracle as C
from oracle import reference_cpu as ref

I32_MIN = -2 ** 31


# ----------------------------------------------------- integer division
def test_floor_divide_mod_brute_force_identity():
    """All a in [-1024, 1024], b in +-[1, 1000]: a == q*b + r with r in
    [0, b) for b > 0 and (b, 0] for b < 0, q == floor(a / b)."""
    a = np.arange(-1024, 1025, dtype=np.int32)
    b = np.concatenate([np.arange(1, 1001), -np.arange(1, 1001)]).astype(np.int32)
    A, B = np.meshgrid(a, b, indexing="ij")
    q = ref.floor_divide(A, B)
    r = ref.mod(A, B)
    assert q.dtype == np.int32 and r.dtype == np.int32
    assert np.array_equal(q.astype(np.int64) * B + r, A)
    pos = B > 0
    assert np.all((r[pos] >= 0) & (r[pos] < B[pos]))
    assert np.all((r[~pos] <= 0) & (r[~pos] > B[~pos]))
    exact = np.array([[math.floor(x / y) for y in (7, -7, 1000, -1)] for x in range(-50, 51)])
    got = ref.floor_divide(np.arange(-50, 51, dtype=np.int32)[:, None],
                           np.array([7, -7, 1000, -1], dtype=np.int32)[None, :])
    assert np.array_equal(got, exact)


def test_integer_edge_cases_hand_derived():
    a = np.array([7, -7, 7, -7, 0, I32_MIN, I32_MIN, 5, -5, 2 ** 31 - 1], np.int32)
    b = np.array([2, 2, -2, -2, 3, -1, 1, 0, 0, -1], np.int32)
    # floor(7/2)=3, floor(-7/2)=-4, floor(7/-2)=-4, floor(-7/-2)=3, 0,
    # INT_MIN//-1 wraps to INT_MIN, x//0 -> 0 (NumPy), INT_MAX//-1 = -INT_MAX
    assert ref.floor_divide(a, b).tolist() == [3, -4, -4, 3, 0, I32_MIN, I32_MIN, 0, 0, -(2 ** 31 - 1)]
    assert ref.mod(a, b).tolist() == [1, 1, -1, -1, 0, 0, 0, 0, 0, 0]


def test_c_restatement_agrees_with_numpy_restatement():
    g = np.random.default_rng(11)
    a = g.integers(-2 ** 31, 2 ** 31, 1 << 20, dtype=np.int64).astype(np.int32)
    b = g.integers(-2000, 2000, 1 << 20, dtype=np.int32)
    b[::97] = 0
    b[::89] = -1
    a[::83] = I32_MIN
    assert np.array_equal(C.floor_divide_i32(a, b), ref.floor_divide(a, b))
    assert np.array_equal(C.mod_i32(a, b), ref.mod(a, b))


def test_reference_test_literals_float():
    """Literal inputs of tests/test_math_ops.py:446-453 / test_math_ext.py:302-307
    (mod) and test_untested_math.py:227-232 (floor_divide); answers by hand."""
    a = np.array([-7.0, 8.0, -9.0], np.float32)
    b = np.array([3.0, -3.0, -4.0], np.float32)
    assert ref.mod(a, b).tolist() == [2.0, -1.0, -1.0]
    fa = np.array([-7.0, -10.0, 7.0], np.float32)
    fb = np.array([2.0, 3.0, -2.0], np.float32)
    assert ref.floor_divide(fa, fb).tolist() == [-4.0, -4.0, -4.0]
    # test_ndarray_gaps.py:667-678: 10.0 % [2,3,4] and [10,20,30] % 7.0
    assert (np.float32(10.0) % np.array([2.0, 3.0, 4.0], np.float32)).tolist() == [0.0, 1.0, 2.0]
    assert ref.mod(np.array([10.0, 20.0, 30.0], np.float32), np.float32(7.0)).tolist() == [3.0, 6.0, 2.0]


def test_float_divmod_identity_and_sign():
    g = np.random.default_rng(5)
    a = (g.standard_normal(200000) * 1000).astype(np.float32)
    b = (g.standard_normal(200000) * 10).astype(np.float32)
    q = ref.floor_divide(a, b)
    r = ref.mod(a, b)
    assert np.all(q == np.floor(q))
    nz = r != 0
    assert np.all(np.sign(r[nz]) == np.sign(b[nz]))
    assert np.all(np.abs(r) <= np.abs(b))
    resid = np.abs(q.astype(np.float64) * b + r - a)
    assert np.all(resid <= 4 * np.spacing(np.abs(a).astype(np.float32)) + np.abs(b) * 1e-6)
    # mod is not C fmod: opposite signs differ
    assert ref.mod(np.float32(-7), np.float32(3)) == 2 and np.fmod(np.float32(-7), np.float32(3)) == -1


# ------------------------------------------------------ transcendentals
@pytest.mark.parametrize("op,fn64,lo,hi", [
    ("sin_op", np.sin, -10, 10), ("exp_op", np.exp, -80, 80), ("tanh_op", np.tanh, -10, 10),
    ("log1p_op", np.log1p, -0.99, 100), ("sqrt_op", np.sqrt, 0, 1e6), ("cos_op", np.cos, -10, 10),
    ("log_op", np.log, 1e-30, 1e30), ("expm1_op", np.expm1, -5, 5),
])
def test_float32_transcendentals_within_ulp_of_float64(op, fn64, lo, hi):
    """The oracle computes the named function: float32 results within 2 ULP
    of the float64 evaluation rounded once."""
    x = np.random.default_rng(1).uniform(lo, hi, 100000).astype(np.float32)
    got = ref.unary(op, x)
    want = ref.correctly_rounded(fn64, x)
    assert got.dtype == np.float32
    assert int(ref.ulp_distance(got, want).max()) <= 2


def test_ulp_distance_helper():
    one = np.float32(1.0)
    nxt = np.nextafter(one, np.float32(2))
    assert ref.ulp_distance(np.array([one]), np.array([nxt]))[0] == 1
    assert ref.ulp_distance(np.array([np.float32(-0.0)]), np.array([np.float32(0.0)]))[0] == 0
    assert ref.ulp_distance(np.array([np.float32(np.nan)]), np.array([np.float32(np.nan)]))[0] == 0
    assert ref.ulp_distance(np.array([-nxt]), np.array([nxt]))[0] == 2 * 0x3F800001


@pytest.mark.parametrize("dt,one_bits", [(np.float16, 0x3C00), (np.float64, 0x3FF0000000000000)])
def test_ulp_distance_helper_float16_float64(dt, one_bits):
    """The float16 and float64 branches (the comparator of the float16 and
    float64 GPU tests): adjacent values 1 apart, across zero and across a
    binade; -0 vs +0 and NaN vs NaN 0; -x vs x twice x's bit pattern."""
    one = dt(1.0)
    nxt = np.nextafter(one, dt(2))
    prv = np.nextafter(one, dt(0))
    d = ref.ulp_distance
    assert d(np.array([one], dt), np.array([nxt], dt))[0] == 1
    assert d(np.array([prv], dt), np.array([nxt], dt))[0] == 2      # across the binade edge
    tiny = np.nextafter(dt(0), dt(1))
    assert d(np.array([-tiny], dt), np.array([tiny], dt))[0] == 2   # across zero
    assert d(np.array([dt(-0.0)], dt), np.array([dt(0.0)], dt))[0] == 0
    assert d(np.array([dt(np.nan)], dt), np.array([dt(np.nan)], dt))[0] == 0
    assert d(np.array([-nxt], dt), np.array([nxt], dt))[0] == 2 * (one_bits + 1)
    assert d(np.array([-one], dt), np.array([one], dt))[0] == 2 * one_bits
    # symmetric, and counts every representable value in between
    x = np.array([dt(0.75)], dt)
    y = x.copy()
    for _ in range(37):
        y = np.nextafter(y, dt(2))
    assert d(x, y)[0] == 37 and d(y, x)[0] == 37


# ------------------------------------------------------------ reductions
def test_sum_closed_forms():
    # tests/test_edge_shapes.py:367-378: sum of 1M ones is 1e6
    assert ref.sum(np.ones(1_000_000, np.float32)) == 1e6
    n = 100000
    assert ref.sum_f64(np.arange(n, dtype=np.float32)) == n * (n - 1) / 2
    assert ref.sum(np.ones(7, np.int32)).dtype == np.int64
    assert ref.mean(np.arange(10, dtype=np.int32)) == 4.5
    x = np.random.default_rng(2).standard_normal(1 << 16).astype(np.float32)
    assert math.isclose(C.sum_f32(x), float(ref.sum_f64(x)), rel_tol=1e-12)


def test_argmax_first_occurrence_and_nan():
    x = np.array([1, 5, 3, 5, 2], np.float32)
    assert ref.argmax(x) == 1  # first of the tied maxima
    y = np.array([1, np.nan, 9, np.nan], np.float32)
    assert ref.argmax(y) == 1  # first NaN wins
    g = np.random.default_rng(3)
    for _ in range(20):
        v = g.integers(0, 5, 37).astype(np.float32)
        assert ref.argmax(v) == min(i for i in range(37) if v[i] == v.max())
        assert C.argmax_f32(v) == ref.argmax(v)
    m = g.standard_normal((9, 13)).astype(np.float32)
    assert np.array_equal(ref.argmax(m, axis=1), [int(np.argmax(r)) for r in m])


def test_cumsum_int64_and_invariants():
    x = np.random.default_rng(4).integers(-100, 100, 100001, endpoint=True, dtype=np.int32)
    c = ref.cumsum(x)
    assert c.dtype == np.int64
    assert np.array_equal(np.diff(c), x[1:].astype(np.int64)) and c[0] == x[0]
    assert c[-1] == x.astype(np.int64).sum()
    assert np.array_equal(c, C.cumsum_i32(x))
    assert np.array_equal(ref.cumsum(np.ones(1000, np.int32)), np.arange(1, 1001))
    f = np.random.default_rng(4).random(1 << 16, dtype=np.float32)
    c64 = ref.cumsum_f64(f)
    assert c64.dtype == np.float64 and math.isclose(c64[-1], float(ref.sum_f64(f)), rel_tol=1e-12)


# ---------------------------------------------------------------- matmul
def test_matmul_known_answers():
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    assert ref.matmul(a, b).tolist() == [[19, 22], [43, 50]]
    e = np.eye(5, dtype=np.float32)
    m = np.random.default_rng(0).standard_normal((5, 5)).astype(np.float32)
    assert np.array_equal(ref.matmul(m, e), m)
    # tests/test_error_handling.py:107-114: 1-D @ 1-D is the inner product
    assert ref.matmul(np.arange(3, dtype=np.float32), np.arange(3, dtype=np.float32)) == 5.0
    t = np.random.default_rng(1).standard_normal((4, 3, 6))
    u = np.random.default_rng(2).standard_normal((4, 6, 2))
    loop = np.array([[[sum(t[k, i, p] * u[k, p, j] for p in range(6)) for j in range(2)]
                      for i in range(3)] for k in range(4)])
    assert np.allclose(ref.matmul_f64(t, u), loop, rtol=1e-12)
    assert ref.normwise_rel_error(ref.matmul(a, b), [[19, 22], [43, 50]]) == 0.0


# ------------------------------------------------------------- fusion
def test_fused_elementwise_scalar_values():
    x = np.array([0.0, 1.0, -4.0], np.float32)
    y = ref.fused_elementwise(x)
    expect = [1.0, 1.0 + math.exp(-1.0), 2.0 + math.exp(-16.0)]
    assert np.allclose(y, expect, rtol=2e-7)


def test_fusion_chain_against_python_loop():
    g = np.random.default_rng(7)
    x = g.standard_normal((3, 17)).astype(np.float32)
    r = g.uniform(0.5, 2.0, (1, 17)).astype(np.float32)
    z = ref.fusion_chain_f64(x, r)
    loop = [sum(math.tanh(float(x[i, j]) * float(r[0, j]) + 1.0) * math.exp(-abs(float(x[i, j])))
                - math.log1p(float(x[i, j]) ** 2) for j in range(17)) for i in range(3)]
    assert np.allclose(z, loop, rtol=1e-5)
    assert z.shape == (3,)


# ------------------------------------------- bitwise / logical / predicates
def _wrap(v, dtype):
    """Python int -> dtype's two's-complement value."""
    bits = np.dtype(dtype).itemsize * 8
    v &= (1 << bits) - 1
    if np.issubdtype(dtype, np.signedinteger) and v >= 1 << (bits - 1):
        v -= 1 << bits
    return v


@pytest.mark.parametrize("dtype", [np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64])
def test_shift_and_bitwise_closed_forms(dtype):
    """Shifts: counts in [0, bits) shift (left wraps, right is arithmetic
    for signed types); any other count -- negative ones included -- gives 0
    (or -1 for a negative value shifted right).  Checked against Python's
    unbounded integers over every count in [-3, bits + 3)."""
    info = np.iinfo(dtype)
    bits = info.bits
    vals = sorted({info.min, info.min + 1, -7 if info.min < 0 else 7, -1 if info.min < 0 else 1,
                   0, 1, 5, info.max - 1, info.max, int(info.max // 3)})
    counts = list(range(-3, bits + 3))
    if info.min == 0:
        counts = [c for c in counts if c >= 0]
    a = np.array([v for v in vals for _ in counts], dtype=dtype)
    b = np.array([c for _ in vals for c in counts], dtype=dtype)
    left = ref.binary("lshift_op", a, b)
    right = ref.binary("rshift_op", a, b)
    for x, c, l, r in zip(a.tolist(), b.tolist(), left.tolist(), right.tolist()):
        inside = 0 <= c < bits
        assert l == (_wrap(x << c, dtype) if inside else 0), (x, c)
        assert r == ((x >> c) if inside else (-1 if x < 0 else 0)), (x, c)
    x = a[:: len(counts)]
    y = x[::-1].copy()
    mask = (1 << bits) - 1
    for op, f in (("bit_and_op", lambda p, q: p & q), ("bit_or_op", lambda p, q: p | q),
                  ("bit_xor_op", lambda p, q: p ^ q)):
        got = ref.binary(op, x, y).tolist()
        assert got == [_wrap(f(p & mask, q & mask), dtype) for p, q in zip(x.tolist(), y.tolist())]
    assert ref.unary("invert_op", x).tolist() == [_wrap(~p, dtype) for p in x.tolist()]


def test_predicates_and_truth_values_hand_derived():
    specials = [np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -2.5]
    # (isnan, isinf, isfinite, signbit, logical_not) per value
    expect = [(1, 0, 0, 0, 0), (1, 0, 0, 1, 0), (0, 1, 0, 0, 0), (0, 1, 0, 1, 0),
              (0, 0, 1, 0, 1), (0, 0, 1, 1, 1), (0, 0, 1, 0, 0), (0, 0, 1, 1, 0)]
    for dt in (np.float16, np.float32, np.float64):
        x = np.array(specials, dtype=dt)
        x[1] = -np.abs(x[1])  # a NaN with the sign bit set
        for k, op in enumerate(("isnan_op", "isinf_op", "isfinite_op", "signbit_op",
                                "logical_not_op")):
            assert ref.unary(op, x).astype(int).tolist() == [e[k] for e in expect], (dt, op)
    i = np.array([-3, 0, 7], dtype=np.int32)
    assert ref.unary("isnan_op", i).tolist() == [False] * 3
    assert ref.unary("isfinite_op", i).tolist() == [True] * 3
    assert ref.unary("signbit_op", i).tolist() == [True, False, False]
    # truth table (NaN is true, -0.0 false), mixed operand dtypes
    p = np.array([0.0, -0.0, np.nan, 2.0, 0.0, 3.0], dtype=np.float32)
    q = np.array([0, 1, 0, 5, 7, 0], dtype=np.int16)
    tp = [False, False, True, True, False, True]
    tq = [False, True, False, True, True, False]
    assert ref.binary("logical_and_op", p, q).tolist() == [u and v for u, v in zip(tp, tq)]
    assert ref.binary("logical_or_op", p, q).tolist() == [u or v for u, v in zip(tp, tq)]
    assert ref.binary("logical_xor_op", p, q).tolist() == [u != v for u, v in zip(tp, tq)]


def test_where_clip_any_all_count_against_python():
    rng = np.random.default_rng(11)
    c = rng.random(50) < 0.4
    x = rng.standard_normal(50).astype(np.float32)
    y = np.float32(-9.5)
    got = ref.where(c, x, y)
    assert got.dtype == np.float32
    assert got.tolist() == [xi if ci else -9.5 for ci, xi in zip(c.tolist(), x.tolist())]
    # clip = min(max(a, lo), hi) with NaN propagating from any operand; lo > hi gives hi
    a = np.array([-2.0, 0.5, 3.0, np.nan], dtype=np.float32)
    assert ref.clip(a, -1.0, 1.0).tolist()[:3] == [-1.0, 0.5, 1.0]
    assert np.isnan(ref.clip(a, -1.0, 1.0)[3])
    assert ref.clip(a[:3], 2.0, 1.0).tolist() == [1.0, 1.0, 1.0]
    assert np.isnan(ref.clip(a[:3], np.nan, 1.0)).all()
    assert ref.clip(np.arange(5, dtype=np.int32), 1, 3).tolist() == [1, 1, 2, 3, 3]
    m = np.array([[0.0, np.nan, 0.0], [0.0, 0.0, 0.0], [1.0, -0.0, 2.0]], dtype=np.float32)
    rows = m.tolist()

    def truth(v):
        return v != 0 or v != v

    assert ref.any_(m, axis=1).tolist() == [any(truth(v) for v in r) for r in rows]
    assert ref.all_(m, axis=1).tolist() == [all(truth(v) for v in r) for r in rows]
    assert ref.count_nonzero(m, axis=0).tolist() == [
        sum(truth(r[j]) for r in rows) for j in range(3)]
    assert ref.count_nonzero(m) == 3
    assert ref.any_(np.zeros((2, 0)), axis=1).tolist() == [False, False]
    assert ref.all_(np.zeros((2, 0)), axis=1).tolist() == [True, True]


# ------------------------------------------------------- NaN reductions
def test_nan_reductions_against_python_loops():
    """Each nan* function equals the plain operation over the non-NaN
    elements of each row (first index for the arg ops); all-NaN rows give
    0 / 1 / NaN, and the arg ops raise."""
    rows = [[1.5, np.nan, -2.0, 7.0, 7.0], [np.nan] * 5, [0.0, -0.0, np.nan, -np.inf, 3.0],
            [2.0, 2.0, 2.0, np.nan, 1.0]]
    x = np.array(rows, np.float64)

    def clean(r):
        return [v for v in r if v == v]

    assert ref.nan_reduce("nansum", x, axis=1).tolist() == [sum(clean(r)) for r in rows]
    np.testing.assert_array_equal(ref.nan_reduce("nanprod", x, axis=1),
                                  [math.prod(clean(r)) for r in rows])  # 0 * -inf is NaN
    for name, f in (("nanmax", max), ("nanmin", min)):
        got = ref.nan_reduce(name, x, axis=1)
        for g, r in zip(got.tolist(), rows):
            assert (g != g) if not clean(r) else g == f(clean(r))
    got = ref.nan_reduce("nanmean", x, axis=1)
    for g, r in zip(got.tolist(), rows):
        c = clean(r)
        assert (g != g) if not c else g == sum(c) / len(c)
    v1 = ref.nan_reduce("nanvar", x[[0, 3]], axis=1, ddof=1)
    for g, r in zip(v1.tolist(), (rows[0], rows[3])):
        c = clean(r)
        m = sum(c) / len(c)
        assert math.isclose(g, sum((t - m) ** 2 for t in c) / (len(c) - 1), rel_tol=1e-12)
    ok = x[[0, 2, 3]]
    for name, f in (("nanargmax", max), ("nanargmin", min)):
        got = ref.nan_reduce(name, ok, axis=1).tolist()
        want = [next(i for i, v in enumerate(r) if v == f(clean(r))) for r in ok.tolist()]
        assert got == want
        with pytest.raises(ValueError):
            ref.nan_reduce(name, x, axis=1)
    cs = ref.nan_reduce("nancumsum", x[0])
    acc, want = 0.0, []
    for v in rows[0]:
        acc += 0.0 if v != v else v
        want.append(acc)
    assert cs.tolist() == want
    # nanstd: the square root of the (pinned above) Python-loop variance
    s1 = ref.nan_reduce("nanstd", x[[0, 3]], axis=1, ddof=1)
    for g, r in zip(s1.tolist(), (rows[0], rows[3])):
        c = clean(r)
        m = sum(c) / len(c)
        assert math.isclose(g, math.sqrt(sum((t - m) ** 2 for t in c) / (len(c) - 1)),
                            rel_tol=1e-12)
    s0 = ref.nan_reduce("nanstd", x[[0, 3]], axis=1)
    for g, r in zip(s0.tolist(), (rows[0], rows[3])):
        c = clean(r)
        m = sum(c) / len(c)
        assert math.isclose(g, math.sqrt(sum((t - m) ** 2 for t in c) / len(c)), rel_tol=1e-12)
    assert math.isnan(ref.nan_reduce("nanstd", x[1]))                 # all NaN
    # nancumprod: a running product with NaN taken as 1
    for r in rows:
        acc, want = 1.0, []
        for v in r:
            acc *= 1.0 if v != v else v
            want.append(acc)
        got = ref.nan_reduce("nancumprod", np.array(r, np.float64))
        np.testing.assert_array_equal(got, want)


# -------------------------------------------------------------- sorting
def test_sort_argsort_searchsorted_against_python():
    """np.sort / stable argsort / searchsorted against Python's sorted()
    with NaN ordered last, stable ties by position, and bisect."""
    import bisect
    rng = np.random.default_rng(21)
    x = rng.integers(-5, 5, 300).astype(np.float64)
    x[::17] = np.nan
    x[5] = -0.0
    xs = x.tolist()

    def key(i):
        v = xs[i]
        return (v != v, 0.0 if v != v else v)

    order = sorted(range(len(xs)), key=key)          # stable
    assert ref.argsort_stable(x).tolist() == order
    got = ref.sort(x, kind="stable")
    want = np.array([xs[i] for i in order])
    assert np.array_equal(got, want, equal_nan=True)
    assert np.array_equal(np.signbit(got), np.signbit(want))  # -0.0 kept in place
    a = np.sort(rng.integers(0, 50, 200)).astype(np.int64)
    al = a.tolist()
    v = np.arange(-2, 53)
    assert ref.searchsorted(a, v).tolist() == [bisect.bisect_left(al, t) for t in v.tolist()]
    assert ref.searchsorted(a, v, side="right").tolist() == [
        bisect.bisect_right(al, t) for t in v.tolist()]
    f = np.array([1.0, 2.0, np.nan, np.nan])
    assert ref.searchsorted(f, [np.nan, np.inf, 2.0], side="left").tolist() == [2, 2, 1]
    assert ref.searchsorted(f, [np.nan], side="right").tolist() == [4]


# ------------------------------------------- pins added for every remaining def
def test_mean_f64_closed_forms():
    """mean of arange(n) is (n-1)/2; along each axis of a known matrix the
    means are the row / column midpoints; mean == sum / count."""
    for n in (1, 2, 7, 100001):
        assert ref.mean_f64(np.arange(n, dtype=np.float32)) == (n - 1) / 2
    m = np.arange(12, dtype=np.float32).reshape(3, 4)   # m[i, j] = 4 i + j
    assert ref.mean_f64(m, axis=1).tolist() == [1.5, 5.5, 9.5]
    assert ref.mean_f64(m, axis=0).tolist() == [4.0, 5.0, 6.0, 7.0]
    assert ref.mean_f64(m) == 5.5
    x = np.random.default_rng(31).standard_normal((17, 33)).astype(np.float32)
    for ax, cnt in ((None, x.size), (0, 17), (1, 33)):
        assert np.allclose(ref.mean_f64(x, axis=ax), ref.sum_f64(x, axis=ax) / cnt,
                           rtol=1e-15, atol=0)
    # float64 accumulation: a float32 accumulator would lose the small term
    big = np.array([2.0 ** 25, 1.0, -(2.0 ** 25), 1.0], np.float32)
    assert ref.mean_f64(big) == 0.5
    assert ref.mean_f64(big).dtype == np.float64


def test_normwise_rel_error_known_answers():
    """||c - ref|| / ||ref||: c=[3,5], ref=[3,4] -> 1/5; invariant under a
    common scale; a transposed result is an error, not zero."""
    assert math.isclose(ref.normwise_rel_error([3.0, 5.0], [3.0, 4.0]), 0.2, rel_tol=1e-15)
    for s in (1e-3, 7.0, 1e6):
        assert math.isclose(ref.normwise_rel_error([3.0 * s, 5.0 * s], [3.0 * s, 4.0 * s]),
                            0.2, rel_tol=1e-12)
    a = np.array([[1.0, 2.0], [3.0, 4.0]])
    # ||a.T - a||_F = sqrt(2) * 1, ||a||_F = sqrt(30)
    assert math.isclose(ref.normwise_rel_error(a.T, a), math.sqrt(2.0 / 30.0), rel_tol=1e-14)
    assert ref.normwise_rel_error(-a, a) == 2.0


def test_fusion_chain_float32_path_against_python_loop():
    """fusion_chain (the reference's float32 np.sum) and fusion_chain_terms
    against per-element math-module loops; the float32 sum stays within
    float32 accumulation error of the exact row sum."""
    g = np.random.default_rng(8)
    x = g.standard_normal((4, 257)).astype(np.float32)
    r = g.uniform(0.5, 2.0, (1, 257)).astype(np.float32)
    terms = ref.fusion_chain_terms(x, r)
    assert terms.dtype == np.float32 and terms.shape == (4, 257)
    pos = np.array([[math.tanh(float(np.float32(x[i, j] * r[0, j]) + np.float32(1.0)))
                     * math.exp(-abs(float(x[i, j]))) for j in range(257)] for i in range(4)])
    neg = np.array([[math.log1p(float(np.float32(x[i, j] * x[i, j]))) for j in range(257)]
                    for i in range(4)])
    loop_t = pos - neg
    # each float32 term is within a few roundings of its two parts' size
    eps = float(np.finfo(np.float32).eps)
    assert np.all(np.abs(terms - loop_t) <= 4 * eps * (np.abs(pos) + np.abs(neg)))
    z = ref.fusion_chain(x, r)
    assert z.dtype == np.float32 and z.shape == (4,)
    exact = loop_t.sum(axis=1)
    bound = 257 * eps * (np.abs(pos) + np.abs(neg)).sum(axis=1)
    assert np.all(np.abs(z - exact) <= bound)
    # a dropped term (no log1p) or a wrong sign would be far outside the bound
    wrong = np.sum(np.tanh(x * r + np.float32(1.0)) * np.exp(-np.abs(x)), axis=1)
    assert np.all(np.abs(wrong - exact) > bound)


# Known answers for every entry of the oracle's unary table: exact values a
# plausible mistake (floor vs trunc, rint vs round-half-away, degrees vs
# radians, log2 vs log10, reciprocal vs negation ...) would violate.
_PI32 = np.float32(math.pi)
UNARY_KNOWN = {
    "neg_op": ([2.5, -0.0, 3.0], [-2.5, 0.0, -3.0]),
    "negative_op": ([2.5, -1.0], [-2.5, 1.0]),
    "positive_op": ([2.5, -1.0], [2.5, -1.0]),
    "abs_op": ([-2.5, 3.0, -0.0], [2.5, 3.0, 0.0]),
    "sign_op": ([-3.0, 0.0, 7.5], [-1.0, 0.0, 1.0]),
    "square_op": ([-3.0, 1.5], [9.0, 2.25]),
    "reciprocal_op": ([4.0, -0.5], [0.25, -2.0]),
    "sqrt_op": ([16.0, 2.25, 0.0], [4.0, 1.5, 0.0]),
    "cbrt_op": ([-27.0, 8.0, 0.125], [-3.0, 2.0, 0.5]),
    "exp_op": ([0.0], [1.0]),
    "exp2_op": ([3.0, -1.0, 10.0], [8.0, 0.5, 1024.0]),
    "expm1_op": ([0.0], [0.0]),
    "log_op": ([1.0], [0.0]),
    "log2_op": ([1024.0, 0.25, 1.0], [10.0, -2.0, 0.0]),
    "log10_op": ([1000.0, 0.01, 1.0], [3.0, -2.0, 0.0]),
    "log1p_op": ([0.0], [0.0]),
    "sin_op": ([0.0], [0.0]),
    "cos_op": ([0.0], [1.0]),
    "tan_op": ([0.0], [0.0]),
    "asin_op": ([0.0, 1.0], [0.0, np.float32(math.pi / 2)]),
    "acos_op": ([1.0, -1.0], [0.0, _PI32]),
    "atan_op": ([0.0, 1.0], [0.0, np.float32(math.pi / 4)]),
    "sinh_op": ([0.0], [0.0]),
    "cosh_op": ([0.0], [1.0]),
    "tanh_op": ([0.0, 20.0, -20.0], [0.0, 1.0, -1.0]),
    "asinh_op": ([0.0], [0.0]),
    "acosh_op": ([1.0], [0.0]),
    "atanh_op": ([0.0], [0.0]),
    # halves and negatives separate floor / ceil / rint / trunc / round
    "floor_op": ([-2.5, -1.5, -0.5, 0.5, 1.5, 2.5], [-3.0, -2.0, -1.0, 0.0, 1.0, 2.0]),
    "ceil_op": ([-2.5, -1.5, -0.5, 0.5, 1.5, 2.5], [-2.0, -1.0, -0.0, 1.0, 2.0, 3.0]),
    "rint_op": ([-2.5, -1.5, -0.5, 0.5, 1.5, 2.5], [-2.0, -2.0, -0.0, 0.0, 2.0, 2.0]),
    "trunc_op": ([-2.5, -1.5, -0.5, 0.5, 1.5, 2.5], [-2.0, -1.0, -0.0, 0.0, 1.0, 2.0]),
    "degrees_op": ([_PI32, 0.0], [np.float32(180.0), 0.0]),
    "radians_op": ([180.0, 90.0], [_PI32, np.float32(math.pi / 2)]),
    "invert_op": ([0, -1, 5], [-1, 0, -6]),
    "logical_not_op": ([0.0, 2.0, -0.0], [True, False, True]),
    "isnan_op": ([np.nan, 1.0, np.inf], [True, False, False]),
    "isinf_op": ([np.nan, -np.inf, np.inf, 1.0], [False, True, True, False]),
    "isfinite_op": ([np.nan, np.inf, 1.0], [False, False, True]),
    "signbit_op": ([-0.0, 0.0, -1.0, 2.0], [True, False, True, False]),
}


# float32 library functions (not correctly rounded in NumPy): ULP-bounded
_UNARY_LIBM = frozenset({"cbrt_op", "exp2_op", "log2_op", "log10_op", "asin_op", "acos_op",
                         "atan_op", "degrees_op", "radians_op"})


def test_unary_table_known_answers_cover_every_entry():
    assert set(UNARY_KNOWN) == set(ref.UNARY), set(ref.UNARY) ^ set(UNARY_KNOWN)
    for op, (xs, want) in UNARY_KNOWN.items():
        dt = np.int32 if op == "invert_op" else np.float32
        got = ref.unary(op, np.array(xs, dtype=dt))
        w = np.array(want, dtype=got.dtype)
        assert got.dtype in (np.dtype(dt), np.dtype(np.bool_)), (op, got.dtype)
        if op in _UNARY_LIBM:  # NumPy's float32 libm: within 2 ULP
            assert int(ref.ulp_distance(got, w).max()) <= 2, (op, got, w)
            continue
        assert np.array_equal(got, w), (op, got, w)
        if got.dtype.kind == "f":  # signed zeros are part of the answer
            assert np.array_equal(np.signbit(got), np.signbit(w)), (op, got, w)


BINARY_KNOWN = {
    "add_op": ([1.5, -2.0], [2.25, 2.0], [3.75, 0.0]),
    "sub_op": ([1.5, -2.0], [2.25, 2.0], [-0.75, -4.0]),
    "mul_op": ([1.5, -2.0], [2.0, 3.0], [3.0, -6.0]),
    "div_op": ([1.0, -3.0], [4.0, 2.0], [0.25, -1.5]),
    "pow_op": ([2.0, 9.0, 4.0], [10.0, 0.5, -1.0], [1024.0, 3.0, 0.25]),
    "mod_op": ([-7.0, 7.0], [3.0, -3.0], [2.0, -2.0]),
    "fmod_op": ([-7.0, 7.0], [3.0, -3.0], [-1.0, 1.0]),
    "floor_divide_op": ([-7.0, 7.0], [2.0, -2.0], [-4.0, -4.0]),
    "min_op": ([1.0, np.nan], [2.0, 0.0], [1.0, np.nan]),
    "max_op": ([1.0, np.nan], [2.0, 0.0], [2.0, np.nan]),
    "fmin_op": ([1.0, np.nan], [2.0, 0.0], [1.0, 0.0]),
    "fmax_op": ([1.0, np.nan], [2.0, 0.0], [2.0, 0.0]),
    "atan2_op": ([1.0, 0.0], [1.0, -1.0], [np.float32(math.pi / 4), _PI32]),
    "hypot_op": ([3.0, 5.0], [4.0, 12.0], [5.0, 13.0]),
    "copysign_op": ([2.0, -3.0], [-1.0, 0.0], [-2.0, 3.0]),
    "logaddexp_op": ([0.0], [0.0], [np.float32(math.log(2.0))]),
    "logaddexp2_op": ([1.0, 3.0], [1.0, 3.0], [2.0, 4.0]),
    "heaviside_op": ([-1.0, 0.0, 2.0], [0.5, 0.5, 0.5], [0.0, 0.5, 1.0]),
    "nextafter_op": ([1.0], [2.0], [np.nextafter(np.float32(1.0), np.float32(2.0))]),
    "bit_and_op": ([12, -1], [10, 7], [8, 7]),
    "bit_or_op": ([12, -8], [10, 1], [14, -7]),
    "bit_xor_op": ([12, -1], [10, 0], [6, -1]),
    "lshift_op": ([1, 3], [4, 1], [16, 6]),
    "rshift_op": ([16, -16], [2, 2], [4, -4]),
    "logical_and_op": ([1.0, 0.0, 2.0], [1.0, 1.0, 0.0], [True, False, False]),
    "logical_or_op": ([1.0, 0.0, 0.0], [0.0, 0.0, 3.0], [True, False, True]),
    "logical_xor_op": ([1.0, 0.0, 1.0], [1.0, 0.0, 0.0], [False, False, True]),
}


def test_binary_table_known_answers_cover_every_entry():
    assert set(BINARY_KNOWN) == set(ref.BINARY), set(ref.BINARY) ^ set(BINARY_KNOWN)
    for op, (xa, xb, want) in BINARY_KNOWN.items():
        dt = np.int32 if op in ("bit_and_op", "bit_or_op", "bit_xor_op", "lshift_op",
                                "rshift_op") else np.float32
        got = ref.binary(op, np.array(xa, dtype=dt), np.array(xb, dtype=dt))
        w = np.array(want, dtype=got.dtype)
        if op in ("atan2_op", "logaddexp_op"):  # float32 libm: within 2 ULP
            assert int(ref.ulp_distance(got, w).max()) <= 2, (op, got, w)
            continue
        assert np.array_equal(got, w, equal_nan=got.dtype.kind == "f"), (op, got, w)


def test_correctly_rounded_helper():
    # float64 evaluation rounded once: sqrt(2) and e to the nearest float32
    assert ref.correctly_rounded(np.sqrt, np.float32(2.0)) == np.float32(1.4142135)
    assert ref.correctly_rounded(np.exp, np.float32(1.0)) == np.float32(2.7182817)
    got = ref.correctly_rounded(np.sin, np.array([0.5], np.float32))
    assert got.dtype == np.float32 and got[0] == np.float32(math.sin(0.5))


def test_every_oracle_function_is_exercised_here():
    """Each public function of the NumPy restatement is called by a test in
    this file (so none is left without a check)."""
    import inspect
    src = open(__file__).read()
    names = [n for n, f in inspect.getmembers(ref, inspect.isfunction)
             if f.__module__ == ref.__name__ and not n.startswith("_")]
    missing = [n for n in names if f"ref.{n}(" not in src]
    assert not missing, missing
