"""Elementwise parity on the GPU against the oracle (NumPy restatement of the
reference's CPU path).  Bars: integer ops bit-exact; float add/sub/mul/div,
sqrt, abs, neg, square, rounding, floor_divide, mod bit-exact; float32
transcendentals within 2 ULP of NumPy and of the float64 evaluation."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd import _abi
from macmetalpy_amd.workloads import c1_inputs, c2_float_inputs, c2_int_inputs
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

SPECIALS32 = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45,
                       3.4e38, -3.4e38, 0.5, -0.5, 2.5, -2.5, 1e-30, 100.0], np.float32)

EXACT_UNARY = ["neg_op", "positive_op", "abs_op", "sign_op", "square_op", "reciprocal_op",
               "sqrt_op", "floor_op", "ceil_op", "rint_op", "trunc_op", "degrees_op",
               "radians_op"]
# (op, float64 function, domain) for the ULP-checked transcendentals
TRANSCENDENTAL = [
    ("cbrt_op", np.cbrt, (-1e6, 1e6)), ("exp_op", np.exp, (-87, 88)),
    ("exp2_op", np.exp2, (-126, 127)), ("expm1_op", np.expm1, (-20, 20)),
    ("log_op", np.log, (1e-30, 1e30)), ("log2_op", np.log2, (1e-30, 1e30)),
    ("log10_op", np.log10, (1e-30, 1e30)), ("log1p_op", np.log1p, (-0.999, 1e6)),
    ("sin_op", np.sin, (-100, 100)), ("cos_op", np.cos, (-100, 100)),
    ("tan_op", np.tan, (-1.5, 1.5)), ("asin_op", np.arcsin, (-1, 1)),
    ("acos_op", np.arccos, (-1, 1)), ("atan_op", np.arctan, (-1e4, 1e4)),
    ("sinh_op", np.sinh, (-80, 80)), ("cosh_op", np.cosh, (-80, 80)),
    ("tanh_op", np.tanh, (-20, 20)), ("asinh_op", np.arcsinh, (-1e4, 1e4)),
    ("acosh_op", np.arccosh, (1, 1e4)), ("atanh_op", np.arctanh, (-0.999, 0.999)),
]


def _dev_unary(op, x):
    from macmetalpy_amd import _elementwise as ew
    return ew.unary(op, cp.array(x)).get()


def _dev_binary(op, a, b):
    from macmetalpy_amd import _elementwise as ew
    aa = cp.array(a) if isinstance(a, np.ndarray) else a
    bb = cp.array(b) if isinstance(b, np.ndarray) else b
    return ew.binary(op, aa, bb).get()


def _bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.dtype == b.dtype, (a.dtype, b.dtype)
    assert a.shape == b.shape
    if a.dtype.kind == "f":
        nan = np.isnan(a) & np.isnan(b)
        ua = a.view(f"u{a.itemsize}")
        ub = b.view(f"u{b.itemsize}")
        bad = (ua != ub) & ~nan
        assert not bad.any(), f"{bad.sum()} mismatches, first at {np.argmax(bad)}: " \
                              f"{a.ravel()[np.argmax(bad)]} vs {b.ravel()[np.argmax(bad)]}"
    else:
        assert np.array_equal(a, b)


@pytest.mark.parametrize("op", EXACT_UNARY)
@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.float64])
def test_exact_unary(op, dtype):
    x = np.concatenate([SPECIALS32.astype(dtype),
                        (np.random.default_rng(0).standard_normal(5000) * 50).astype(dtype)])
    _bits_equal(_dev_unary(op, x), ref.unary(op, x))


# float32 ops evaluated through float64 on the device (<= 1 ULP of exact);
# NumPy's own float32 results for these are up to 3 ULP from exact.
VIA_F64 = {"exp2_op", "log10_op", "asin_op", "acos_op", "atan2_op"}


def _check_f32_ulp(op, got, want_np, want_cr, check_cr=True):
    d_np = ref.ulp_distance(got, want_np)
    d_cr = ref.ulp_distance(got, want_cr)
    if op in VIA_F64:
        assert int(d_cr.max()) <= 1
        np_err = ref.ulp_distance(want_np, want_cr)
        assert np.all(d_np <= np.maximum(2, np_err + 1))
    else:
        assert int(d_np.max()) <= 2
        if check_cr:
            assert int(d_cr.max()) <= 2


@pytest.mark.parametrize("op,fn64,dom", TRANSCENDENTAL)
def test_transcendental_f32_ulp(op, fn64, dom):
    x = np.random.default_rng(1).uniform(*dom, 200000).astype(np.float32)
    x = np.concatenate([x, SPECIALS32])
    got = _dev_unary(op, x)
    _check_f32_ulp(op, got, ref.unary(op, x), ref.correctly_rounded(fn64, x))


@pytest.mark.parametrize("op,fn64,dom", TRANSCENDENTAL[:12])
def test_transcendental_f16_f64(op, fn64, dom):
    x = np.random.default_rng(2).uniform(*dom, 20000)
    x16 = x.astype(np.float16)
    assert int(ref.ulp_distance(_dev_unary(op, x16), ref.unary(op, x16)).max()) <= 1
    x64 = x.astype(np.float64)
    assert int(ref.ulp_distance(_dev_unary(op, x64), ref.unary(op, x64)).max()) <= 2


@pytest.mark.parametrize("op", ["add_op", "sub_op", "mul_op", "div_op", "floor_divide_op",
                                "mod_op", "max_op", "min_op", "fmax_op", "fmin_op",
                                "copysign_op", "fmod_op", "heaviside_op", "nextafter_op"])
@pytest.mark.parametrize("dtype", [np.float32, np.float64, np.float16])
def test_exact_binary_float(op, dtype):
    g = np.random.default_rng(3)
    a = np.concatenate([np.repeat(SPECIALS32, len(SPECIALS32)),
                        (g.standard_normal(20000) * 100)]).astype(dtype)
    b = np.concatenate([np.tile(SPECIALS32, len(SPECIALS32)),
                        (g.standard_normal(20000) * 10)]).astype(dtype)
    _bits_equal(_dev_binary(op, a, b), ref.binary(op, a, b))


@pytest.mark.parametrize("op", ["pow_op", "atan2_op", "hypot_op", "logaddexp_op",
                                "logaddexp2_op"])
def test_binary_transcendental_f32(op):
    g = np.random.default_rng(4)
    a = np.abs(g.standard_normal(100000)).astype(np.float32) * 4
    b = (g.standard_normal(100000) * 3).astype(np.float32)
    got = _dev_binary(op, a, b)
    want = ref.binary(op, a, b)
    fn64 = {"pow_op": np.power, "atan2_op": np.arctan2, "hypot_op": np.hypot,
            "logaddexp_op": np.logaddexp, "logaddexp2_op": np.logaddexp2}[op]
    with np.errstate(all="ignore"):
        cr = fn64(a.astype(np.float64), b.astype(np.float64)).astype(np.float32)
    _check_f32_ulp(op, got, want, cr, check_cr=False)


INT_EDGE = np.array([0, 1, -1, 2, -2, 7, -7, 100, -100, 2 ** 31 - 1, -2 ** 31,
                     12345, -12345], np.int64)


@pytest.mark.parametrize("op", ["add_op", "sub_op", "mul_op", "floor_divide_op", "mod_op",
                                "max_op", "min_op", "fmod_op", "fmax_op", "fmin_op"])
@pytest.mark.parametrize("dtype", [np.int32, np.int16, np.int64, np.uint32, np.uint16,
                                   np.uint64])
def test_integer_binary_bit_exact(op, dtype):
    info = np.iinfo(dtype)
    edge = np.clip(INT_EDGE, info.min, info.max)
    edge = np.concatenate([edge, [info.min, info.max]]).astype(dtype)
    a = np.repeat(edge, len(edge))
    b = np.tile(edge, len(edge))
    g = np.random.default_rng(5)
    ra = g.integers(info.min, info.max, 50000, dtype=dtype, endpoint=True)
    rb = g.integers(info.min, info.max, 50000, dtype=dtype, endpoint=True)
    rb2 = g.integers(-1000 if info.min < 0 else 0, 1000, 50000, dtype=dtype)
    a = np.concatenate([a, ra, ra])
    b = np.concatenate([b, rb, rb2])
    _bits_equal(_dev_binary(op, a, b), ref.binary(op, a, b))


@pytest.mark.parametrize("dtype", [np.int32, np.int64, np.uint16])
def test_integer_power_and_unary(dtype):
    g = np.random.default_rng(6)
    a = g.integers(0 if dtype == np.uint16 else -50, 50, 10000).astype(dtype)
    e = g.integers(0, 12, 10000).astype(dtype)
    _bits_equal(_dev_binary("pow_op", a, e), ref.binary("pow_op", a, e))
    for op in ["neg_op", "abs_op", "sign_op", "square_op", "floor_op", "trunc_op"]:
        _bits_equal(_dev_unary(op, a), ref.unary(op, a))


def test_integer_negative_power_raises():
    with pytest.raises(ValueError, match="negative integer powers"):
        (cp.array(np.array([2, 3], np.int32)) ** cp.array(np.array([1, -1], np.int32))).get()


def test_c2_int_semantics_sample():
    a, b = c2_int_inputs(1 << 20)
    _bits_equal(_dev_binary("floor_divide_op", a, b), ref.floor_divide(a, b))
    _bits_equal(_dev_binary("mod_op", a, b), ref.mod(a, b))
    ga, gb = cp.array(a), cp.array(b)
    _bits_equal((ga // gb).get(), a // b)
    _bits_equal((ga % gb).get(), a % b)
    _bits_equal(cp.floor_divide(ga, gb).get(), np.floor_divide(a, b))
    _bits_equal(cp.mod(ga, gb).get(), np.mod(a, b))


def test_c2_full_size_properties():
    """2^28 elements: float add bit-exact over every element; sin within
    2 ULP of NumPy and of the correctly rounded value over a contiguous
    2^24-element block plus a strided sample of the rest; int
    floor_divide/mod: division identity and remainder-sign invariants over
    every element."""
    n = 1 << 28
    a, b = c2_float_inputs(n)
    ga, gb = cp.array(a), cp.array(b)
    s = (ga + gb).get()
    want = np.add(a, b)
    assert s.view(np.uint32).tobytes() == want.view(np.uint32).tobytes()
    del s, want
    idx = np.arange(0, n, 4099)
    sn = cp.sin(ga).get()
    blk = slice(n // 2, n // 2 + (1 << 24))
    assert int(ref.ulp_distance(sn[blk], np.sin(a[blk])).max()) <= 2
    assert int(ref.ulp_distance(sn[blk], ref.correctly_rounded(np.sin, a[blk])).max()) <= 2
    assert int(ref.ulp_distance(sn[idx], np.sin(a[idx])).max()) <= 2
    del sn, ga, gb, a, b
    ai, bi = c2_int_inputs(n)
    gai, gbi = cp.array(ai), cp.array(bi)
    q = (gai // gbi).get()
    r = cp.mod(gai, gbi).get()
    assert np.array_equal(q.astype(np.int64) * bi + r, ai)
    pos = bi > 0
    assert np.all(np.where(pos, (r >= 0) & (r < bi), (r <= 0) & (r > bi)))
    _bits_equal(q[idx], np.floor_divide(ai[idx], bi[idx]))


def test_promotion_scalars_broadcast():
    g = np.random.default_rng(7)
    x32 = g.standard_normal((64, 33)).astype(np.float32)
    i32 = g.integers(-100, 100, (64, 33), dtype=np.int32)
    r = g.standard_normal((1, 33)).astype(np.float32)
    c = g.standard_normal((64, 1)).astype(np.float32)
    X, I, R, Cc = cp.array(x32), cp.array(i32), cp.array(r), cp.array(c)
    _bits_equal((X + 1.0).get(), x32 + 1.0)
    _bits_equal((2.5 - X).get(), 2.5 - x32)
    _bits_equal((I + 1.5).get(), i32 + 1.5)          # float64 (NumPy promotion)
    _bits_equal((I * 3).get(), i32 * 3)
    with np.errstate(all="ignore"):
        _bits_equal((I / I).get(), i32 / i32)        # true_divide of ints: float64
    _bits_equal((X * R).get(), x32 * r)
    _bits_equal((X * R + Cc).get(), x32 * r + c)
    _bits_equal((I + X).get(), i32 + x32)            # float64
    _bits_equal((I // 7).get(), i32 // 7)
    with np.errstate(all="ignore"):
        _bits_equal((7 % I[:, :1] + I).get(), 7 % i32[:, :1] + i32)
    _bits_equal((X[::2, 1::3] * 2.0).get(), x32[::2, 1::3] * 2.0)
    _bits_equal((X.T + 1.0).get(), x32.T + 1.0)
    sin_i = cp.sin(I).get()
    assert sin_i.dtype == np.float64
    assert int(ref.ulp_distance(sin_i, np.sin(i32)).max()) <= 2
    _bits_equal((X > 0.5).get(), x32 > 0.5)
    _bits_equal((I == I.T.T).get(), np.ones_like(i32, dtype=bool))
    _bits_equal((X ** 2).get(), x32 ** 2)
    _bits_equal((abs(X) ** 0.5).get(), np.abs(x32) ** 0.5)


def test_fusion_c1_matches_oracle_and_unfused():
    x_np = c1_inputs()
    x = cp.array(x_np)
    y = cp.sqrt(cp.abs(x)) + cp.exp(-x ** 2)
    assert y._fusion_node is not None
    fused = y.get()
    want = ref.fused_elementwise(x_np)
    assert int(ref.ulp_distance(fused, want).max()) <= 2
    cp.set_config(fusion=False)
    x2 = cp.array(x_np)
    unfused = (cp.sqrt(cp.abs(x2)) + cp.exp(-x2 ** 2)).get()
    cp.set_config(fusion=True)
    _bits_equal(fused, unfused)


def test_fusion_depth_and_dependents():
    x_np = np.linspace(-2, 2, 4097, dtype=np.float32)
    x = cp.array(x_np)
    y = x
    for _ in range(40):                      # beyond the depth cap of 16
        y = cp.sin(y) + 0.5
    want = x_np
    for _ in range(40):
        want = np.sin(want) + np.float32(0.5)
    assert int(ref.ulp_distance(y.get(), want).max()) <= 8
    # a pending expression must not see a later in-place write to its input
    a = cp.array(np.ones(1000, np.float32))
    lazy = a * 3.0
    a[...] = 5.0
    assert np.all(lazy.get() == 3.0)
    a += 1.0
    assert np.all(a.get() == 6.0)


def test_astype_and_copies():
    g = np.random.default_rng(8)
    x = (g.standard_normal((50, 70)) * 1000).astype(np.float32)
    X = cp.array(x)
    for dt in [np.float16, np.float64, np.int32, np.int16, np.uint16, np.int64, np.bool_]:
        with np.errstate(invalid="ignore"):
            want = x.astype(dt)
        got = X.astype(dt).get()
        if np.dtype(dt).kind in "iu":
            ok = np.abs(x) < np.iinfo(dt).max
            assert np.array_equal(got[ok], want[ok])
        else:
            _bits_equal(got, want)
    _bits_equal(X[3:40:3, ::-2].copy().get(), x[3:40:3, ::-2])
    _bits_equal(X.T.get(), x.T)


@pytest.mark.parametrize("src", [np.float16, np.float32, np.float64])
def test_float_to_unsigned_casts_wrap(src):
    """Negative floats cast to unsigned integers wrap through int64, as
    NumPy's C casts on x86-64 (-1.0 -> 65535 for uint16), in the copy
    kernels and in fused casts; float64 values of 2^63 and more go to
    uint64 directly."""
    x = np.array([-1.0, -2.5, -300.75, 0.0, 1.9, 250.5, -65535.0, 40000.0], src)
    if src == np.float64:
        x = np.concatenate([x, [2.0 ** 63, 1.5 * 2.0 ** 63, -2.0 ** 40]])
    for dt in (np.uint16, np.uint32, np.uint64):
        with np.errstate(invalid="ignore"):
            want = x.astype(dt)
        ok = np.isfinite(x) & ((np.abs(x.astype(np.float64)) < np.iinfo(dt).max) if dt != np.uint64
                               else True)
        assert np.array_equal(cp.array(x).astype(dt).get()[ok], want[ok]), dt
        assert np.array_equal((cp.array(x) + 0).astype(dt).get()[ok], want[ok]), dt


def test_empty_and_tiny():
    e = cp.array(np.zeros((0, 3), np.float32))
    assert (cp.sin(e) + 1).shape == (0, 3)
    one = cp.array(np.array([2.0], np.float32))
    assert float((one * one).get()[0]) == 4.0
    z = cp.array(np.float32(3.0))
    assert float((z + 1).get()) == 4.0


def test_log1p_f32_dense_sweep_and_specials():
    """float32 log1p (own implementation: exact range reduction plus a
    fitted polynomial) over every 61st bit pattern of (-1, +inf): at most
    1 ULP from the correctly rounded value, and NumPy's special values."""
    pos = np.arange(0, 0x7F800000, 61, dtype=np.int64).astype(np.uint32).view(np.float32)
    neg = np.arange(0x80000000, 0xBF800000, 61, dtype=np.int64).astype(np.uint32).view(np.float32)
    for x in (pos, neg):
        got = _dev_unary("log1p_op", x)
        d = ref.ulp_distance(got, ref.correctly_rounded(np.log1p, x))
        assert int(d.max()) <= 1, x[int(np.argmax(d))]
    sp = np.array([-1.0, -1.5, -np.inf, np.nan, np.inf, 0.0, -0.0, 1e-30, -1e-30, 1e-45,
                   -0.99999994, 3.4e38], np.float32)
    got = _dev_unary("log1p_op", sp)
    with np.errstate(all="ignore"):
        want = np.log1p(sp)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
