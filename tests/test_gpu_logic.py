"""Bitwise, shift, logical, predicate, where / clip and any / all /
count_nonzero parity on the GPU against the oracle (NumPy, the reference's
CPU path).  Bar: bit-exact values and identical dtypes and shapes."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd import _elementwise as ew
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

INT_DTYPES = [np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64]
FLOAT_DTYPES = [np.float16, np.float32, np.float64]


def _same(got, want, nan_bits=True):
    """Identical dtype, shape and bits; with nan_bits=False a NaN only has
    to meet a NaN (any sign or payload)."""
    got, want = np.asarray(got), np.asarray(want)
    assert got.dtype == want.dtype, (got.dtype, want.dtype)
    assert got.shape == want.shape, (got.shape, want.shape)
    if got.dtype.kind == "f":
        u = f"u{got.itemsize}"
        if not nan_bits:
            gn, wn = np.isnan(got), np.isnan(want)
            assert np.array_equal(gn, wn)
            got, want = got[~gn], want[~wn]
        assert np.array_equal(got.view(u), want.view(u))
    else:
        assert np.array_equal(got, want)


def _ints(dtype, n, seed):
    info = np.iinfo(dtype)
    rng = np.random.default_rng(seed)
    x = rng.integers(info.min, info.max, n, dtype=dtype, endpoint=True)
    x[:4] = [info.min, info.max, 0, 1]
    return x


def _floats(dtype, n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(n) * 3).astype(dtype)
    sp = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -1.0], dtype=dtype)
    sp[1] = -np.abs(sp[1])
    x[:len(sp)] = sp
    return x


@pytest.mark.parametrize("dtype", INT_DTYPES + [np.bool_])
@pytest.mark.parametrize("op", ["bit_and_op", "bit_or_op", "bit_xor_op"])
def test_bitwise_binary(op, dtype):
    n = 10007
    if dtype is np.bool_:
        rng = np.random.default_rng(1)
        a, b = rng.random(n) < 0.5, rng.random(n) < 0.5
    else:
        a, b = _ints(dtype, n, 1), _ints(dtype, n, 2)
    _same(ew.binary(op, cp.array(a), cp.array(b)).get(), ref.binary(op, a, b))
    # Python scalar operand (weak) on either side
    _same(ew.binary(op, cp.array(a), 1).get(), ref.binary(op, a, 1))
    _same(ew.binary(op, True, cp.array(a)).get(), ref.binary(op, True, a))


@pytest.mark.parametrize("dtype", INT_DTYPES)
def test_shifts_every_count(dtype):
    """All counts in [-3, bits + 3) against every test value: NumPy's
    out-of-range rules (0, or -1 for negative values shifted right)."""
    info = np.iinfo(dtype)
    counts = np.arange(-3 if info.min < 0 else 0, info.bits + 3)
    vals = _ints(dtype, 64, 3)
    a = np.repeat(vals, len(counts)).astype(dtype)
    b = np.tile(counts, len(vals)).astype(dtype)
    for op in ("lshift_op", "rshift_op"):
        _same(ew.binary(op, cp.array(a), cp.array(b)).get(), ref.binary(op, a, b))
    _same(ew.binary("lshift_op", cp.array(vals), 3).get(), ref.binary("lshift_op", vals, 3))


@pytest.mark.parametrize("dtype", INT_DTYPES + [np.bool_])
def test_invert(dtype):
    x = (np.random.default_rng(4).random(999) < 0.5) if dtype is np.bool_ else _ints(dtype, 999, 4)
    _same(ew.unary("invert_op", cp.array(x)).get(), ref.unary("invert_op", x))
    _same((~cp.array(x)).get(), ~x)


def test_bitwise_rejects_floats():
    a = cp.array(np.ones(4, np.float32))
    for op in ("bit_and_op", "lshift_op"):
        with pytest.raises(TypeError):
            ew.binary(op, a, a)
    with pytest.raises(TypeError):
        ew.unary("invert_op", a)


@pytest.mark.parametrize("dtype", FLOAT_DTYPES + INT_DTYPES + [np.bool_])
@pytest.mark.parametrize("op", ["isnan_op", "isinf_op", "isfinite_op", "signbit_op",
                                "logical_not_op"])
def test_predicates(op, dtype):
    if np.dtype(dtype).kind == "f":
        x = _floats(dtype, 4099, 5)
    elif dtype is np.bool_:
        x = np.random.default_rng(5).random(4099) < 0.5
    else:
        x = _ints(dtype, 4099, 5)
    _same(ew.unary(op, cp.array(x)).get(), ref.unary(op, x))


@pytest.mark.parametrize("op", ["logical_and_op", "logical_or_op", "logical_xor_op"])
def test_logical_mixed_dtypes(op):
    f = _floats(np.float32, 3001, 6)
    f[::3] = 0.0
    i = _ints(np.int16, 3001, 7)
    i[::5] = 0
    h = _floats(np.float16, 3001, 8)
    for a, b in ((f, i), (i, h), (h, f), (f, f)):
        _same(ew.binary(op, cp.array(a), cp.array(b)).get(), ref.binary(op, a, b))
    _same(ew.binary(op, cp.array(f), 0).get(), ref.binary(op, f, 0))


def test_dunders_inplace_and_array_ufunc():
    a = _ints(np.int32, 2048, 9)
    b = _ints(np.int32, 2048, 10)
    ca, cb = cp.array(a), cp.array(b)
    _same((ca & cb).get(), a & b)
    _same((ca | 7).get(), a | 7)
    _same((5 ^ cb).get(), 5 ^ b)
    _same((ca << 3).get(), a << 3)
    _same((ca >> 2).get(), a >> 2)
    _same(np.bitwise_and(ca, cb).get(), np.bitwise_and(a, b))
    _same(np.isnan(cp.array(_floats(np.float32, 64, 1))).get(),
          np.isnan(_floats(np.float32, 64, 1)))
    c = a.copy()
    cc = cp.array(c) + 0  # device-resident, so a basic slice is a device view
    view = cc[:1024]
    cc &= 0xFF
    cc |= 0x100
    cc ^= 3
    cc <<= 1
    cc >>= 2
    c &= 0xFF
    c |= 0x100
    c ^= 3
    c <<= 1
    c >>= 2
    _same(cc.get(), c)
    _same(view.get(), c[:1024])


def test_fused_chain_with_broadcast_and_unfused_mode():
    rng = np.random.default_rng(12)
    x = _ints(np.int64, 64 * 300, 12).reshape(64, 300)
    r = rng.integers(0, 70, (1, 300)).astype(np.int64)
    want = ((x >> r) & 0xFFFF) ^ (x << 1)
    got = ((cp.array(x) >> cp.array(r)) & 0xFFFF) ^ (cp.array(x) << 1)
    _same(got.get(), want)
    cp.set_config(fusion=False)
    got2 = ((cp.array(x) >> cp.array(r)) & 0xFFFF) ^ (cp.array(x) << 1)
    _same(got2.get(), want)


# ------------------------------------------------------------ where / clip
@pytest.mark.parametrize("xdt,ydt", [(np.float32, np.float32), (np.int32, np.float64),
                                     (np.int16, np.uint16), (np.float16, np.float32),
                                     (np.bool_, np.int64)])
def test_where_dtypes_and_broadcast(xdt, ydt):
    rng = np.random.default_rng(13)
    cond = rng.random((37, 129)) < 0.5
    x = (rng.standard_normal((37, 129)) * 100).astype(xdt)
    y = (rng.standard_normal((1, 129)) * 100).astype(ydt)
    _same(cp.where(cp.array(cond), cp.array(x), cp.array(y)).get(), ref.where(cond, x, y))


def test_where_scalars_truthy_conditions_and_lazy_inputs():
    rng = np.random.default_rng(14)
    x = _floats(np.float32, 5000, 14)
    c = _floats(np.float32, 5000, 15)  # float condition: NaN and -0.0 included
    _same(cp.where(cp.array(c), cp.array(x), -1.5).get(), ref.where(c, x, np.float32(-1.5)))
    _same(cp.where(cp.array(c), 2, cp.array(x)).get(), ref.where(c, 2, x))
    _same(cp.where(cp.array(c), 1, 0).get(), ref.where(c, 1, 0))
    cx = cp.array(x)
    got = cp.where(cx > 0, cp.sqrt(cx), cx * 2.0)  # lazy condition and operands
    with np.errstate(invalid="ignore"):
        want = np.where(x > 0, np.sqrt(x), x * np.float32(2.0))
    _same(got.get(), want)
    _same(cp.where(cp.array(np.zeros((0, 3), bool)), 1.0, 2.0).get(), np.where(np.zeros((0, 3), bool), 1.0, 2.0))
    got1 = cp.where(cp.array(c))
    assert len(got1) == c.ndim
    for g, w in zip(got1, np.where(c)):
        _same(g.get(), w)


@pytest.mark.parametrize("dtype", FLOAT_DTYPES + [np.int32, np.uint16, np.int64])
def test_clip(dtype):
    if np.dtype(dtype).kind == "f":
        a = _floats(dtype, 7001, 16)
        lo, hi = -1.0, 2.0
    else:
        a = _ints(dtype, 7001, 16)
        lo, hi = 10, 5000
    _same(cp.clip(cp.array(a), lo, hi).get(), ref.clip(a, lo, hi))
    _same(cp.clip(cp.array(a), None, hi).get(), ref.clip(a, None, hi))
    _same(cp.clip(cp.array(a), lo, None).get(), ref.clip(a, lo, None))
    _same(cp.array(a).clip(hi, lo).get(), ref.clip(a, hi, lo))  # lo > hi -> hi
    lo_arr = np.sort(a[:16]).reshape(1, 16)
    a2 = a[:16 * 400].reshape(400, 16)
    _same(cp.clip(cp.array(a2), cp.array(lo_arr), hi).get(), ref.clip(a2, lo_arr, hi))


def test_clip_nan_bounds_and_int_to_float():
    """A NaN bound makes every element NaN.  NumPy's scalar-bound loop
    returns the bound's NaN and its array-bound loop the element's NaN (a
    negative NaN stays negative there); which NaN is not compared."""
    a = _floats(np.float32, 1000, 17)
    _same(cp.clip(cp.array(a), np.float32(np.nan), np.float32(1.0)).get(),
          ref.clip(a, np.float32(np.nan), np.float32(1.0)), nan_bits=False)
    i = _ints(np.int32, 1000, 18)
    _same(cp.clip(cp.array(i), 0.5, 1e6).get(), ref.clip(i, 0.5, 1e6))


# ------------------------------------------------ any / all / count_nonzero
@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.int32, np.bool_, np.uint64])
def test_any_all_count_nonzero_axes(dtype):
    rng = np.random.default_rng(19)
    shape = (6, 5, 1031)
    if np.dtype(dtype).kind == "f":
        x = (rng.random(shape) < 0.01).astype(dtype)
        x[0, 0, 7] = np.nan
        x[1] = 1.0
        x[2] = 0.0
        x[3, :, 5] = -0.0
    else:
        x = (rng.random(shape) < 0.01).astype(dtype)
        x[1] = 1
        x[2] = 0
    cx = cp.array(x)
    for axis in (None, 0, 1, 2, -1, (0, 2), (1, 2)):
        for keep in (False, True):
            _same(cp.any(cx, axis=axis, keepdims=keep).get(), ref.any_(x, axis, keep))
            _same(cp.all(cx, axis=axis, keepdims=keep).get(), ref.all_(x, axis, keep))
            got = cp.count_nonzero(cx, axis=axis, keepdims=keep)
            want = ref.count_nonzero(x, axis, keep)
            if axis is None and not keep:
                assert got == want and type(got) is int
            else:
                _same(got.get(), np.asarray(want, dtype=np.int64))
    _same(cx.any(axis=2).get(), x.any(axis=2))
    _same(cx.all().get(), np.asarray(x.all()))


def test_any_all_empty_and_lazy():
    z = np.zeros((4, 0), np.float32)
    _same(cp.any(cp.array(z), axis=1).get(), ref.any_(z, 1))
    _same(cp.all(cp.array(z), axis=1).get(), ref.all_(z, 1))
    _same(cp.all(cp.array(z)).get(), np.asarray(ref.all_(z)))
    x = _floats(np.float32, 1 << 20, 20)
    cx = cp.array(x)
    with np.errstate(invalid="ignore"):
        _same(cp.any(cp.sqrt(cx) > 1.5).get(), np.asarray(np.any(np.sqrt(x) > 1.5)))
        _same(cp.all(cp.isfinite(cx * 0.0)).get(), np.asarray(np.all(np.isfinite(x * 0.0))))
    assert cp.count_nonzero(cp.isnan(cx)) == int(np.count_nonzero(np.isnan(x)))


# ------------------------------------------------------- where= masks
def test_reductions_with_where_masks():
    rng = np.random.default_rng(30)
    x = rng.standard_normal((37, 515)).astype(np.float32)
    x[3, 7] = np.nan
    m_row = rng.random(515) < 0.6               # broadcast along rows
    m_full = rng.random((37, 515)) < 0.5
    m_full[3, 7] = False                        # the NaN is masked out
    cx = cp.array(x)
    x64 = x.astype(np.float64)
    for m in (m_row, m_full, cp.array(m_full)):
        mn = m.get() if hasattr(m, "get") else m
        for axis in (None, 1, 0):
            got = cp.sum(cx, axis=axis, where=m).get()
            want = np.sum(x64, axis=axis, where=mn)
            assert np.allclose(got, want, rtol=1e-5, atol=1e-5, equal_nan=True)
            with np.errstate(all="ignore"):
                gm = cp.mean(cx, axis=axis, where=m).get()
                wm = np.mean(x64, axis=axis, where=mn)
            assert gm.dtype == np.float32
            assert np.allclose(gm, wm, rtol=1e-5, atol=1e-6, equal_nan=True)
            _same(cp.max(cx, axis=axis, where=m, initial=-5.0).get(),
                  np.max(x, axis=axis, where=mn, initial=-5.0))
            _same(cp.min(cx, axis=axis, where=m, initial=5.0).get(),
                  np.min(x, axis=axis, where=mn, initial=5.0))
            _same(cp.any(cx > 1, axis=axis, where=m).get(), np.asarray(np.any(x > 1, axis=axis, where=mn)))
            _same(cp.all(cx > -3, axis=axis, where=m).get(), np.asarray(np.all(x > -3, axis=axis, where=mn)))
    p = (1 + 0.01 * rng.standard_normal((8, 100))).astype(np.float32)
    mp = rng.random((8, 100)) < 0.5
    assert np.allclose(cp.prod(cp.array(p), axis=1, where=mp).get(),
                       np.prod(p.astype(np.float64), axis=1, where=mp), rtol=1e-5)
    with pytest.raises(ValueError):
        cp.max(cx, where=m_row)                 # needs initial, as NumPy
    with pytest.raises(ValueError):
        cp.sum(cx, where=np.ones((2, 2), bool))
