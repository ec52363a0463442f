"""Seeded random unary ufunc calls over the ten device dtypes.

The reference's _unary_op (ndarray.py:1161-1243) and its math_ops /
ufunc_ops front-ends (math_ops.py:15-67, 368-508; ufunc_ops.py:38-152)
follow NumPy's result dtypes.  Each case here draws a unary ufunc, a dtype,
a shape and view (contiguous, stepped, transposed) and values with the edge
cases of the dtype (zeros, signed zero, inf, NaN, the extreme integers),
and compares with NumPy, fused and op by op:

* NumPy's result dtype (int8 / uint8 results mapped to int16 / uint16 by
  the device dtype policy, as the reference's _dtypes.py:77-146 maps them)
  and shape;
* exact ops bit for bit (NaN == NaN): sign, rounding, abs, negation,
  square, reciprocal, sqrt, degree conversions, logical / bitwise not,
  classification (isnan ...), signbit, spacing, bitwise_count;
* the other float ops within 2 ULP of NumPy or of the float64 evaluation
  rounded to the result dtype (NumPy's own float16 / float32 results are not
  always correctly rounded);
* where NumPy rejects the dtype (negative of bool, invert of a float ...),
  the same exception class."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd._dtypes import resolve_dtype
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

DTYPES = [np.bool_, np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64,
          np.float16, np.float32, np.float64]
EXACT = ["negative", "positive", "absolute", "fabs", "sign", "square", "reciprocal", "sqrt",
         "floor", "ceil", "rint", "trunc", "logical_not", "invert", "isnan", "isinf",
         "isfinite", "signbit", "spacing", "bitwise_count", "degrees", "radians"]
ROUNDED = ["cbrt", "exp", "exp2", "expm1", "log", "log2", "log10", "log1p", "sin", "cos",
           "tan", "arcsin", "arccos", "arctan", "sinh", "cosh", "tanh", "arcsinh", "arccosh",
           "arctanh"]
# input ranges of the float draws per op (outside them the ops give only NaN,
# inf or zero); special values are added to every draw
DOMAIN = {"arcsin": (-1, 1), "arccos": (-1, 1), "arctanh": (-1, 1), "arccosh": (1, 100),
          "log": (0, 1e4), "log2": (0, 1e4), "log10": (0, 1e4), "log1p": (-1, 1e4),
          "sqrt": (0, 1e4), "exp": (-80, 80), "exp2": (-120, 120), "expm1": (-80, 80),
          "sinh": (-80, 80), "cosh": (-80, 80), "tan": (-1.5, 1.5), "sin": (-100, 100),
          "cos": (-100, 100)}
SHAPES = [(1000,), (7, 129), (3, 5, 17), (1,), (64, 64)]


def _values(rng, shape, dtype, op):
    dt = np.dtype(dtype)
    if dt == np.bool_:
        return rng.random(shape) < 0.5
    if dt.kind in "iu":
        info = np.iinfo(dt)
        if op == "reciprocal":                 # NumPy's integer reciprocal divides 1 by x
            return rng.integers(max(info.min, -3), 4, shape).astype(dt)
        v = rng.integers(info.min, info.max, shape, dtype=dt, endpoint=True)
        flat = v.reshape(-1)
        k = min(flat.size, 4)
        flat[rng.integers(0, flat.size, k)] = rng.choice(np.array([0, info.min, info.max, 1], dt), k)
        return v
    lo, hi = DOMAIN.get(op, (-100, 100))
    if dt == np.float16:
        hi = min(hi, 11 if op in ("exp", "sinh", "cosh", "expm1") else hi)
        lo = max(lo, -11 if op in ("exp", "sinh", "cosh", "expm1") else lo)
    v = rng.uniform(lo, hi, shape).astype(dt)
    flat = v.reshape(-1)
    k = min(flat.size, 6)
    flat[rng.integers(0, flat.size, k)] = rng.choice(
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0], dt), k)
    return v


def _case(seed):
    rng = np.random.default_rng(15000 + seed)
    op = (EXACT + ROUNDED)[int(rng.integers(len(EXACT) + len(ROUNDED)))]
    dt = DTYPES[int(rng.integers(len(DTYPES)))]
    shape = SHAPES[int(rng.integers(len(SHAPES)))]
    view = int(rng.integers(3))
    base = _values(rng, (2 * shape[0],) + shape[1:] if view == 1 else shape[::-1] if view == 2
                   else shape, dt, op)
    return op, base, view


def _view(x, view):
    if view == 1:
        return x[::2]
    if view == 2:
        return x.T
    return x


@pytest.mark.parametrize("seed", range(300))
def test_random_unary(seed):
    op, base, view = _case(seed)
    h = _view(base, view)
    try:
        with np.errstate(all="ignore"):
            want = np.asarray(getattr(np, op)(h))
        want = want.astype(resolve_dtype(want.dtype), copy=False)
        err = None
    except (TypeError, ValueError) as e:
        err = e
    for fusion in (True, False):
        cp.set_config(fusion=fusion)
        d = _view(cp.array(base), view)
        if err is not None:
            base_cls = TypeError if isinstance(err, TypeError) else ValueError
            with pytest.raises(base_cls):
                getattr(cp, op)(d).get()
            continue
        got = np.asarray(getattr(cp, op)(d).get())
        assert got.dtype == want.dtype and got.shape == want.shape, (op, h.dtype, got.dtype,
                                                                     want.dtype)
        if want.dtype.kind != "f" or op in EXACT:
            gn = np.isnan(got) if got.dtype.kind == "f" else False
            wn = np.isnan(want) if want.dtype.kind == "f" else False
            same = (np.ascontiguousarray(got).view(np.uint8).reshape(got.shape + (-1,))
                    == np.ascontiguousarray(want).view(np.uint8).reshape(want.shape + (-1,))).all(-1)
            bad = ~(same | (gn & wn))
            assert not np.any(bad), (op, h.dtype, h[bad][:4], got[bad][:4], want[bad][:4])
            continue
        with np.errstate(all="ignore"):
            cr = np.asarray(getattr(np, op)(h.astype(np.float64))).astype(want.dtype)
        dist = np.minimum(ref.ulp_distance(got, want), ref.ulp_distance(got, cr))
        assert int(np.max(dist, initial=0)) <= 2, (op, h.dtype, int(np.max(dist)))
