"""Seeded random binary ufunc calls over mixed dtype pairs.

The reference's _binary_op (ndarray.py:960-1113) promotes with NumPy's
rules (_dtypes.py:139-146), wraps Python scalars and broadcasts before
launching an elementwise kernel.  Each case here draws an op, two operand
dtypes among the ten device dtypes (or a Python int / float / bool for one
side), broadcastable shapes and values with edge cases (zeros, signed zero,
inf, NaN, extreme integers, shift counts beyond the width), and compares
with NumPy, fused and op by op:

* NumPy's result dtype (int8 / uint8 results mapped to int16 / uint16 by
  the device dtype policy, as the reference's _dtypes.py:77-146 maps them)
  and shape;
* exact ops bit for bit (NaN == NaN): arithmetic, division and remainder
  (integer division by zero included), min / max and their NaN-ignoring
  forms, comparisons, logical and bitwise ops, shifts, copysign,
  nextafter, heaviside, ldexp, gcd / lcm, integer powers;
* power, float_power, arctan2, hypot, logaddexp, logaddexp2 within 2 ULP
  of NumPy or of the float64 evaluation rounded to the result dtype;
* where NumPy rejects the call (no loop for the dtypes, a Python int out of
  the array's range), the same exception class."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd._dtypes import resolve_dtype
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

DTYPES = [np.bool_, np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64,
          np.float16, np.float32, np.float64]
EXACT = ["add", "subtract", "multiply", "true_divide", "floor_divide", "remainder", "fmod",
         "maximum", "minimum", "fmax", "fmin", "equal", "not_equal", "less", "less_equal",
         "greater", "greater_equal", "logical_and", "logical_or", "logical_xor",
         "bitwise_and", "bitwise_or", "bitwise_xor", "left_shift", "right_shift",
         "copysign", "nextafter", "heaviside", "ldexp", "gcd", "lcm", "power"]
ROUNDED = ["power", "float_power", "arctan2", "hypot", "logaddexp", "logaddexp2"]
SHAPES = [((7, 33), (7, 33)), ((7, 33), (1, 33)), ((7, 1), (1, 33)), ((33,), (7, 33)),
          ((5, 1, 9), (4, 1)), ((1000,), (1000,)), ((64, 64), (64, 1))]


def _values(rng, shape, dtype, op, second):
    dt = np.dtype(dtype)
    if dt == np.bool_:
        return rng.random(shape) < 0.5
    if dt.kind in "iu":
        info = np.iinfo(dt)
        if op in ("left_shift", "right_shift") and second:
            lo = -2 if dt.kind == "i" else 0
            return rng.integers(lo, 8 * dt.itemsize + 3, shape).astype(dt)
        if op == "power" and second:
            return rng.integers(0, 6, shape).astype(dt)
        if op in ("power", "lcm", "gcd", "ldexp"):
            lo = -20 if dt.kind == "i" else 0
            return rng.integers(lo, 20, shape).astype(dt)
        r = rng.random()
        if r < 0.4:
            v = rng.integers(info.min, info.max, shape, dtype=dt, endpoint=True)
        else:
            v = rng.integers(max(info.min, -1000), 1000, shape).astype(dt)
        flat = v.reshape(-1)
        k = min(flat.size, 4)
        flat[rng.integers(0, flat.size, k)] = rng.choice(
            np.array([0, info.min, info.max, 1], dtype=dt), k)
        return v
    v = (rng.standard_normal(shape) * 100).astype(dt)
    if op in ("power", "float_power") and not second:
        v = np.abs(v) / 10 + np.array(0.5, dt)
    if op in ("power", "float_power") and second:
        v = (rng.standard_normal(shape) * 3).astype(dt)
    flat = v.reshape(-1)
    k = min(flat.size, 6)
    flat[rng.integers(0, flat.size, k)] = rng.choice(
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0], dtype=dt), k)
    return v


def _scalar(rng, op, second):
    r = rng.random()
    if op in ("left_shift", "right_shift") and second:
        return int(rng.integers(0, 12))
    if op in ("power", "float_power") and second:
        return int(rng.integers(0, 4)) if r < 0.5 else float(rng.integers(-2, 3)) + 0.5
    if r < 0.4:
        return int(rng.choice([0, 3, -7, 255, 300000, -2 ** 40]))
    if r < 0.8:
        return float(rng.choice([2.5, -0.0, 1e10, 0.1, -3.0]))
    return bool(rng.random() < 0.5)


def _case(seed):
    rng = np.random.default_rng(13000 + seed)
    op = (EXACT + ROUNDED)[int(rng.integers(len(EXACT) + len(ROUNDED)))]
    sa, sb = SHAPES[int(rng.integers(len(SHAPES)))]
    if rng.random() < 0.5:
        sa, sb = sb, sa
    operands = []
    for side, shape in ((0, sa), (1, sb)):
        if side == 1 and rng.random() < 0.2 or side == 0 and rng.random() < 0.1:
            operands.append(_scalar(rng, op, side == 1))
        else:
            dt = DTYPES[int(rng.integers(len(DTYPES)))]
            operands.append(_values(rng, shape, dt, op, side == 1))
    if not any(isinstance(o, np.ndarray) for o in operands):
        operands[0] = _values(rng, sa, np.float32, op, False)
    return op, operands


def _close(got, want, h_ops, op):
    if want.dtype.kind != "f" or op not in ROUNDED:
        gn, wn = np.isnan(got) if got.dtype.kind == "f" else 0, np.isnan(want) if want.dtype.kind == "f" else 0
        same = (np.ascontiguousarray(got).view(np.uint8).reshape(got.shape + (-1,))
                == np.ascontiguousarray(want).view(np.uint8).reshape(want.shape + (-1,))).all(-1)
        assert np.all(same | (gn & wn)), int(np.sum(~(same | (gn & wn))))
        return
    with np.errstate(all="ignore"):
        f64 = getattr(np, op)(*[o.astype(np.float64) if isinstance(o, np.ndarray) else o
                                for o in h_ops])
    cr = np.asarray(f64).astype(want.dtype)
    d = np.minimum(ref.ulp_distance(got, want), ref.ulp_distance(got, cr))
    assert int(np.max(d, initial=0)) <= 2, int(np.max(d))


@pytest.mark.parametrize("seed", range(300))
def test_random_binary(seed):
    op, h_ops = _case(seed)
    try:
        with np.errstate(all="ignore"):
            want = np.asarray(getattr(np, op)(*h_ops))
        want = want.astype(resolve_dtype(want.dtype), copy=False)   # int8 -> int16 policy
        err = None
    except (TypeError, OverflowError, ValueError) as e:
        err = e
    for fusion in (True, False):
        cp.set_config(fusion=fusion)
        d_ops = [cp.array(o) if isinstance(o, np.ndarray) else o for o in h_ops]
        if err is not None:
            base = next(c for c in (TypeError, OverflowError, ValueError) if isinstance(err, c))
            with pytest.raises(base):
                r = getattr(cp, op)(*d_ops)
                r.get()
            continue
        r = getattr(cp, op)(*d_ops)
        got = np.asarray(r.get() if isinstance(r, cp.ndarray) else r)
        assert got.dtype == want.dtype and got.shape == want.shape, (
            op, [getattr(o, "dtype", type(o)) for o in h_ops], got.dtype, want.dtype)
        _close(got, want, h_ops, op)
