"""Seeded random ufunc calls with out= / where= / dtype= / casting=.

NumPy ufuncs take ``out``, ``where``, ``dtype`` and ``casting``; the
reference forwards NumPy ufunc calls on its arrays (ndarray.py:2681-2720).
Each case draws a unary or binary ufunc, operand dtypes, an ``out`` array
(same or another dtype), a ``where`` mask (with or without ``out``), a
``dtype`` and a ``casting`` rule, and calls it both as ``cp.<ufunc>(...)``
and as ``np.<ufunc>(...)`` on device arrays (the ufunc protocol).  The
result must match NumPy's: values bit for bit (outside ``where`` with no
``out`` NumPy leaves them undefined, so only the selected ones count; the
float transcendentals within 2 ULP), ``out`` written in place, and the
same exception class where NumPy rejects the call (a casting violation)."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

BINARY = ["add", "subtract", "multiply", "maximum", "minimum", "true_divide", "floor_divide",
          "arctan2", "hypot"]
UNARY = ["negative", "absolute", "square", "sqrt", "sin", "exp", "floor", "sign"]
ROUNDED = {"arctan2", "hypot", "sin", "exp"}
DTYPES = [np.float32, np.float64, np.int32, np.int16, np.float16]


def _values(rng, shape, dt):
    if np.dtype(dt).kind == "f":
        return (rng.standard_normal(shape) * 3).astype(dt)
    v = rng.integers(-50, 50, shape).astype(dt)
    v[v == 0] = 1
    return v


def _case(seed):
    rng = np.random.default_rng(35000 + seed)
    binary = rng.random() < 0.6
    name = (BINARY if binary else UNARY)[int(rng.integers(len(BINARY if binary else UNARY)))]
    shape = [(7, 33), (64,), (5, 1, 9)][int(rng.integers(3))]
    ins = [_values(rng, shape, DTYPES[int(rng.integers(len(DTYPES)))])
           for _ in range(2 if binary else 1)]
    if binary and rng.random() < 0.3:
        ins[1] = ins[1][..., :1]                          # broadcast along the last axis
    kw = {}
    with np.errstate(all="ignore"):
        base = getattr(np, name)(*ins)
    r = rng.random()
    if r < 0.35:
        kw["out"] = DTYPES[int(rng.integers(len(DTYPES)))]
    if rng.random() < 0.4:
        kw["where"] = rng.random(base.shape[-1:] if rng.random() < 0.5 else base.shape) < 0.5
    if rng.random() < 0.25:
        kw["dtype"] = [np.float64, np.float32][int(rng.integers(2))]
    if rng.random() < 0.15:
        kw["casting"] = "unsafe"
    return name, ins, kw, base.shape, rng


def _np_call(name, ins, kw, out_init):
    kw = dict(kw)
    if "out" in kw:
        kw["out"] = out_init.copy()
    with np.errstate(all="ignore"):
        r = getattr(np, name)(*ins, **kw)
    return r


def _compare(got, want, name, mask):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape and got.dtype == want.dtype, (name, got.dtype, want.dtype)
    if mask is not None:
        m = np.broadcast_to(mask, want.shape)
        got, want = got[m], want[m]
    if name in ROUNDED and want.dtype.kind == "f":
        assert int(np.max(ref.ulp_distance(got, want), initial=0)) <= 2, name
    else:
        assert np.array_equal(got, want, equal_nan=True), name


@pytest.mark.parametrize("seed", range(120))
@pytest.mark.parametrize("form", ["function", "protocol"])
def test_random_ufunc_kwargs(seed, form):
    name, ins, kw, shape, rng = _case(seed)
    out_init = None
    if "out" in kw:
        out_init = _values(rng, shape, kw["out"])
    try:
        want = _np_call(name, ins, kw, out_init)
        err = None
    except (TypeError, ValueError) as e:
        err = e
    dkw = dict(kw)
    if "out" in dkw:
        dkw["out"] = cp.array(out_init)
    if "where" in dkw:
        dkw["where"] = cp.array(kw["where"])
    d_ins = [cp.array(x) for x in ins]
    mod = cp if form == "function" else np
    if err is not None:
        with pytest.raises(TypeError if isinstance(err, TypeError) else ValueError):
            r = getattr(mod, name)(*d_ins, **dkw)
            r.get()
        return
    r = getattr(mod, name)(*d_ins, **dkw)
    if "out" in kw:
        assert r is dkw["out"]                     # written in place and returned
    mask = kw["where"] if ("where" in kw and "out" not in kw) else None
    _compare(r.get(), want, name, mask)
