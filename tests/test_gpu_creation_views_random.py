"""Seeded random creation calls and view chains against NumPy.

* Creation (reference creation.py:36-114 and the NumPy names it forwards):
  arange with integer and float steps (NumPy's length rule and
  start + i * step values), linspace / logspace / geomspace with and
  without the endpoint, full / zeros / ones / eye / identity / tri /
  *_like with explicit dtypes.  Values bit for bit, except the
  transcendental spacings (logspace, geomspace) within 2 ULP.
* View chains (reference ndarray reshape / transpose / slicing,
  ndarray.py:245-618): random sequences of reshape (with -1),
  transpose / swapaxes / moveaxis, expand_dims / squeeze, basic slices
  (negative steps too), broadcast_to, ravel and .T, applied to a device
  array and to its NumPy copy; the result (read through get()) and an
  elementwise op on the view must match bit for bit."""
import numpy as np
import pytest

import macmetalpy_amd as cp
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu

DTYPES = [np.float32, np.float64, np.int32, np.int64, np.int16, np.uint16, np.float16]


def _both(f):
    """f(np) against f(cp): equal results, or the same exception class."""
    try:
        want = np.asarray(f(np))
    except (OverflowError, ValueError, TypeError) as e:
        base = next(c for c in (OverflowError, ValueError, TypeError) if isinstance(e, c))
        with pytest.raises(base):
            f(cp).get()
        return
    _same(f(cp).get(), want)


def _same(got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape and got.dtype == want.dtype, (got.shape, want.shape,
                                                                 got.dtype, want.dtype)
    assert np.array_equal(got, want, equal_nan=want.dtype.kind == "f")


@pytest.mark.parametrize("seed", range(80))
def test_random_creation(seed):
    rng = np.random.default_rng(31000 + seed)
    k = int(rng.integers(8))
    dt = DTYPES[int(rng.integers(len(DTYPES)))]
    if k == 0:                                   # integer arange
        a, b = sorted(int(v) for v in rng.integers(-500, 500, 2))
        step = int(rng.choice([1, 2, 3, 7, -1, -3]))
        if step < 0:
            a, b = b, a
        args = (a, b, step)
        _both(lambda m: m.arange(*args))
        _both(lambda m: m.arange(*args, dtype=dt))
    elif k == 1:                                 # float arange
        a = float(np.round(rng.uniform(-10, 10), 3))
        step = float(rng.choice([0.1, 0.25, 0.3, -0.7, 1.5]))
        b = a + step * float(rng.integers(1, 200)) + float(rng.uniform(-0.5, 0.5)) * step
        _same(cp.arange(a, b, step).get(), np.arange(a, b, step))
        if dt in (np.float32, np.float64):
            _same(cp.arange(a, b, step, dtype=dt).get(), np.arange(a, b, step, dtype=dt))
    elif k == 2:                                 # linspace
        a, b = (float(np.round(v, 3)) for v in rng.uniform(-100, 100, 2))
        n = int(rng.choice([0, 1, 2, 5, 50, 1001]))
        ep = bool(rng.random() < 0.7)
        _same(cp.linspace(a, b, n, endpoint=ep).get(), np.linspace(a, b, n, endpoint=ep))
        if dt in (np.float32, np.float64):
            _same(cp.linspace(a, b, n, endpoint=ep, dtype=dt).get(),
                  np.linspace(a, b, n, endpoint=ep, dtype=dt))
    elif k == 3:                                 # logspace / geomspace
        n = int(rng.choice([1, 2, 7, 100]))
        ep = bool(rng.random() < 0.7)
        a, b = (float(np.round(v, 2)) for v in rng.uniform(-3, 3, 2))
        for got, want in ((cp.logspace(a, b, n, endpoint=ep).get(), np.logspace(a, b, n, endpoint=ep)),
                          (cp.geomspace(10 ** a, 10 ** b, n, endpoint=ep).get(),
                           np.geomspace(10 ** a, 10 ** b, n, endpoint=ep))):
            assert got.shape == want.shape and got.dtype == want.dtype
            assert int(np.max(ref.ulp_distance(got, want), initial=0)) <= 2
    elif k == 4:                                 # full / zeros / ones
        shape = tuple(int(v) for v in rng.integers(0, 9, int(rng.integers(0, 4))))
        fill = {np.float32: 2.5, np.float64: -1e300, np.float16: 65504.0}.get(dt, 7)
        _same(cp.full(shape, fill, dtype=dt).get(), np.full(shape, fill, dtype=dt))
        _same(cp.zeros(shape, dtype=dt).get(), np.zeros(shape, dtype=dt))
        _same(cp.ones(shape, dtype=dt).get(), np.ones(shape, dtype=dt))
    elif k == 5:                                 # eye / identity / tri
        n, m = (int(v) for v in rng.integers(1, 40, 2))
        kk = int(rng.integers(-5, 6))
        _same(cp.eye(n, m, k=kk, dtype=dt).get(), np.eye(n, m, k=kk, dtype=dt))
        _same(cp.identity(n, dtype=dt).get(), np.identity(n, dtype=dt))
        _same(cp.tri(n, m, k=kk, dtype=dt).get(), np.tri(n, m, k=kk, dtype=dt))
    elif k == 6:                                 # *_like
        x = (rng.standard_normal((int(rng.integers(1, 9)), 5)) * 10).astype(dt)
        d = cp.array(x)
        _same(cp.zeros_like(d).get(), np.zeros_like(x))
        _same(cp.ones_like(d).get(), np.ones_like(x))
        _same(cp.full_like(d, 3).get(), np.full_like(x, 3))
    else:                                        # array / asarray from nested lists and scalars
        lst = rng.integers(-100, 100, (3, 4)).tolist()
        _same(cp.array(lst).get(), np.array(lst))
        _both(lambda m: m.asarray(lst, dtype=dt))
        _same(cp.array(2.5).get(), np.array(2.5))


def _chain(rng, shape):
    """A random list of view steps valid for an array of ``shape``."""
    steps = []
    cur = tuple(shape)
    for _ in range(int(rng.integers(1, 6))):
        k = int(rng.integers(8))
        nd = len(cur)
        if k == 0 and nd:                        # reshape (keeps the size), one -1
            n = int(np.prod(cur))
            divs = [d for d in range(1, n + 1) if n % d == 0] if 0 < n <= 100000 else [n]
            d = int(rng.choice(divs))
            new = (d, -1) if rng.random() < 0.5 else (-1, d)
            steps.append(("reshape", new))
            cur = (d, n // d) if new[0] == d else (n // d, d)
        elif k == 1 and nd > 1:
            p = tuple(int(i) for i in rng.permutation(nd))
            steps.append(("transpose", p))
            cur = tuple(cur[i] for i in p)
        elif k == 2 and nd > 1:
            a, b = (int(v) for v in rng.choice(nd, 2, replace=False))
            steps.append(("swapaxes", a, b))
            cur = list(cur); cur[a], cur[b] = cur[b], cur[a]; cur = tuple(cur)
        elif k == 3 and nd:
            a, b = int(rng.integers(nd)), int(rng.integers(nd))
            steps.append(("moveaxis", a, b))
            c = list(cur); v = c.pop(a); c.insert(b, v); cur = tuple(c)
        elif k == 4:
            a = int(rng.integers(nd + 1))
            steps.append(("expand_dims", a))
            c = list(cur); c.insert(a, 1); cur = tuple(c)
        elif k == 5 and 1 in cur:
            steps.append(("squeeze",))
            cur = tuple(v for v in cur if v != 1)
        elif k == 6 and nd:
            ax = int(rng.integers(nd))
            step = int(rng.choice([2, -1, -2, 3]))
            lo = int(rng.integers(0, max(1, cur[ax])))
            steps.append(("slice", ax, lo, step))
            idx = [slice(None)] * nd
            idx[ax] = slice(lo, None, step)
            cur = np.empty(cur)[tuple(idx)].shape
        elif k == 7 and nd and 1 in cur:
            tgt = tuple(3 if v == 1 else v for v in cur)
            steps.append(("broadcast_to", tgt))
            cur = tgt
    return steps


def _apply(m, x, steps):
    for s in steps:
        if s[0] == "reshape":
            x = x.reshape(s[1])
        elif s[0] == "transpose":
            x = x.transpose(s[1])
        elif s[0] == "swapaxes":
            x = m.swapaxes(x, s[1], s[2])
        elif s[0] == "moveaxis":
            x = m.moveaxis(x, s[1], s[2])
        elif s[0] == "expand_dims":
            x = m.expand_dims(x, s[1])
        elif s[0] == "squeeze":
            x = m.squeeze(x)
        elif s[0] == "slice":
            idx = [slice(None)] * x.ndim
            idx[s[1]] = slice(s[2], None, s[3])
            x = x[tuple(idx)]
        else:
            x = m.broadcast_to(x, s[1])
    return x


@pytest.mark.parametrize("seed", range(100))
def test_random_view_chain(seed):
    rng = np.random.default_rng(33000 + seed)
    shape = tuple(int(rng.choice([1, 2, 3, 4, 6, 12])) for _ in range(int(rng.integers(1, 5))))
    dt = DTYPES[int(rng.integers(len(DTYPES)))]
    x = (rng.standard_normal(shape) * 50).astype(dt)
    steps = _chain(rng, shape)
    want = _apply(np, x, steps)
    got = _apply(cp, cp.array(x), steps)
    _same(got.get(), want)
    _same(got.ravel().get(), want.ravel())
    _same(got.T.get(), want.T)
    _same((got * 2).get(), want * np.array(2, dt))
