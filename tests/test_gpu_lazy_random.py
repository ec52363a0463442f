"""Seeded random programs mixing lazy expressions with in-place writes.

The reference defers elementwise results as lazy DAG nodes and
materialises them on demand (_fusion.py:416-486, ndarray.py:478-481), and
must keep NumPy's eager semantics while doing so: a pending expression
sees its inputs as they were when it was built, even if they are written
later; in-place ops and slice assignments are visible through every view
of the written array.  Each case here runs a random program -- new lazy
results of unary / binary ops on arrays and basic-slice views (including
overlapping ones such as x[1:] and x[:-1]), in-place ops, slice
assignments, reductions and reads in random order -- on the device and,
eagerly, with NumPy, then compares every array.  Operations NumPy rejects
(an in-place result that does not broadcast to its target, a same_kind
cast violation) must raise the same exception class and leave the arrays
unchanged."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu

UNARY = [lambda m, x: m.sin(x), lambda m, x: -x, lambda m, x: m.abs(x) * 0.5,
         lambda m, x: m.tanh(x), lambda m, x: x * x]
BINARY = [lambda a, b: a + b, lambda a, b: a - b, lambda a, b: a * b,
          lambda a, b: a * 0.5 + b]
INPLACE = ["+=", "-=", "*="]


def _views(rng, shape):
    """A random basic-slice view spec for a 2-D array of ``shape``."""
    R, C = shape
    k = int(rng.integers(7))
    if k == 0:
        return (slice(None), slice(None))
    if k == 1:
        return (slice(1, None), slice(None))          # overlaps (:-1)
    if k == 2:
        return (slice(None, -1), slice(None))
    if k == 3:
        return (slice(None), slice(None, None, 2))
    if k == 4:
        return (slice(None, None, -1), slice(None))
    if k == 5:
        return (int(rng.integers(R)), slice(None))     # a row
    return (slice(None), slice(1, None))


def _run(seed):
    rng = np.random.default_rng(23000 + seed)
    R, C = [(6, 9), (17, 33), (64, 100), (3, 4)][seed % 4]
    dt = np.float32 if seed % 3 else np.float64
    h, d = [], []                                      # NumPy mirrors, device arrays
    for _ in range(3):
        x = rng.standard_normal((R, C)).astype(dt)
        h.append(x.copy())
        d.append(cp.array(x))
    for step in range(14):
        r = rng.random()
        i = int(rng.integers(len(h)))
        j = int(rng.integers(len(h)))
        vi, vj = _views(rng, (R, C)), _views(rng, (R, C))
        if r < 0.3:                                    # a new lazy result
            if rng.random() < 0.4:
                f = UNARY[int(rng.integers(len(UNARY)))]
                hv, dv = f(np, h[i][vi]), f(cp, d[i][vi])
            else:
                f = BINARY[int(rng.integers(len(BINARY)))]
                a_h, b_h = h[i][vi], h[j][vj]
                try:
                    np.broadcast_shapes(a_h.shape, b_h.shape)
                except ValueError:
                    continue
                hv, dv = f(a_h, b_h), f(d[i][vi], d[j][vj])
            if hv.shape != (R, C) or hv.dtype != dt:
                # a result of another shape is checked now rather than kept
                _close(dv.get(), hv, dt)
                continue
            h.append(hv)
            d.append(dv)
        elif r < 0.6:                                  # in-place op through a view
            op = INPLACE[int(rng.integers(len(INPLACE)))]
            tgt_h, src_h = h[i][vi], h[j][vj]
            tgt_d, src_d = d[i][vi], d[j][vj]
            if rng.random() < 0.3:
                src_h = src_d = float(np.round(rng.uniform(-2, 2), 2))
            try:
                ok = True
                exec(f"tgt_h {op} src_h")
            except ValueError:
                ok = False
            if ok:
                exec(f"tgt_d {op} src_d")
            else:
                before = [x.get() for x in d]
                with pytest.raises(ValueError):
                    exec(f"tgt_d {op} src_d")
                for b, x in zip(before, d):
                    np.testing.assert_array_equal(x.get(), b)
        elif r < 0.75:                                 # slice assignment
            src_h = h[j][vj]
            try:
                h_copy = h[i].copy()
                h_copy[vi] = src_h
                ok = True
            except ValueError:
                ok = False
            if ok:
                h[i][vi] = src_h
                d[i][vi] = d[j][vj]
        elif r < 0.9:                                  # a read now
            _close(d[i].get(), h[i], dt)
        else:                                          # a reduction now
            got = cp.sum(d[i][vi], axis=-1).get()
            want = np.sum(h[i][vi].astype(np.float64), axis=-1)
            np.testing.assert_allclose(got, want.astype(dt), rtol=2e-6 if dt == np.float32 else 1e-12,
                                       atol=1e-5)
    for x_d, x_h in zip(d, h):
        _close(x_d.get(), x_h, dt)


def _close(got, want, dt):
    """Exact ops give NumPy's bits; transcendentals may differ by 2 ULP
    from NumPy's, and the difference propagates through later steps."""
    assert got.shape == want.shape and got.dtype == want.dtype
    tol = 1e-12 if dt == np.float64 else 2e-5
    np.testing.assert_allclose(got, want, rtol=tol, atol=tol)


@pytest.mark.parametrize("seed", range(64))
def test_random_lazy_program(seed):
    _run(seed)


def test_inplace_result_must_broadcast_to_target():
    a = cp.zeros((1, 5), dtype=np.float32)
    with pytest.raises(ValueError):
        a += cp.ones((3, 5), dtype=np.float32)
    np.testing.assert_array_equal(a.get(), np.zeros((1, 5), np.float32))
    b = cp.zeros((4, 5), dtype=np.float32)
    b[1:] += b[:-1] + 1                                 # overlapping views
    want = np.zeros((4, 5), np.float32)
    want[1:] += want[:-1] + 1
    np.testing.assert_array_equal(b.get(), want)
