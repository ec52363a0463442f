"""Seeded random checks of the ndarray object against NumPy's.

The reference's ndarray (ndarray.py:245-618, 2501-2912) mirrors NumPy's
attributes, conversions and methods.  Each case draws a dtype, a shape and
a view (contiguous, stepped, transposed, a row, 0-d) and compares:
shape / ndim / size / itemsize / nbytes / strides, tolist(), item(),
iteration and len(), bool / int / float / index conversions (and NumPy's
exception class where they are refused), copy() independence, fill(),
astype(copy=False), view(dtype) bit reinterpretation, flatten(), and the
method forms of sum / argmax / cumsum / sort / clip / round / any / all /
nonzero / diagonal / trace / repeat / take / tobytes."""
import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu

DTYPES = [np.float32, np.float64, np.int32, np.int64, np.int16, np.uint16, np.float16, np.bool_]


def _data(rng, shape, dt):
    if dt == np.bool_:
        return rng.random(shape) < 0.5
    return (rng.standard_normal(shape) * 20).astype(dt)


def _case(seed):
    rng = np.random.default_rng(37000 + seed)
    dt = DTYPES[int(rng.integers(len(DTYPES)))]
    k = int(rng.integers(6))
    if k == 5:
        base = _data(rng, (), dt)
        return rng, dt, base, ()
    shape = [(7, 5), (4, 6, 3), (16,), (1, 1), (9, 8)][int(rng.integers(5))]
    base = _data(rng, shape, dt)
    view = [(), (slice(None, None, 2),), "T", (0,), (slice(None, None, -1),)][k]
    return rng, dt, base, view


def _view(x, view):
    if view == "T":
        return x.T
    return x[view] if view != () else x


def _raises_same(f_np, f_cp):
    try:
        want = f_np()
    except (TypeError, ValueError, IndexError) as e:
        cls = next(c for c in (TypeError, ValueError, IndexError) if isinstance(e, c))
        with pytest.raises(cls):
            f_cp()
        return None, None
    return want, f_cp()


@pytest.mark.parametrize("seed", range(120))
def test_random_ndarray_object(seed):
    rng, dt, base, view = _case(seed)
    h = _view(base, view)
    d = _view(cp.array(base), view)
    # attributes
    assert d.shape == h.shape and d.ndim == h.ndim and d.size == h.size
    assert d.dtype == h.dtype and d.itemsize == h.itemsize and d.nbytes == h.nbytes
    assert d.strides == h.strides, (d.strides, h.strides)
    # element access and conversions
    assert d.tolist() == h.tolist()
    if h.size:
        i = int(rng.integers(h.size))
        assert d.item(i) == h.item(i) and type(d.item(i)) is type(h.item(i))
    for conv in (bool, int, float):
        w, g = _raises_same(lambda c=conv: c(h), lambda c=conv: c(d))
        assert w == g
    w, g = _raises_same(lambda: len(h), lambda: len(d))
    assert w == g
    if h.ndim:
        rows = [r.get() if isinstance(r, cp.ndarray) else r for r in d]
        assert len(rows) == len(h)
        for r, hr in zip(rows, h):
            assert np.array_equal(np.asarray(r), hr)
    # copies, fill, astype, view
    c = d.copy()
    c.fill(1)
    assert np.array_equal(d.get(), h)                       # the copy is independent
    assert np.array_equal(c.get(), np.ones_like(h))
    assert d.astype(dt, copy=False).dtype == h.dtype
    if h.ndim and h.flags.c_contiguous and dt in (np.float32, np.int32):
        other = np.int32 if dt == np.float32 else np.float32
        assert np.array_equal(d.view(other).get().view(np.uint32), h.view(other).view(np.uint32))
    assert np.array_equal(d.flatten().get(), h.flatten())
    assert d.tobytes() == h.tobytes()


@pytest.mark.parametrize("seed", range(80))
def test_random_ndarray_methods(seed):
    rng, dt, base, view = _case(seed)
    h = _view(base, view)
    d = _view(cp.array(base), view)
    if h.ndim == 0:
        return
    checks = [
        (lambda x: x.sum(axis=-1), "sum"), (lambda x: x.argmax(axis=0), "argmax"),
        (lambda x: x.cumsum(axis=0), "cumsum"), (lambda x: x.any(axis=-1), "any"),
        (lambda x: x.all(), "all"), (lambda x: x.repeat(2, axis=0), "repeat"),
        (lambda x: x.take([0, -1], axis=0), "take"), (lambda x: x.nonzero(), "nonzero"),
    ]
    if dt != np.bool_:
        checks += [(lambda x: x.clip(-5, 5), "clip"), (lambda x: np.sort(x, axis=-1), "sort")]
    if dt in (np.float32, np.float64, np.float16):
        checks += [(lambda x: x.round(1), "round")]
    if h.ndim == 2:
        checks += [(lambda x: x.diagonal(), "diagonal"), (lambda x: x.trace(), "trace")]
    for f, name in checks:
        with np.errstate(all="ignore"):
            want = f(h)
        got = f(d)
        if isinstance(want, tuple):
            assert len(got) == len(want)
            for g, w in zip(got, want):
                assert np.array_equal(g.get() if hasattr(g, "get") else g, w), name
            continue
        got = got.get() if isinstance(got, cp.ndarray) else np.asarray(got)
        want = np.asarray(want)
        assert got.shape == want.shape and got.dtype == want.dtype, (name, got.dtype, want.dtype)
        if name == "sum" and want.dtype.kind == "f":
            tol = np.finfo(want.dtype).eps * np.sum(np.abs(h.astype(np.float64)), axis=-1) * 2
            assert np.all(np.abs(got.astype(np.float64) - want) <= tol + np.finfo(want.dtype).tiny), name
        elif name in ("cumsum", "trace") and want.dtype.kind == "f":
            # NumPy accumulates in the dtype, the device in float64
            np.testing.assert_allclose(got, want, rtol=1e-2 if dt == np.float16 else 1e-5,
                                       atol=1e-2 if dt == np.float16 else 1e-4)
        else:
            assert np.array_equal(got, want, equal_nan=want.dtype.kind == "f"), name
