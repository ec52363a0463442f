"""The reference's Python-level kernel interface on the device:
``MetalBackend().execute_kernel(src, name, grid, buffers)`` with source from
``KernelCache().get_shader(category, dtype)``, then ``synchronize()``
(reference: _metal_backend.py:313-372, _kernel_cache.py:192-229, used as in
_fusion.py:457-460 and math_ops.py:155-157), and the fast_math switch
(_config.py:33-64, _kernels.py:26-27) against its stated bound."""
import numpy as np
import pytest

import macmetalpy as cp
from macmetalpy._kernel_cache import KernelCache
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu


class _Size:  # the reference's MetalSize shape: width / height / depth
    def __init__(self, w, h=1, d=1):
        self.width, self.height, self.depth = w, h, d


def _bits(a, b):
    assert a.dtype == b.dtype and a.shape == b.shape
    assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("n", [1000, 4096, 65537])
def test_execute_kernel_elementwise_like_reference(n):
    g = np.random.default_rng(n)
    a_np = g.standard_normal(n).astype(np.float32)
    b_np = g.standard_normal(n).astype(np.float32)
    backend = cp.MetalBackend()
    shader = KernelCache().get_shader("elementwise", np.float32)
    a, b = cp.array(a_np), cp.array(b_np)
    a._ensure_gpu()
    b._ensure_gpu()
    out = cp.zeros(n, dtype=np.float32)
    out._ensure_gpu()  # small creations start on the host (as the reference's)
    backend.execute_kernel(shader, "add_op", a.size, [a._buffer, b._buffer, out._buffer])
    backend.synchronize()
    _bits(out.get(), a_np + b_np)
    backend.execute_kernel(shader, b"sin_op", _Size(n), [a._buffer, out._buffer])
    backend.synchronize()
    _bits(out.get(), cp.sin(a).get())  # same device function as the cp op
    assert int(ref.ulp_distance(out.get(), np.sin(a_np)).max()) <= 2
    backend.execute_kernel(shader, "floor_divide_op", (n,), [a._buffer, b._buffer, out._buffer])
    backend.synchronize()
    _bits(out.get(), np.floor_divide(a_np, b_np))
    val = backend.array_to_buffer(np.array([2.5], np.float32))
    backend.execute_kernel(shader, "fill_scalar", n, [out._buffer, val])
    cp.synchronize()
    _bits(out.get(), np.full(n, 2.5, np.float32))


def test_execute_kernel_refuses_unbound_buffers():
    be = cp.MetalBackend()
    shader = KernelCache().get_shader("elementwise", np.float32)
    host = cp.zeros(16, dtype=np.float32)  # host-resident: no device buffer yet
    assert host._buffer is None
    with pytest.raises(ValueError, match="None"):
        be.execute_kernel(shader, "neg_op", 16, [host._buffer, host._buffer])


def test_execute_kernel_comparison_where_clip_int():
    g = np.random.default_rng(3)
    n = 3000
    x_np = g.integers(-50, 50, n).astype(np.int32)
    y_np = g.integers(-50, 50, n).astype(np.int32)
    be = cp.MetalBackend()
    kc = KernelCache()
    x, y = cp.array(x_np), cp.array(y_np)
    flags = be.create_buffer(n, np.int32)
    be.execute_kernel(kc.get_shader("comparison", np.int32), "lt_op", n, [x, y, flags])
    got = be.read_buffer(flags, 0, np.empty(n, np.int32))
    assert np.array_equal(got, (x_np < y_np).astype(np.int32))
    out = cp.empty(n, dtype=np.int32)
    be.execute_kernel(kc.get_shader("where", np.int32), "where_op", n, [flags, x, y, out])
    assert np.array_equal(out.get(), np.where(x_np < y_np, x_np, y_np))
    lo = cp.array(np.full(n, -10, np.int32))
    hi = cp.array(np.full(n, 10, np.int32))
    be.execute_kernel(kc.get_shader("clip", np.int32), "clip_op", n, [x, lo, hi, out])
    assert np.array_equal(out.get(), np.clip(x_np, -10, 10))
    be.execute_kernel(kc.get_shader("elementwise", np.int32), "mod_op", n, [x, y, out])
    with np.errstate(all="ignore"):
        assert np.array_equal(out.get(), np.mod(x_np, y_np))


# fast_math: the stated bound is the reference's unary-math tolerance
# (tests/conftest.py:83-86: rtol = atol = 1e-5) on the stated domains.
FAST_UNARY = [
    ("exp_op", np.exp, -80, 80), ("exp2_op", np.exp2, -100, 100), ("log_op", np.log, 1e-30, 1e30),
    ("log2_op", np.log2, 1e-30, 1e30), ("log10_op", np.log10, 1e-30, 1e30),
    ("sin_op", np.sin, -100, 100), ("cos_op", np.cos, -100, 100), ("tan_op", np.tan, -1.4, 1.4),
    ("sqrt_op", np.sqrt, 0, 1e30), ("reciprocal_op", np.reciprocal, 1e-30, 1e30),
    ("tanh_op", np.tanh, -10, 10), ("sinh_op", np.sinh, -10, 10), ("cosh_op", np.cosh, -10, 10),
]
FNS = {"exp_op": cp.exp, "exp2_op": cp.exp2, "log_op": cp.log, "log2_op": cp.log2,
       "log10_op": cp.log10, "sin_op": cp.sin, "cos_op": cp.cos, "tan_op": cp.tan,
       "sqrt_op": cp.sqrt, "reciprocal_op": cp.reciprocal, "tanh_op": cp.tanh,
       "sinh_op": cp.sinh, "cosh_op": cp.cosh}


def _fast_bound(got, want):
    return np.abs(got.astype(np.float64) - want) <= 1e-5 + 1e-5 * np.abs(want)


@pytest.mark.parametrize("op,fn64,lo,hi", FAST_UNARY)
def test_fast_math_within_reference_tolerance(op, fn64, lo, hi):
    g = np.random.default_rng(7)
    if lo > 0 and hi / lo > 1e6:  # log-uniform over wide positive ranges
        x = np.exp(g.uniform(np.log(lo), np.log(hi), 200000)).astype(np.float32)
    else:
        x = g.uniform(lo, hi, 200000).astype(np.float32)
    want = fn64(x.astype(np.float64))
    X = cp.array(x)
    exact = FNS[op](X).get()
    cp.set_config(fast_math=True)
    try:
        fast = FNS[op](X).get()
        shader = KernelCache().get_shader("elementwise", np.float32)
        out = cp.empty(x.size, dtype=np.float32)
        cp.MetalBackend().execute_kernel(shader, op, x.size, [X, out])
        via_cache = out.get()
    finally:
        cp.set_config(fast_math=False)
    ok = _fast_bound(fast, want)
    assert ok.all(), (op, x[~ok][:5], fast[~ok][:5], want[~ok][:5])
    _bits(via_cache, fast)
    # switching back gives the exact kernels again (cache keyed on the flag)
    _bits(FNS[op](X).get(), exact)


def test_fast_math_divide_power_and_fused_chain():
    g = np.random.default_rng(8)
    a = g.uniform(1e-3, 100, 100000).astype(np.float32)
    b = g.uniform(-4, 4, 100000).astype(np.float32)
    A, B = cp.array(a), cp.array(b)
    x = g.standard_normal((256, 8192)).astype(np.float32)
    r = g.uniform(0.5, 2.0, (1, 8192)).astype(np.float32)
    X, R = cp.array(x), cp.array(r)
    cp.set_config(fast_math=True)
    try:
        q = (A / B).get()
        p = (A ** B).get()
        z = cp.sum(cp.tanh(X * R + 1.0) * cp.exp(-cp.abs(X)) - cp.log1p(X * X), axis=1).get()
    finally:
        cp.set_config(fast_math=False)
    assert _fast_bound(q, a.astype(np.float64) / b).all()
    assert _fast_bound(p, np.power(a.astype(np.float64), b.astype(np.float64))).all()
    x64, r64 = x.astype(np.float64), r.astype(np.float64)
    terms = np.tanh(x64 * r64 + 1.0) * np.exp(-np.abs(x64)) - np.log1p(x64 * x64)
    scale = np.abs(terms).sum(axis=1)
    assert np.all(np.abs(z - terms.sum(axis=1)) <= 1e-5 * scale)
