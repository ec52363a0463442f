"""Failure paths of the device library, forced from the host.

Every case makes a call fail without a faulting or hung kernel: allocation,
runtime-compile and launch failures are injected by the library's test hook
(``mmp_debug_fail_next``), and a bounded cross-workgroup wait of a split
reduction is made to give up at once by having its readers expect a tag
that no writer produces (the kernel still finishes); a scan in that state
sums its tiles' predecessors itself and stays exact.  The reference
has no error channel below Python (its metalgpu calls return void,
_metal_backend.py:221-263); its Python-level errors (``ndarray.py:355-359``,
``_dtypes.py:133-134``) are covered by the host-logic tests.
"""
import gc

import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd._backend import HipBackend, HipError, HipWaitTimeoutError

pytestmark = pytest.mark.gpu


def _in_use():
    gc.collect()
    cp.synchronize()
    return HipBackend().memory_stats()[0]


@pytest.fixture
def be():
    b = HipBackend()
    yield b
    b.debug_fail_next(0, 0)  # disarm whatever a failed test left armed


def test_forced_reduction_wait_timeout_raises_on_synchronize(be):
    x_np = np.random.default_rng(40).standard_normal(1 << 22).astype(np.float32)
    x = cp.array(x_np)
    good = float(cp.sum(x).get())
    be.debug_fail_next(4, 1)
    s = cp.sum(x)
    with pytest.raises(HipWaitTimeoutError, match="reduction"):
        cp.synchronize()
    del s
    # the flags were cleared by the report; the next sum is right again
    assert be.wait_status() == 0
    assert float(cp.sum(x).get()) == good
    assert abs(good - float(np.sum(x_np, dtype=np.float64))) <= 1e-5 * abs(good) + 1e-3


def test_forced_reduction_wait_timeout_raises_on_get(be):
    x = cp.array(np.random.default_rng(41).standard_normal((4, 1 << 20)).astype(np.float32))
    be.debug_fail_next(4, 1)
    m = cp.max(x, axis=1)
    with pytest.raises(HipWaitTimeoutError):
        m.get()
    assert be.wait_status() == 0


@pytest.mark.parametrize("n", [1 << 22, 3 * 16384 + 4096])
def test_scan_without_predecessor_descriptors_sums_them_itself(be, n):
    """A scan whose tiles find no predecessor's descriptor (every reader
    expects a tag no writer produces) sums each missing predecessor's input
    itself: the result is exact and no wait is reported.  The fallback
    combines a predecessor's elements in the order that tile's own
    workgroup does, and a floating scan's prefixes have an association
    fixed by tile position, so float results are bit-identical to a run
    that found every descriptor."""
    g = np.random.default_rng(42)
    x_np = g.integers(-100, 100, n, dtype=np.int32)
    x = cp.array(x_np)
    be.debug_fail_next(4, 1)
    c = cp.cumsum(x)
    if n % 16384:  # the row tail's prefix comes from the last whole tile
        with pytest.raises(HipWaitTimeoutError, match="scan"):
            c.get()
    else:
        assert np.array_equal(c.get(), np.cumsum(x_np))
    assert be.wait_status() == 0
    assert np.array_equal(cp.cumsum(x).get(), np.cumsum(x_np))
    f_np = g.random(n, dtype=np.float32)
    f = cp.array(f_np)
    be.debug_fail_next(4, 1)
    cf = cp.cumsum(f)
    if n % 16384 == 0:
        ref = np.cumsum(f_np, dtype=np.float64)
        got = cf.get()
        assert np.all(np.abs(got - ref) <= 1e-5 * ref + 1e-6)
        assert np.array_equal(got, cp.cumsum(f).get())  # the same bits as a normal run
        assert be.wait_status() == 0
        d_np = g.random(n)                              # float64: 8192-element tiles
        d = cp.array(d_np)
        be.debug_fail_next(4, 1)
        got = cp.cumsum(d).get()
        want = np.cumsum(d_np)
        assert np.all(np.abs(got - want) <= 1e-12 * want)
        assert np.array_equal(got, cp.cumsum(d).get())
        h_np = (g.random(3 * 16384) + 0.5).astype(np.float32)
        h = cp.array(h_np)
        be.debug_fail_next(4, 1)
        got = cp.cumprod(h).get()
        want = np.cumprod(h_np.astype(np.float64))
        ok = (want > 1e-30) & (want < 1e30)          # float32 normal range
        assert np.all(np.abs(got[ok] - want[ok]) <= 1e-5 * want[ok])
        assert np.array_equal(got, cp.cumprod(h).get())
    else:
        with pytest.raises(HipWaitTimeoutError, match="scan"):
            cf.get()
    assert be.wait_status() == 0


def test_float_scan_walk_beyond_kept_windows_same_bits(be):
    """A floating scan tile keeps the last 512 predecessors it walked past
    for its tile-ordered fold.  With every descriptor withheld, the tiles
    of a 528-tile float32 row walk back to the row start, so the last ones
    walk past more than that and take the other branch: re-read the tiles
    after the inclusive prefix in order, summing each missing one itself.
    The bits must equal a normal run's (which walks a few windows)."""
    n = 528 * 16384
    g = np.random.default_rng(44)
    f_np = g.random(n, dtype=np.float32)
    f = cp.array(f_np)
    normal = cp.cumsum(f).get()
    be.debug_fail_next(4, 1)
    got = cp.cumsum(f).get()
    assert be.wait_status() == 0
    assert np.array_equal(got, normal)
    ref = np.cumsum(f_np, dtype=np.float64)
    assert np.all(np.abs(got - ref) <= 1e-5 * ref + 1e-6)


def test_injected_allocation_failure_leaks_nothing(be):
    a = cp.array(np.ones(1 << 20, np.float32))
    b = cp.array(np.full(1 << 20, 2.0, np.float32))
    (a + b).get()  # warm caches
    before = _in_use()
    be.debug_fail_next(1, 1)
    with pytest.raises(HipError, match="injected"):
        (a + b)._materialize_if_lazy()
    assert _in_use() == before
    assert np.array_equal((a + b).get(), np.full(1 << 20, 3.0, np.float32))


def test_injected_launch_failure_leaks_nothing(be):
    a = cp.array(np.arange(1 << 20, dtype=np.float32))
    (a * 2.0).get()
    before = _in_use()
    be.debug_fail_next(3, 1)
    with pytest.raises(HipError, match="injected"):
        (a * 2.0)._materialize_if_lazy()
    assert _in_use() == before
    assert np.array_equal((a * 2.0).get(), np.arange(1 << 20, dtype=np.float32) * 2)


def test_injected_compile_failure_is_not_cached(be):
    g = np.random.default_rng(43)
    a_np = g.uniform(0.5, 2.0, 4097).astype(np.float32)
    b_np = g.uniform(0.5, 2.0, 4097).astype(np.float32)
    a, b = cp.array(a_np), cp.array(b_np)
    a._ensure_gpu()
    b._ensure_gpu()
    before = _in_use()

    def expr():  # a structure no other test builds: compiled on first use
        return cp.hypot(cp.arctan(a), cp.cbrt(b) * 0.375) - cp.expm1(a) * 0.625

    be.debug_fail_next(2, 1)
    with pytest.raises(HipError, match="injected"):
        expr()._materialize_if_lazy()
    assert _in_use() == before
    with np.errstate(all="ignore"):
        want = (np.hypot(np.arctan(a_np), np.cbrt(b_np) * np.float32(0.375))
                - np.expm1(a_np) * np.float32(0.625))
    got = expr().get()
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_rawkernel_compile_error_carries_the_log(be):
    k = cp.RawKernel('extern "C" __global__ void bad(float* x) { x[0] = undefined_name; }', "bad")
    with pytest.raises(HipError, match="undefined_name"):
        k((64,), (cp.zeros(64, dtype=np.float32),))
