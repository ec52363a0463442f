"""Array calls from several host threads at once.

ctypes releases the GIL around every call into libmmp_hip.so, so calls
from several Python threads reach the library concurrently.  The
reductions and scans share per-process scratch slots that grow (free and
replace their block) when a larger call arrives, and tag their tile flags
with a call generation; the library serialises the slot lookup, the tag
and the launches of each call, and every call enqueues on the one library
stream.  Each thread here runs its own seeded sequence of sums, argmaxes,
cumsums, fused expressions and products over sizes that force the slots
to grow in the middle of other threads' calls; every result must equal
NumPy's (integers bit for bit, floats within the summation bound)."""
import threading

import numpy as np
import pytest

import macmetalpy_amd as cp

pytestmark = pytest.mark.gpu

SIZES = [1000, 65537, 1 << 20, 3 << 20, 9 << 20, 24 << 20]


def _worker(tid, errors):
    rng = np.random.default_rng(41000 + tid)
    try:
        for step in range(14):
            n = int(SIZES[(step + tid) % len(SIZES)])
            k = int(rng.integers(5))
            if k == 0:
                h = rng.integers(-1000, 1000, n).astype(np.int32)
                got = int(cp.array(h).sum())
                assert got == int(h.sum(dtype=np.int64)), (tid, step, "sum")
            elif k == 1:
                h = rng.standard_normal(n).astype(np.float32)
                got = float(cp.array(h).sum())
                bound = np.finfo(np.float32).eps * float(np.abs(h).sum()) * 2 + 1e-6
                assert abs(got - float(h.astype(np.float64).sum())) <= bound, (tid, step, "fsum")
            elif k == 2:
                rows = 8
                h = rng.integers(-10 ** 6, 10 ** 6, (rows, n // rows)).astype(np.int64)
                got = cp.argmax(cp.array(h), axis=1).get()
                assert np.array_equal(got, np.argmax(h, axis=1)), (tid, step, "argmax")
            elif k == 3:
                h = rng.integers(-100, 100, n).astype(np.int32)
                got = cp.cumsum(cp.array(h)).get()
                assert np.array_equal(got, np.cumsum(h)), (tid, step, "cumsum")
            else:
                a = rng.standard_normal(n).astype(np.float32)
                b = rng.standard_normal(n).astype(np.float32)
                da, db = cp.array(a), cp.array(b)
                got = (da * db + da).get()
                assert np.array_equal(got, a * b + a), (tid, step, "fused")
                m = 96
                x = rng.standard_normal((m, m)).astype(np.float32)
                y = rng.standard_normal((m, m)).astype(np.float32)
                gm = cp.matmul(cp.array(x), cp.array(y)).get()
                np.testing.assert_allclose(gm, x.astype(np.float64) @ y, rtol=1e-4, atol=1e-3)
    except BaseException as e:                     # reported by the main thread
        errors.append((tid, repr(e)))


def test_threads_share_the_library():
    errors = []
    threads = [threading.Thread(target=_worker, args=(t, errors)) for t in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=110)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors
    cp.synchronize()
