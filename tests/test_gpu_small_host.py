"""Small host-resident operands through the native gate, on the device.

Arrays made from NumPy data start host-resident (reference ndarray.py:
284-331).  The reference's C gate answers small ones on the CPU
(_accelerator.c:549-712 fast_binary / fast_unary, :798-858 fast_reduce);
here the gate uploads them in C (page-locked staging, no host wait) and runs
the same device kernels as for device-resident data.  Checked: the gate's
counters show the calls taken natively (uploads, op, materialisation, no
hand-back to Python), results match the oracle (IEEE add exact, sin within
2 ULP, sum within 1e-5 of the float64 sum), and a run of uploads that wraps
the staging ring several times before the device has consumed them keeps
every operand intact.
"""
import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd import _gate
from oracle import reference_cpu as ref

pytestmark = pytest.mark.gpu


def _delta(s0, s1):
    return {k: s1[k] - s0[k] for k in ("native_uploads", "native_ops", "native_materialize",
                                       "fallbacks")}


@pytest.mark.parametrize("n", [1 << 10, 1 << 16])
def test_small_host_calls_take_the_native_gate(n):
    print(f"small host calls n={n}", flush=True)
    # (run first in a process, this also checks that the gate sets up the
    # device itself on the first host upload)
    g = np.random.default_rng(n)
    a_np = g.standard_normal(n, dtype=np.float32)
    b_np = g.standard_normal(n, dtype=np.float32)

    s0 = _gate.stats()
    got = (cp.array(a_np) + cp.array(b_np)).get()
    d = _delta(s0, _gate.stats())
    assert d == {"native_uploads": 2, "native_ops": 1, "native_materialize": 1, "fallbacks": 0}, d
    assert np.array_equal(got, ref.binary("add_op", a_np, b_np))

    s0 = _gate.stats()
    got = cp.sin(cp.array(a_np)).get()
    d = _delta(s0, _gate.stats())
    assert d == {"native_uploads": 1, "native_ops": 1, "native_materialize": 1, "fallbacks": 0}, d
    assert int(ref.ulp_distance(got, ref.unary("sin_op", a_np)).max()) <= 2

    s0 = _gate.stats()
    got = float(cp.sum(cp.array(a_np)))
    d = _delta(s0, _gate.stats())
    assert d == {"native_uploads": 1, "native_ops": 1, "native_materialize": 0, "fallbacks": 0}, d
    want = float(ref.sum_f64(a_np))
    assert abs(got - want) <= 1e-5 * max(1.0, abs(want))

    # argmax of host data: a Python int through the same upload
    s0 = _gate.stats()
    assert cp.argmax(cp.array(a_np)) == int(np.argmax(a_np))
    assert _delta(s0, _gate.stats())["native_uploads"] == 1


def test_uploads_wrapping_the_staging_ring_stay_intact():
    """64 uploads of 256 KiB (16 MiB, twice the staging ring) queued before
    any of them is read: each operand's bytes must reach the device before
    its staging segment is reused.  x * 1.0 is exact, so every result must
    equal its input bit for bit."""
    print("staging ring wrap: 64 x 256 KiB", flush=True)
    g = np.random.default_rng(7)
    xs = [g.standard_normal(1 << 16, dtype=np.float32) for _ in range(64)]
    s0 = _gate.stats()
    ys = [cp.array(x) * 1.0 for x in xs]
    assert _gate.stats()["native_uploads"] - s0["native_uploads"] == 64
    tot = ys[0]
    for y in ys[1:8]:
        tot = tot + y
    for x, y in zip(xs, ys):
        assert np.array_equal(y.get(), x)
    want = xs[0].copy()
    for x in xs[1:8]:
        want = want + x
    assert np.array_equal(tot.get(), want)


def test_uploads_of_changing_host_data_and_sizes():
    """One NumPy buffer rewritten between uploads (each upload must have
    copied it at call time), sizes around the 1 MiB staging limit (staged
    and direct copies interleaved), and set() of a host array."""
    print("staging: rewritten source, sizes around 1 MiB", flush=True)
    src = np.zeros(1 << 18, dtype=np.float32)       # exactly 1 MiB
    arrs, wants = [], []
    for i in range(20):
        src[:] = i
        arrs.append(cp.array(src) * 1.0)
        wants.append(np.full(src.shape, i, np.float32))
    for n in ((1 << 18) - 1, (1 << 18) + 1, 3, 1 << 19, 17):
        h = np.arange(n, dtype=np.float32)
        arrs.append(cp.array(h) + 0.0)
        wants.append(h)
    for a, w in zip(arrs, wants):
        assert np.array_equal(a.get(), w)
    d = cp.zeros(1000, dtype=np.float32)
    d._ensure_gpu()
    for i in range(5):
        d.set(np.full(1000, i, np.float32))
    assert np.array_equal((d + 0.0).get(), np.full(1000, 4, np.float32))
