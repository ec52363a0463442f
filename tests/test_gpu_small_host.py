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
    copied it at call time), sizes around the 32 KiB kernel-copy limit
    (kernel and DMA transfers, up and down) and the 1 MiB staging limit
    (staged and direct copies interleaved), and set() of a host array."""
    print("staging: rewritten source, sizes around 32 KiB and 1 MiB", flush=True)
    src = np.zeros(1 << 18, dtype=np.float32)       # exactly 1 MiB
    arrs, wants = [], []
    for i in range(20):
        src[:] = i
        arrs.append(cp.array(src) * 1.0)
        wants.append(np.full(src.shape, i, np.float32))
    for n in ((1 << 18) - 1, (1 << 18) + 1, 3, 1 << 19, 17, (1 << 13) - 1, 1 << 13,
              (1 << 13) + 1, 8190, 8195):
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


_HOST_DTYPES = [np.bool_, np.int16, np.uint16, np.int32, np.uint32, np.int64, np.float16,
                np.float32, np.float64]
_UNARY = ["negative", "absolute", "sqrt", "exp", "sin", "floor", "square"]
_BINARY = ["add", "subtract", "multiply", "maximum", "less", "floor_divide"]
_REDUCE = ["sum", "max", "argmax", "mean"]


def _host_values(rng, shape, dtype):
    dt = np.dtype(dtype)
    if dt == np.bool_:
        return rng.random(shape) < 0.5
    if dt.kind in "iu":
        lo = -50 if dt.kind == "i" else 1
        return rng.integers(lo, 50, shape).astype(dt)
    return rng.standard_normal(shape).astype(dt)


def _same(got, want, dtype):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    if np.dtype(dtype).kind == "f" and want.dtype.kind == "f":
        if want.dtype == np.float16:
            assert int(ref.ulp_distance(got.astype(np.float16), want).max(initial=0)) <= 2
        else:
            assert np.allclose(got, want, rtol=1e-5, atol=1e-6, equal_nan=True)
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("seed", range(40))
def test_random_calls_on_fresh_host_arrays(seed):
    """Random unary / binary / reduction calls whose operands are arrays made
    from NumPy data in the call (0-d to 3-D, broadcasting pairs, strided
    host views that the gate hands to the Python path) match NumPy; every
    contiguous operand is uploaded by the gate."""
    print(f"fresh host arrays seed={seed}", flush=True)
    rng = np.random.default_rng(1000 + seed)
    shapes = [(), (1,), (7,), (3, 5), (2, 3, 4), (1000,)]
    for _ in range(12):
        dt = _HOST_DTYPES[rng.integers(len(_HOST_DTYPES))]
        shape = shapes[rng.integers(len(shapes))]
        x_np = _host_values(rng, shape, dt)
        strided = len(shape) >= 1 and shape[-1] > 1 and rng.random() < 0.2
        src = np.repeat(x_np, 2, axis=-1)[..., ::2] if strided else x_np
        kind = rng.integers(3)
        s0 = _gate.stats()["native_uploads"]
        if kind == 0:
            op = _UNARY[rng.integers(len(_UNARY))]
            if dt == np.bool_ and op != "absolute":
                continue
            with np.errstate(all="ignore"):
                want = getattr(np, op)(x_np)
            got = getattr(cp, op)(cp.asarray(src)).get()
            _same(got, want, want.dtype)
            ups = 0 if strided else 1
        elif kind == 1:
            op = _BINARY[rng.integers(len(_BINARY))]
            if dt == np.bool_ and op in ("subtract", "floor_divide"):
                continue
            other_shape = shape[-1:] if len(shape) >= 1 and rng.random() < 0.5 else shape
            y_np = _host_values(rng, other_shape, dt)
            if op == "floor_divide" and np.dtype(dt).kind in "iu":
                y_np = np.where(y_np == 0, 1, y_np).astype(dt)
            with np.errstate(all="ignore"):
                want = getattr(np, op)(x_np, y_np)
            got = getattr(cp, op)(cp.asarray(src), cp.array(y_np)).get()
            _same(got, want, want.dtype)
            ups = 0 if strided else 2
        else:
            op = _REDUCE[rng.integers(len(_REDUCE))]
            axis = None if len(shape) == 0 or rng.random() < 0.5 else -1
            if op == "mean" and dt == np.float16:
                continue
            if op == "sum" and np.dtype(dt).kind == "f":
                # float sums accumulate in float64 and round once
                want = np.sum(x_np.astype(np.float64), axis=axis).astype(dt)
            else:
                want = getattr(np, op)(x_np, axis=axis)
            got = getattr(cp, op)(cp.asarray(src), axis=axis)
            got = got.get() if hasattr(got, "get") else got
            _same(got, want, np.asarray(want).dtype)
            ups = 0 if strided else 1
        assert _gate.stats()["native_uploads"] - s0 >= ups, (kind, op, dt, shape, strided)


def test_small_copies_with_host_memory_pointers():
    """mmp_h2d / mmp_d2h accept page-locked host memory on the device side
    of the copy as DMA copies do: a pointer the runtime does not know as
    device memory takes the DMA path, not the copy kernel."""
    import ctypes
    from macmetalpy_amd._backend import HipBackend, load_library
    print("small copies with host memory pointers", flush=True)
    HipBackend()
    lib = load_library()
    p = ctypes.c_void_p()
    assert lib.mmp_host_alloc(4096, ctypes.byref(p)) == 0
    try:
        src = np.arange(1024, dtype=np.int32)
        assert lib.mmp_h2d(p.value, src.ctypes.data, src.nbytes) == 0   # "device" side is host memory
        got = np.empty(1024, np.int32)
        assert lib.mmp_d2h(got.ctypes.data, p.value, got.nbytes) == 0
        assert np.array_equal(got, src)
    finally:
        assert lib.mmp_host_free(p.value) == 0
