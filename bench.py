"""Benchmark of the MI355X array-compute hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--suite all|headline]

Prints ONE JSON line.  The headline ``value`` is the whole-job HBM
throughput (algorithmic GB/s) of the binary-elementwise workload at 2^28
elements -- one step = a+b and sin(a) on float32, floor_divide(a, b) and
mod(a, b) on int32 -- with inputs resident in HBM.  ``roofline`` describes
the step's dominant kernel, timed with HIP events on the library stream over
the timed region.  ``cpu_baseline`` times the reference's CPU/NumPy path
(the oracle restatement) on a bounded sample on this host.  ``configs``
holds the other workloads (fused elementwise, reductions, scans, matmul,
fusion chain) measured the same way.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
PEAK_TFLOPS = {"float32": 157.3, "float16": 2500.0, "bfloat16": 2500.0, "float64": 78.6}
N28 = 1 << 28


def _log(msg):
    print(msg, file=sys.stderr, flush=True)


class EventTimer:
    """Per-op kernel time from event pairs recorded on the library stream."""

    def __init__(self, be):
        self.be = be
        self.pairs = {}

    def run(self, name, fn):
        s, e = self.be.event(), self.be.event()
        self.be.record(s)
        out = fn()
        self.be.record(e)
        self.pairs.setdefault(name, []).append((s, e))
        return out

    def ms(self, name):
        vals = [self.be.elapsed_ms(s, e) for s, e in self.pairs[name]]
        return statistics.mean(vals), vals

    def close(self):
        for lst in self.pairs.values():
            for s, e in lst:
                self.be.destroy_event(s)
                self.be.destroy_event(e)
        self.pairs = {}


def _traffic_table():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f)
    return {}


# --------------------------------------------------------------- C2
def bench_c2(cp, be, steps, warmup):
    """Headline: a+b, sin(a) (float32) and floor_divide, mod (int32), 2^28."""
    from macmetalpy_amd.workloads import c2_float_inputs, c2_int_inputs
    t0 = time.time()
    a_np, b_np = c2_float_inputs(N28)
    a, b = cp.array(a_np), cp.array(b_np)
    del a_np, b_np
    ai_np, bi_np = c2_int_inputs(N28)
    ai, bi = cp.array(ai_np), cp.array(bi_np)
    del ai_np, bi_np
    for x in (a, b, ai, bi):
        x._ensure_gpu()
    cp.synchronize()
    _log(f"c2 inputs ready in {time.time() - t0:.1f}s")
    ops = {
        "add_f32": (lambda: a + b, 12),
        "sin_f32": (lambda: cp.sin(a), 8),
        "floor_divide_i32": (lambda: cp.floor_divide(ai, bi), 12),
        "mod_i32": (lambda: cp.mod(ai, bi), 12),
    }

    def step(timer=None, timed=()):
        outs = []
        for name, (fn, _) in ops.items():
            if timer is None or name not in timed:
                r = fn()
                r._materialize_if_lazy()
            else:
                r = timer.run(name, lambda fn=fn: _mat(fn()))
            outs.append(r)
        return outs

    for _ in range(warmup):
        step()
    cp.synchronize()
    # The timed steps carry one event pair, around the roofline kernel (a+b):
    # an event record between two kernels costs the step ~4 us of device
    # time, and one pair per op made the step ~30 us (1.5 %) longer.
    timer = EventTimer(be)
    t = time.perf_counter()
    for _ in range(steps):
        step(timer, timed=("add_f32",))
    cp.synchronize()
    wall = time.perf_counter() - t
    # the other ops' kernel times: the same steps again, an event pair per op
    for _ in range(steps):
        step(timer, timed=tuple(n for n in ops if n != "add_f32"))
    cp.synchronize()
    per_op = {}
    for name, (_, bpe) in ops.items():
        ms, _ = timer.ms(name)
        per_op[name] = {"kernel_ms": round(ms, 4), "bytes": bpe * N28,
                        "gbs": round(bpe * N28 / ms / 1e6, 1),
                        "frac_of_peak": round(bpe * N28 / ms / 1e6 / HBM_PEAK_GBS, 4)}
    timer.close()
    bytes_per_step = sum(bpe for _, bpe in ops.values()) * N28
    return {"wall_s": wall, "bytes_per_step": bytes_per_step, "per_op": per_op}


def _mat(r):
    r._materialize_if_lazy()
    return r


# The reference's published "scaling story" (README.md:107-118: speedup of
# macmetalpy over NumPy on an M4 Mac mini, float32, at 1K / 100K / 1M).
REFERENCE_SCALING = {
    "add": (0.40, 0.93, 0.98), "sin": (0.69, 0.98, 2.41), "exp": (0.72, 0.96, 2.12),
    "cumsum": (0.59, 1.40, 1.39), "floor_divide": (0.79, 3.04, 11.12),
    "mod": (0.76, 2.35, 7.57), "randn": (2.88, 3.71, 3.69), "normal": (2.02, 2.48, 2.47),
    "sort": (0.84, 0.93, 1.57), "searchsorted": (0.01, 4.12, 32.50),
}
SCALING_SIZES = (1_000, 100_000, 1_000_000)


def bench_scaling_vs_numpy(cp, be, warm=2, reps=15):
    """The reference's scaling table re-measured here with its method
    (bench_core.py:276-357, 368-402; bench_advanced.py:316-365, 550-608):
    inputs made with np.random (rand + 0.1 for the ufuncs, rand for cumsum
    and sort, a sorted base with size // 10 queries for searchsorted) and
    put on the device once; a timed call is the op plus .get() of its
    result (randn / normal: generation plus .get()); NumPy runs the same
    call on the host copy.  Medians of ``reps`` after ``warm`` warm-ups
    (the reference: 5 after 2).  ``speedup`` = NumPy time / this time;
    ``reference_speedup`` is the README's M4 figure for the same cell."""
    rng = np.random.default_rng(31)

    def median_s(f):
        for _ in range(warm):
            f()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            f()
            ts.append(time.perf_counter() - t)
        return statistics.median(ts)

    res = {}
    for si, n in enumerate(SCALING_SIZES):
        a_np = (rng.random(n) + 0.1).astype(np.float32)
        b_np = (rng.random(n) + 0.1).astype(np.float32)
        r_np = rng.random(n).astype(np.float32)
        base_np = np.sort(rng.random(n).astype(np.float32))
        q_np = rng.random(max(n // 10, 1)).astype(np.float32)
        a, b, r, base, q = (cp.array(x) for x in (a_np, b_np, r_np, base_np, q_np))
        for x in (a, b, r, base, q):
            x._ensure_gpu()
        cases = {
            "add": (lambda: cp.add(a, b).get(), lambda: np.add(a_np, b_np)),
            "sin": (lambda: cp.sin(a).get(), lambda: np.sin(a_np)),
            "exp": (lambda: cp.exp(a).get(), lambda: np.exp(a_np)),
            "cumsum": (lambda: cp.cumsum(r).get(), lambda: np.cumsum(r_np)),
            "floor_divide": (lambda: cp.floor_divide(a, b).get(),
                             lambda: np.floor_divide(a_np, b_np)),
            "mod": (lambda: cp.mod(a, b).get(), lambda: np.mod(a_np, b_np)),
            "randn": (lambda: cp.random.randn(n).get(), lambda: np.random.randn(n)),
            "normal": (lambda: cp.random.normal(0.0, 1.0, size=(n,)).get(),
                       lambda: np.random.normal(0.0, 1.0, size=(n,))),
            "sort": (lambda: cp.sort(r).get(), lambda: np.sort(r_np)),
            "searchsorted": (lambda: cp.searchsorted(base, q).get(),
                             lambda: np.searchsorted(base_np, q_np)),
        }
        label = {1_000: "1K", 100_000: "100K", 1_000_000: "1M"}[n]
        sec = {}
        for name, (dev, host) in cases.items():
            t_dev = median_s(dev)
            t_np = median_s(host)
            sec[name] = {"us": round(t_dev * 1e6, 1), "numpy_us": round(t_np * 1e6, 1),
                         "speedup": round(t_np / t_dev, 2),
                         "reference_speedup": REFERENCE_SCALING[name][si]}
        res[label] = sec
        del a, b, r, base, q
    return res


def vendor_copy(cp, be, reps=20):
    """The HIP runtime's own device-to-device copy (hipMemcpyAsync on the
    library stream) of 2^28 float32 beside the library's copy kernel and
    a + b over the same arrays: GB/s of the algorithmic bytes (copy 8 B,
    a + b 12 B per element), mean of ``reps`` back-to-back calls."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    hip.hipMemcpyAsync.argtypes = [vp, vp, ctypes.c_size_t, ctypes.c_int, vp]
    hip.hipMemcpyAsync.restype = ctypes.c_int
    stream = vp()
    if be._lib.mmp_stream(ctypes.byref(stream)) != 0:
        raise RuntimeError("mmp_stream failed")
    from macmetalpy_amd.workloads import c2_float_inputs
    a, b = (cp.array(x) for x in c2_float_inputs(N28))
    for x in (a, b):
        x._ensure_gpu()
    dst = be.create_buffer(N28, np.float32)

    def d2d():
        if hip.hipMemcpyAsync(dst.ptr, a._ptr, 4 * N28, 3, stream) != 0:  # DeviceToDevice
            raise RuntimeError("hipMemcpyAsync failed")

    res = {}
    for name, f, bpe in (("hipMemcpy_d2d", d2d, 8), ("library_copy", lambda: _mat(a.copy()), 8),
                         ("library_add", lambda: _mat(a + b), 12)):
        ms = _launch_ms(cp, be, f, reps)
        res[name] = {"ms": round(ms, 4), "gbs": round(bpe * N28 / ms / 1e6, 1)}
    return res


_VENDOR_TORCH = r"""
import json, torch
torch.backends.cuda.matmul.allow_tf32 = False
out = {"torch": torch.__version__, "elementwise_2p28": {}, "gemm": {}}


def timed(f, warm, reps):
    for _ in range(warm):
        f()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        f()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


n = 1 << 28
g = torch.Generator(device="cuda").manual_seed(2)
a = torch.randn(n, device="cuda", generator=g)
b = torch.randn(n, device="cuda", generator=g)
c = torch.empty_like(a)
for name, f, bpe in (("copy", lambda: c.copy_(a), 8), ("add", lambda: torch.add(a, b, out=c), 12),
                     ("sin", lambda: torch.sin(a, out=c), 8)):
    ms = timed(f, 3, REPS)
    out["elementwise_2p28"][name] = {"ms": round(ms, 4), "gbs": round(bpe * n / ms / 1e6, 1)}
del a, b, c
for name, (m, nn, k, bt), dt in (("f32", (4096, 4096, 4096, 1), torch.float32),
                                 ("f16", (8192, 8192, 8192, 1), torch.float16),
                                 ("batched", (1024, 1024, 1024, 64), torch.float32)):
    a = torch.randn((bt, m, k) if bt > 1 else (m, k), device="cuda", dtype=dt, generator=g)
    c = torch.randn((bt, k, nn) if bt > 1 else (k, nn), device="cuda", dtype=dt, generator=g)
    ms = timed(lambda: a @ c, 10, REPS)
    out["gemm"][name] = {"kernel_ms": round(ms, 4), "tflops": round(2.0 * m * nn * k * bt / ms / 1e9, 2)}
    del a, c
print(json.dumps(out))
"""


def vendor_torch(cp, be, reps=20):
    """The vendor's own paths on the same device, for scale: torch's copy_,
    add and sin over 2^28 float32 (GB/s of the algorithmic bytes, as C2) and
    torch.matmul (hipBLASLt; TF32 off) on the C4 shapes -- float32 4096^3,
    float16 8192^3, batched float32 64 x 1024^3 -- each ``reps`` back-to-back
    calls between two torch events after a warm-up (3 calls elementwise, 10
    matmul, as c4_matmul).  It runs in a child process: torch does not
    share the device with this process's HIP context."""
    import subprocess
    p = subprocess.run([sys.executable, "-c", _VENDOR_TORCH.replace("REPS", str(int(reps)))],
                       capture_output=True, text=True, timeout=600)
    if p.returncode != 0:
        raise RuntimeError(f"torch child exited {p.returncode}: {p.stderr[-300:]}")
    return json.loads(p.stdout.strip().splitlines()[-1])


def bench_c2_end_to_end(cp, be, reps=5):
    """The C2 calls timed end to end from Python, as the reference's
    bench_core.py:291-297 times `cp_func(data).get()`: ``call_sync_ms`` is a
    call plus cp.synchronize() (host dispatch, kernel, wait),
    ``call_get_ms`` a call plus .get() (the 1 GiB result copied into host
    memory); medians of ``reps`` after one warm-up, inputs resident in HBM.
    ``d2h_gbs`` is the result bytes over the difference of the two."""
    from macmetalpy_amd.workloads import c2_float_inputs, c2_int_inputs
    a, b = (cp.array(x) for x in c2_float_inputs(N28))
    ai, bi = (cp.array(x) for x in c2_int_inputs(N28))
    for x in (a, b, ai, bi):
        x._ensure_gpu()
    cp.synchronize()
    ops = {"add_f32": lambda: a + b, "sin_f32": lambda: cp.sin(a),
           "floor_divide_i32": lambda: cp.floor_divide(ai, bi), "mod_i32": lambda: cp.mod(ai, bi)}

    def median_ms(f):
        f()
        ts = []
        for _ in range(reps):
            t = time.perf_counter()
            f()
            ts.append((time.perf_counter() - t) * 1e3)
        return statistics.median(ts)

    res = {}
    for name, fn in ops.items():
        sync_ms = median_ms(lambda: (_mat(fn()), cp.synchronize()))
        get_ms = median_ms(lambda: fn().get())
        res[name] = {"call_sync_ms": round(sync_ms, 3), "call_get_ms": round(get_ms, 3),
                     "d2h_gbs": round(4 * N28 / max(get_ms - sync_ms, 1e-6) / 1e6, 1)}
    return res


def _launch_ms(cp, be, f, reps):
    """Mean device time per call over ``reps`` back-to-back calls between
    one pair of events on the library stream: the queue stays ahead of the
    host, so neither the per-call event overhead (a few microseconds) nor
    host gaps enter a kernel's time.  One untimed call is queued ahead of
    the start event, so the device is busy when the window opens (else the
    window would begin with the host's time to issue the first call)."""
    s, e = be.event(), be.event()
    f()
    be.record(s)
    for _ in range(reps):
        f()
    be.record(e)
    cp.synchronize()
    ms = be.elapsed_ms(s, e) / reps
    be.destroy_event(s)
    be.destroy_event(e)
    return ms


# --------------------------------------------------------------- C1
def _call_us(cp, f, n_calls):
    """Host-inclusive time per call: ``n_calls`` back-to-back calls (each
    result evaluated), one synchronisation at the end."""
    t = time.perf_counter()
    for _ in range(n_calls):
        f()
    cp.synchronize()
    return (time.perf_counter() - t) / n_calls * 1e6


def bench_c1(cp, be, reps=50):
    """C1 y = sqrt(abs(x)) + exp(-x**2): ``kernel_ms`` is the device time per
    call over back-to-back calls between one event pair (at 2^20 the device
    waits for the host between launches, so it is the host's call rate),
    ``call_us`` the host-inclusive time per call of back-to-back calls; both
    count the whole call (6 lazy ops, one fused kernel)."""
    from macmetalpy_amd.workloads import c1_inputs
    res = {}
    for label, n in (("2^20", 1 << 20), ("2^28", N28)):
        x = cp.array(c1_inputs(n))
        x._ensure_gpu()
        f = lambda: _mat(cp.sqrt(cp.abs(x)) + cp.exp(-x ** 2))  # noqa: E731
        for _ in range(3):
            f()
        cp.synchronize()
        ms = _launch_ms(cp, be, f, reps if n < N28 else 10)
        res[label] = {"kernel_ms": round(ms, 4), "gbs": round(8 * n / ms / 1e6, 1),
                      "frac_of_peak": round(8 * n / ms / 1e6 / HBM_PEAK_GBS, 4)}
        if n < N28:
            res[label]["call_us"] = round(_call_us(cp, f, 2000), 2)
            # end to end with the result read back to the host each call
            # (the reference's bench_core.py:291-297 times the call + get)
            g = lambda: (cp.sqrt(cp.abs(x)) + cp.exp(-x ** 2)).get()  # noqa: E731
            g()
            t = time.perf_counter()
            for _ in range(200):
                g()
            res[label]["call_get_us"] = round((time.perf_counter() - t) / 200 * 1e6, 2)
        del x
    return res


def bench_small_ops(cp, be, n=1 << 20, calls=2000):
    """Per-call time of single small ops on 2^20 float32 (host dispatch
    included; the reference's bench_vs_numpy.py:30-45 times these calls
    end to end): back-to-back calls, one synchronisation at the end."""
    g = np.random.default_rng(0)
    x = cp.array(g.standard_normal(n, dtype=np.float32))
    y = cp.array(g.standard_normal(n, dtype=np.float32))
    x._ensure_gpu()
    y._ensure_gpu()
    cases = {"add": lambda: _mat(x + y), "mul_scalar": lambda: _mat(x * 2.5),
             "sin": lambda: _mat(cp.sin(x)), "sum": lambda: cp.sum(x),
             "argmax": lambda: cp.argmax(x), "cumsum": lambda: cp.cumsum(x),
             "c1_fused": lambda: _mat(cp.sqrt(cp.abs(x)) + cp.exp(-x ** 2))}
    res = {}
    for name, f in cases.items():
        for _ in range(50):
            f()
        cp.synchronize()
        res[name] = {"call_us": round(_call_us(cp, f, calls), 2)}
    return res


SMALL_HOST_SIZES = (("1K", 1 << 10), ("64K", 1 << 16))


def _small_host_cases(cp, a_np, b_np):
    """The three calls on arrays created from host (NumPy) data each call:
    the case the reference's C gate answers on the CPU (_accelerator.c:
    549-712 fast_binary / fast_unary, :798-858 fast_reduce, below the
    thresholds of ndarray.py:41-44)."""
    return {"add_get": lambda: (cp.array(a_np) + cp.array(b_np)).get(),
            "sin_get": lambda: cp.sin(cp.array(a_np)).get(),
            "sum_float": lambda: float(cp.sum(cp.array(a_np)))}


def bench_small_host_ops(cp, be, calls=1000):
    """Per-call time of (a+b).get(), sin(a).get() and float(sum(a)) on
    float32 arrays made from NumPy data in the call (host-resident until
    the native gate uploads them through page-locked staging), end to end
    with the result back on the host.  ``gate`` is the native gate's
    counters per call: uploads, ops and materialisations done in C, calls
    handed to the Python path.  The NumPy time of the same calls (the
    reference's CPU path) is filled in beside each from ``cpu_baseline``."""
    from macmetalpy_amd import _gate
    res = {}
    for label, n in SMALL_HOST_SIZES:
        g = np.random.default_rng(n)
        a_np = g.standard_normal(n, dtype=np.float32)
        b_np = g.standard_normal(n, dtype=np.float32)
        sec = {}
        for name, f in _small_host_cases(cp, a_np, b_np).items():
            for _ in range(50):
                f()
            k = calls if n <= 4096 else calls // 4
            s0 = _gate.stats()
            t = time.perf_counter()
            for _ in range(k):
                f()
            dt = time.perf_counter() - t
            s1 = _gate.stats()
            per = {key: round((s1[key] - s0[key]) / k, 3)
                   for key in ("native_uploads", "native_ops", "native_materialize", "fallbacks")}
            sec[name] = {"call_us": round(dt / k * 1e6, 2), "gate_per_call": per}
        res[label] = sec
    return res


def _small_host_cpu(reps=2000):
    """NumPy time of the small host calls, as the reference's CPU path runs
    them (the array copy of cp.array, then the NumPy ufunc / reduction);
    the reference's Python wrapper around them is not included."""
    out = {}
    for label, n in SMALL_HOST_SIZES:
        g = np.random.default_rng(n)
        a_np = g.standard_normal(n, dtype=np.float32)
        b_np = g.standard_normal(n, dtype=np.float32)
        cases = {"add_get": lambda: np.add(a_np.copy(), b_np.copy()),
                 "sin_get": lambda: np.sin(a_np.copy()),
                 "sum_float": lambda: float(np.sum(a_np.copy()))}
        sec = {}
        for name, f in cases.items():
            k = reps if n <= 4096 else reps // 4
            for _ in range(50):
                f()
            t = time.perf_counter()
            for _ in range(k):
                f()
            sec[name] = {"call_us": round((time.perf_counter() - t) / k * 1e6, 2)}
        out[label] = sec
    return out


# --------------------------------------------------------------- C3
def bench_c3(cp, be, reps=10):
    from macmetalpy_amd.workloads import c3_matrix, c3_scan_inputs
    A = cp.array(c3_matrix())
    A._ensure_gpu()
    nbytes = 4 * A.size
    res = {}
    cases = {
        "sum_all": lambda: cp.sum(A), "mean_all": lambda: cp.mean(A),
        "sum_axis1": lambda: cp.sum(A, axis=1), "mean_axis1": lambda: cp.mean(A, axis=1),
        "argmax_axis1": lambda: cp.argmax(A, axis=1),
        "argmax_all": lambda: cp.argmax(A, axis=None, keepdims=True),
        # the same matrix reduced over its strided axis
        "sum_axis0": lambda: cp.sum(A, axis=0), "argmax_axis0": lambda: cp.argmax(A, axis=0),
        "cumsum_axis0": lambda: cp.cumsum(A, axis=0),       # 4 B read + 4 B written
    }
    for name, f in cases.items():
        nb = 2 * nbytes if name == "cumsum_axis0" else nbytes
        try:
            f()
            cp.synchronize()
            ms = _launch_ms(cp, be, f, reps)
            res[name] = {"kernel_ms": round(ms, 4), "gbs": round(nb / ms / 1e6, 1),
                         "frac_of_peak": round(nb / ms / 1e6 / HBM_PEAK_GBS, 4)}
        except Exception as e:  # report, keep going
            res[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
    del A
    ci, cf = c3_scan_inputs(N28)
    for name, arr, bpe in (("cumsum_i32_to_i64", ci, 12), ("cumsum_f32", cf, 8)):
        try:
            x = cp.array(arr)
            x._ensure_gpu()
            f = lambda: cp.cumsum(x)  # noqa: E731
            f()
            cp.synchronize()
            ms = _launch_ms(cp, be, f, reps)
            res[name] = {"kernel_ms": round(ms, 4), "gbs": round(bpe * N28 / ms / 1e6, 1),
                         "frac_of_peak": round(bpe * N28 / ms / 1e6 / HBM_PEAK_GBS, 4)}
            del x
        except Exception as e:
            res[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
    return res


# Copy kernels with the data movement of the contiguous scan (k_scan_rows,
# scan.hip) and none of its arithmetic: the same 16384-element tile per
# 256-thread workgroup, all 16-byte loads of the tile issued first, each
# 4096-element sub-tile redistributed through LDS (padded rows) so that a
# thread holds 16 consecutive elements, written back through LDS in the
# output type and stored with 16-byte non-temporal stores, sub-tile by
# sub-tile.  No in-tile scan, no look-back; the LDS stage is sized for the
# wider of the two types, as the scan's.  What the tile shape alone
# allows, beside the scan.
_SCAN_SHAPE_COPY_SRC = r"""
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int pad16(int i) { return i + i / 16; }
template <typename Ti, typename To>
__device__ __forceinline__ void tile_copy(const Ti* __restrict__ x, To* __restrict__ y,
                                          unsigned char* stage) {
  constexpr int kSub = 4096, VI = 16 / sizeof(Ti), VO = 16 / sizeof(To);
  constexpr int NV = kSub / VI / 256, NO = kSub / VO / 256;
  Ti* sx = (Ti*)stage;
  To* sy = (To*)stage;
  const int tid = threadIdx.x;
  const long long base = (long long)blockIdx.x * 4 * kSub;
  const u32x4* xv = (const u32x4*)(x + base);
  u32x4 raw[4][NV];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int k = 0; k < NV; ++k)
      raw[q][k] = __builtin_nontemporal_load(xv + q * (kSub / VI) + k * 256 + tid);
  Ti xin[4][16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (q) __syncthreads();
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      union { u32x4 v; Ti e[VI]; } u;
      u.v = raw[q][k];
#pragma unroll
      for (int e = 0; e < VI; ++e) sx[pad16((k * 256 + tid) * VI + e)] = u.e[e];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 16; ++j) xin[q][j] = sx[pad16(tid * 16 + j)];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int j = 0; j < 16; ++j) sy[pad16(tid * 16 + j)] = (To)xin[q][j];
    __syncthreads();
    u32x4* yv = (u32x4*)(y + base + q * kSub);
#pragma unroll
    for (int k = 0; k < NO; ++k) {
      union { u32x4 v; To e[VO]; } u;
#pragma unroll
      for (int e = 0; e < VO; ++e) u.e[e] = sy[pad16((k * 256 + tid) * VO + e)];
      __builtin_nontemporal_store(u.v, yv + k * 256 + tid);
    }
    __syncthreads();
  }
}
extern "C" __global__ __launch_bounds__(256) void tilecopy_f32(const float* x, float* y) {
  __shared__ __attribute__((aligned(16))) unsigned char stage[4 * 4352];
  tile_copy<float, float>(x, y, stage);
}
extern "C" __global__ __launch_bounds__(256) void tilecopy_i32_i64(const int* x, long long* y) {
  __shared__ __attribute__((aligned(16))) unsigned char stage[8 * 4352];
  tile_copy<int, long long>(x, y, stage);
}
"""


def scan_shape_copy(cp, be, reps=10):
    """GB/s of the scan-shaped copies at 2^28 elements (float32 -> float32,
    int32 -> int64), each output checked against its input, with the scan
    (cumsum) of the same input and the plain library copy beside them."""
    res = {}
    for name, dt_in, dt_out, bpe in (("tilecopy_f32", np.float32, np.float32, 8),
                                     ("tilecopy_i32_i64", np.int32, np.int64, 12)):
        x_np = (np.arange(N28, dtype=np.int64) % 1000003).astype(dt_in)
        x = cp.array(x_np)
        x._ensure_gpu()
        y = cp.empty(N28, dtype=dt_out)
        y._ensure_gpu()
        k = cp.RawKernel(_SCAN_SHAPE_COPY_SRC, name)
        assert N28 % 16384 == 0
        k((N28 // 16384 * 256,), (x, y))
        cp.synchronize()
        ok = bool(np.array_equal(y.get(), x_np.astype(dt_out)))
        ms = _launch_ms(cp, be, lambda: k((N28 // 16384 * 256,), (x, y)), reps)
        res[name] = {"kernel_ms": round(ms, 4), "gbs": round(bpe * N28 / ms / 1e6, 1),
                     "frac_of_peak": round(bpe * N28 / ms / 1e6 / HBM_PEAK_GBS, 4),
                     "copy_exact": ok}
        # the scan itself on the same input, same session
        del y
        cp.cumsum(x)
        cp.synchronize()
        ms_scan = _launch_ms(cp, be, lambda: cp.cumsum(x), reps)
        res[name]["scan_kernel_ms"] = round(ms_scan, 4)
        res[name]["scan_gbs"] = round(bpe * N28 / ms_scan / 1e6, 1)
        res[name]["scan_vs_copy"] = round(ms / ms_scan, 4)
        del x
    x = cp.array(np.ones(N28, dtype=np.float32))
    x._ensure_gpu()
    x.copy()
    cp.synchronize()
    ms = _launch_ms(cp, be, lambda: x.copy(), reps)
    res["library_copy_f32"] = {"kernel_ms": round(ms, 4), "gbs": round(8 * N28 / ms / 1e6, 1),
                               "frac_of_peak": round(8 * N28 / ms / 1e6 / HBM_PEAK_GBS, 4)}
    return res


# --------------------------------------------------------------- C4
# Register-only MFMA loop with random (finite) float16 operands: the matrix
# units' practical ceiling when they are fed with no data movement at all
# (the clock falls with operand toggling, so this sits below the 2.5 PF/s
# dense spec).  Eight independent 16x16x32 (or four 32x32x16) accumulators
# per wave, operands rotated so that consecutive MFMAs see different bits.
_MFMA_CEILING_SRC = r"""
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
__device__ inline h8 operand(unsigned s) {
  u4 u;
  u.x = s * 2654435761u; u.y = u.x * 2246822519u + 7u;
  u.z = u.y * 3266489917u + 11u; u.w = u.z * 668265263u + 13u;
  u &= 0xbfffbfffu;  // clear each half's top exponent bit: finite values
  return __builtin_bit_cast(h8, u);
}
extern "C" __global__ __launch_bounds__(256) void mfma16(float* out, int iters, unsigned seed) {
  const unsigned t = blockIdx.x * 256 + threadIdx.x;
  h8 a[4], b[4];
  for (int i = 0; i < 4; ++i) { a[i] = operand(seed + t * 8 + i); b[i] = operand(seed ^ (t * 8 + i + 4)); }
  f4 c[8];
  for (int i = 0; i < 8; ++i) c[i] = f4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; it += 4) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        c[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i & 3], b[(i + p) & 3], c[i], 0, 0, 0);
  }
  float s = 0.f;
  for (int i = 0; i < 8; ++i) s += c[i].x + c[i].y + c[i].z + c[i].w;
  out[t] = s;
}
extern "C" __global__ __launch_bounds__(256) void mfma32(float* out, int iters, unsigned seed) {
  const unsigned t = blockIdx.x * 256 + threadIdx.x;
  h8 a[4], b[4];
  for (int i = 0; i < 4; ++i) { a[i] = operand(seed + t * 8 + i); b[i] = operand(seed ^ (t * 8 + i + 4)); }
  f16v c[4];
  for (int i = 0; i < 4; ++i) for (int j = 0; j < 16; ++j) c[i][j] = 0.f;
  for (int it = 0; it < iters; it += 4) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        c[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[(i + p) & 3], c[i], 0, 0, 0);
  }
  float s = 0.f;
  for (int i = 0; i < 4; ++i) for (int j = 0; j < 16; ++j) s += c[i][j];
  out[t] = s;
}
"""


def mfma_ceiling(cp, be, iters=16000, reps=3):
    """TFLOP/s of the register-only float16 MFMA loops (2048 workgroups of
    four waves, ``iters`` steps; best of ``reps`` after one warm-up)."""
    nwg = 2048
    out = cp.zeros(nwg * 256, dtype=np.float32)
    out._ensure_gpu()
    res = {}
    for name in ("mfma16", "mfma32"):
        k = cp.RawKernel(_MFMA_CEILING_SRC, name)
        k((nwg * 256,), (out, np.int32(iters), np.uint32(1)))
        best = None
        for rep in range(reps):
            s, e = be.event(), be.event()
            be.record(s)
            k((nwg * 256,), (out, np.int32(iters), np.uint32(2 + rep)))
            be.record(e)
            cp.synchronize()
            ms = be.elapsed_ms(s, e)
            best = ms if best is None else min(best, ms)
        flops = nwg * 4 * iters * 131072  # 8 x 16x16x32 or 4 x 32x32x16 per step
        res[name] = {"ms": round(best, 3), "tflops": round(flops / best / 1e9, 1)}
    return res


# The register-only float16 MFMA loop with the large GEMM's other traffic
# added beside it at the GEMM's ratios, nothing waiting on that traffic: per
# 16 MFMAs (262,144 flops) a wave reads READS x 1 KiB of LDS (ds_read_b128;
# k_gemm16_dma reads 192 KiB per 8.4 MFLOP slab, 6 KiB per 16 MFMAs) and
# issues DMAS x 1 KiB of global -> LDS copies (global_load_lds_dwordx4 from a
# 2 MiB L2-resident buffer; the GEMM copies 64 KiB per slab, 2 KiB per 16
# MFMAs).  Each wave reads the shader clock counter (s_memtime) and the
# 100 MHz constant clock (s_memrealtime) around its loop, so the engine
# clock under each load comes out beside the rate.
_MFMA_LOAD_SRC = r"""
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
__device__ inline h8 operand(unsigned s) {
  u4 u;
  u.x = s * 2654435761u; u.y = u.x * 2246822519u + 7u;
  u.z = u.y * 3266489917u + 11u; u.w = u.z * 668265263u + 13u;
  u &= 0xbfffbfffu;  // clear each half's top exponent bit: finite values
  return __builtin_bit_cast(h8, u);
}
extern "C" __global__ __launch_bounds__(256) void NAME(const unsigned char* g, float* out,
                                                      unsigned long long* clk, int iters,
                                                      unsigned seed) {
  constexpr int R = READS, D = DMAS;
  constexpr unsigned LDS = 32768u, GB = 2u << 20;
  __shared__ __attribute__((aligned(16))) unsigned char s[LDS];
  const unsigned t = blockIdx.x * 256 + threadIdx.x, lane = threadIdx.x & 63,
                 wave = threadIdx.x >> 6;
  for (unsigned i = threadIdx.x * 16; i < LDS; i += 4096) *(u4*)(s + i) = *(const u4*)(g + i);
  h8 a[4], b[4];
  for (int i = 0; i < 4; ++i) { a[i] = operand(seed + t * 8 + i); b[i] = operand(seed ^ (t * 8 + i + 4)); }
  f4 c[8];
  for (int i = 0; i < 8; ++i) c[i] = f4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; it += 4) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      u4 v[R > 0 ? R : 1];
#pragma unroll
      for (int r = 0; r < R; ++r)
        v[r] = *(const u4*)(s + ((unsigned)(p * 8192 + r * 1024) + wave * 4096u + lane * 16u) % LDS);
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const unsigned go = (blockIdx.x * 131072u + wave * 32768u + (unsigned)(it + p) * 2048u +
                             (unsigned)d * 1024u + lane * 16u) % GB;
        __builtin_amdgcn_global_load_lds(g + go, (__attribute__((address_space(3))) void*)(
            s + (wave * 8192u + (unsigned)d * 1024u) % LDS), 16, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i)
        c[i & 7] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i & 3], b[((i >> 2) + p) & 3], c[i & 7], 0, 0, 0);
#pragma unroll
      for (int r = 0; r < R; ++r) asm volatile("" :: "v"(v[r]));
    }
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  __syncthreads();  // no copy into LDS in flight when the workgroup ends
  float sum = 0.f;
  for (int i = 0; i < 8; ++i) sum += c[i].x + c[i].y + c[i].z + c[i].w;
  out[t] = sum;
  if (lane == 0) { clk[(t >> 6) * 2] = t1 - t0; clk[(t >> 6) * 2 + 1] = r1 - r0; }
}
"""
MFMA_LOAD_MIXES = {"mfma": (0, 0), "mfma_lds": (6, 0), "mfma_dma": (0, 2), "mfma_lds_dma": (6, 2)}


def mfma_clock_under_load(cp, be, iters=4096, reps=3):
    """TFLOP/s and the engine clock of the register-only float16 MFMA loop
    alone and with the large GEMM's LDS reads and global -> LDS copies
    issued beside it at the GEMM's bytes per flop (2048 workgroups of four
    waves; best of ``reps`` after one warm-up)."""
    nwg = 2048
    g = cp.array(np.random.default_rng(5).integers(0, 2 ** 16, (2 << 20) // 2, dtype=np.uint16)
                 & np.uint16(0xbfff))
    out = cp.zeros(nwg * 256, dtype=np.float32)
    clk = cp.zeros(nwg * 4 * 2, dtype=np.uint64)
    for x in (g, out, clk):
        x._ensure_gpu()
    res = {}
    for name, (reads, dmas) in MFMA_LOAD_MIXES.items():
        src = _MFMA_LOAD_SRC.replace("NAME", name).replace("READS", str(reads)).replace("DMAS", str(dmas))
        k = cp.RawKernel(src, name)
        args = lambda rep: (g, out, clk, np.int32(iters), np.uint32(2 + rep))  # noqa: E731
        k((nwg * 256,), args(-1))
        best = clock = None
        for rep in range(reps):
            s, e = be.event(), be.event()
            be.record(s)
            k((nwg * 256,), args(rep))
            be.record(e)
            cp.synchronize()
            ms = be.elapsed_ms(s, e)
            if best is None or ms < best:
                c = clk.get().reshape(-1, 2).astype(np.float64)
                best, clock = ms, float(np.mean(c[:, 0] / (c[:, 1] / 100.0)))
        flops = nwg * 4 * iters * 16 * 16384
        res[name] = {"ms": round(best, 3), "tflops": round(flops / best / 1e9, 1),
                     "clock_mhz": round(clock), "lds_read_bytes_per_kflop": round(reads * 1024 * 1000 / 262144, 2),
                     "dma_bytes_per_kflop": round(dmas * 1024 * 1000 / 262144, 2)}
    return res


def bench_c4(cp, be, reps=20, warm=10):
    from macmetalpy_amd.workloads import c4_inputs
    res = {}
    for kind, dt in (("f32", "float32"), ("f16", "float16"), ("batched", "float32")):
        try:
            a_np, b_np = c4_inputs(kind)
            a, b = cp.array(a_np), cp.array(b_np)
            a._ensure_gpu()
            b._ensure_gpu()
            flops = 2.0 * a_np.shape[-2] * a_np.shape[-1] * b_np.shape[-1] * (
                a_np.shape[0] if a_np.ndim == 3 else 1)
            del a_np, b_np
            f = lambda: a @ b  # noqa: E731
            # the matrix cores' clock settles over the first few ms of
            # sustained MFMA work: time steady state, mean of `reps` launches
            for _ in range(warm):
                f()
            cp.synchronize()
            timer = EventTimer(be)
            for _ in range(reps):
                timer.run(kind, f)
            cp.synchronize()
            ms, _ = timer.ms(kind)
            timer.close()
            tf = flops / ms / 1e9
            res[kind] = {"kernel_ms": round(ms, 4), "tflops": round(tf, 2),
                         "peak_tflops": PEAK_TFLOPS[dt],
                         "frac_of_peak": round(tf / PEAK_TFLOPS[dt], 4)}
            del a, b
        except Exception as e:
            res[kind] = {"error": f"{type(e).__name__}: {e}"[:300]}
    try:
        res["fp16_mfma_practical_ceiling"] = mfma_ceiling(cp, be)
    except Exception as e:
        res["fp16_mfma_practical_ceiling"] = {"error": f"{type(e).__name__}: {e}"[:300]}
    try:
        under = res["fp16_mfma_clock_under_gemm_traffic"] = mfma_clock_under_load(cp, be)
        if "tflops" in res.get("f16", {}):
            res["f16"]["frac_of_traffic_ceiling"] = round(
                res["f16"]["tflops"] / under["mfma_lds_dma"]["tflops"], 4)
    except Exception as e:
        res["fp16_mfma_clock_under_gemm_traffic"] = {"error": f"{type(e).__name__}: {e}"[:300]}
    return res


# ------------------------------- bitwise / logical / where / clip / any
def bench_logic(cp, be, reps=10):
    """Bitwise, predicate, where, clip and any/count_nonzero at 2^28 elements
    on the C2 inputs; bytes are each op's algorithmic HBM bytes (operands
    read once, result written once; bool results 1 B)."""
    from macmetalpy_amd.workloads import c2_float_inputs, c2_int_inputs
    a, b = (cp.array(x) for x in c2_float_inputs(N28))
    ia, ib = (cp.array(x) for x in c2_int_inputs(N28))
    for x in (a, b, ia, ib):
        x._ensure_gpu()
    cases = {
        "bitwise_and_i32": (lambda: _mat(ia & ib), 12),
        "right_shift_i32": (lambda: _mat(ia >> 3), 8),
        "isnan_f32": (lambda: _mat(cp.isnan(a)), 5),
        "where_f32": (lambda: _mat(cp.where(a > 0, a, b)), 12),
        "clip_f32": (lambda: _mat(cp.clip(a, -1.0, 1.0)), 8),
        "any_f32": (lambda: cp.any(a > 3.0), 4),
        "count_nonzero_f32": (lambda: cp.count_nonzero(a > 0, axis=0), 4),
    }
    res = {}
    for name, (f, bpe) in cases.items():
        try:
            f()
            cp.synchronize()
            ms = _launch_ms(cp, be, f, reps)
            res[name] = {"kernel_ms": round(ms, 4), "gbs": round(bpe * N28 / ms / 1e6, 1),
                         "frac_of_peak": round(bpe * N28 / ms / 1e6 / HBM_PEAK_GBS, 4)}
        except Exception as e:
            res[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
    return res


# ------------------------------------------------------ NaN reductions
def bench_nan(cp, be, reps=10):
    """NaN-skipping reductions on the C3 matrix (16384 x 16384 float32)
    with 1 % of the elements set to NaN; 4 B/elem read."""
    from macmetalpy_amd.workloads import c3_matrix
    m = c3_matrix()
    m.reshape(-1)[::97] = np.nan
    A = cp.array(m)
    del m
    A._ensure_gpu()
    nbytes = 4 * A.size
    cases = {
        "nansum_all": lambda: cp.nansum(A), "nanmean_axis1": lambda: cp.nanmean(A, axis=1),
        "nanmax_axis1": lambda: cp.nanmax(A, axis=1),
        "nanargmax_axis1": lambda: cp.nanargmax(A, axis=1),
    }
    res = {}
    for name, f in cases.items():
        try:
            f()
            cp.synchronize()
            ms = _launch_ms(cp, be, f, reps)
            res[name] = {"kernel_ms": round(ms, 4), "gbs": round(nbytes / ms / 1e6, 1),
                         "frac_of_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)}
        except Exception as e:
            res[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
    return res


# ------------------------------------------------------------- sorting
def bench_sort(cp, be, reps=5):
    """Radix sort / argsort of 2^24 and 2^28 float32 keys (N(0,1)) and
    searchsorted of 2^20 queries into 2^24 sorted keys.  `gkeys_s` is
    keys per second; `gbs` counts the HBM bytes of the four 8-bit LSD
    passes as designed: per pass the tile histogram reads the keys (4 B)
    and the scatter reads and writes them (8 B) -- 48 B/key for sort; for
    argsort the scatter also moves 4-byte indices (the first pass makes
    them) -- 16 + 3 x 20 = 76 B/key."""
    rng = np.random.default_rng(12)
    res = {}
    for log2n in (24, 28):
        n = 1 << log2n
        x = cp.array(rng.standard_normal(n, dtype=np.float32))
        x._ensure_gpu()
        cases = {f"sort_f32_2^{log2n}": (lambda: cp.sort(x), 48),
                 f"argsort_f32_2^{log2n}": (lambda: cp.argsort(x), 76)}
        for name, (f, bpe) in cases.items():
            try:
                f()
                cp.synchronize()
                timer = EventTimer(be)
                for _ in range(reps):
                    timer.run(name, f)
                cp.synchronize()
                ms, _ = timer.ms(name)
                timer.close()
                res[name] = {"kernel_ms": round(ms, 4), "gkeys_s": round(n / ms / 1e6, 2),
                             "gbs": round(bpe * n / ms / 1e6, 1)}
            except Exception as e:
                res[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
        if log2n == 24:
            a = cp.sort(x)
            q = cp.array(rng.standard_normal(1 << 20, dtype=np.float32))
            q._ensure_gpu()
            f = lambda: cp.searchsorted(a, q)  # noqa: E731
            f()
            cp.synchronize()
            timer = EventTimer(be)
            for _ in range(reps):
                timer.run("searchsorted", f)
            cp.synchronize()
            ms, _ = timer.ms("searchsorted")
            timer.close()
            res["searchsorted_2^20_in_2^24"] = {"kernel_ms": round(ms, 4),
                                                "gqueries_s": round((1 << 20) / ms / 1e6, 2)}
            del a, q
        del x
    # rows of at most one 4096-key tile: one workgroup sorts each row in LDS
    # (8 B/key of HBM traffic for sort: read once, written once)
    xr = cp.array(rng.standard_normal((65536, 1024), dtype=np.float32))
    xr._ensure_gpu()
    n = xr.size
    for name, f in (("sort_rows_f32_65536x1024", lambda: cp.sort(xr, axis=-1)),
                    ("argsort_rows_f32_65536x1024", lambda: cp.argsort(xr, axis=-1))):
        try:
            f()
            cp.synchronize()
            timer = EventTimer(be)
            for _ in range(reps):
                timer.run(name, f)
            cp.synchronize()
            ms, _ = timer.ms(name)
            timer.close()
            res[name] = {"kernel_ms": round(ms, 4), "gkeys_s": round(n / ms / 1e6, 2)}
        except Exception as e:
            res[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
    del xr
    return res


# ------------------------------------------------- indexing / manipulation
def _time(cp, be, name, f, reps):
    f()
    cp.synchronize()
    timer = EventTimer(be)
    for _ in range(reps):
        timer.run(name, f)
    cp.synchronize()
    ms, _ = timer.ms(name)
    timer.close()
    return ms


def bench_indexing(cp, be, reps=5):
    """Advanced indexing, manipulation and order statistics on 2^26-element
    float32 inputs.  `gbs` counts the bytes each operation must move:
    a[idx] (2^26 random int64 indices): 8 B index + 4 B read + 4 B write per
    element; a[a > 0] (about half selected): the mask pass (4 B read + 1 B
    written), its scan (1 B read + 8 B written), the positions (8 B read +
    8 B per selected element written) and the gather (8 + 4 + 4 B per
    selected element); concatenate of two 2^25 arrays: 8 B per element;
    tile 2^13 x 2^13 -> 2x: 4 B read once, 8 B written per source element.
    median / quantile of (8192, 8192) along axis 1 are timed per call (the
    radix sort of the rows dominates: 48 B per element as designed)."""
    rng = np.random.default_rng(13)
    n = 1 << 26
    x = cp.array(rng.standard_normal(n, dtype=np.float32))
    x._ensure_gpu()
    idx = cp.array(rng.integers(0, n, n))
    idx._ensure_gpu()
    res = {}
    cases = {
        "gather_a[idx]_2^26": (lambda: x[idx], 16 * n),
        # a > 0 (4 B read, 1 B written), tile counts (1 B), packing (1 B of
        # mask and 4 B of data read per element, 4 B written per selected one)
        "mask_a[a>0]_2^26": (lambda: x[x > 0], (5 + 1 + 5) * n + 4 * (n // 2)),
        "concatenate_2x2^25": (lambda: cp.concatenate([x[: n // 2], x[n // 2:]]), 8 * n),
        "tile_8192sq_2x2": (lambda: cp.tile(x.reshape(8192, 8192), (2, 2)), 4 * n + 16 * n),
        "transpose_copy_8192sq": (lambda: x.reshape(8192, 8192).T.copy(), 8 * n),
        "take_along_axis_8192sq": (None, 0),
    }
    m = x.reshape(8192, 8192)
    order = cp.argsort(m[:, :64], axis=1)
    order._ensure_gpu()
    cases["take_along_axis_8192sq"] = (lambda: cp.take_along_axis(m[:, :64], order, axis=1),
                                       (8 + 4 + 4) * 8192 * 64)
    for name, (f, nbytes) in cases.items():
        try:
            ms = _time(cp, be, name, f, reps)
            res[name] = {"kernel_ms": round(ms, 4), "gbs": round(nbytes / ms / 1e6, 1)}
        except Exception as e:
            res[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
    for name, f in (("median_axis1_8192sq", lambda: cp.median(m, axis=1)),
                    ("quantile_0.9_axis1_8192sq", lambda: cp.quantile(m, 0.9, axis=1)),
                    ("nanmedian_axis1_8192sq", lambda: cp.nanmedian(m, axis=1)),
                    ("unique_int32_2^24", lambda: cp.unique(ui))):
        try:
            if name.startswith("unique"):
                ui = cp.array(rng.integers(0, 1 << 20, 1 << 24).astype(np.int32))
                ui._ensure_gpu()
            ms = _time(cp, be, name, f, reps)
            res[name] = {"kernel_ms": round(ms, 4)}
        except Exception as e:
            res[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
    return res


# --------------------------------------------------------------- C5
# C5's per-element chain with its loads replaced by register values: the
# row-sum kernel the fusion engine generates for C5 (same mmp_ops.h
# functions, float64 accumulator, 4 elements per step, the same grid of
# 8192 workgroups x 256 threads and 32 elements per thread), but each next
# element is the previous one plus a constant instead of a load.  Its time
# is the VALU-bound time of C5's instruction mix; "long" runs 4 times the
# elements per thread on 2048 workgroups (8 per CU, resident at once: less
# prologue / epilogue weight) for the sustained element rate.
_C5_VALU_SRC = r"""
extern "C" __global__ __launch_bounds__(256) void c5_valu(double* out, int iters, float dx) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  float x[4], r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = -2.0f + (float)((t * 4 + e) & 4095) * (4.0f / 4096.0f);
    r[e] = 0.5f + 1.5f * (float)((t * 4 + e) & 255) * (1.0f / 256.0f);
  }
  const float s0 = 1.0f;
  double acc = 0;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float t0 = x[e];
      const float t1 = r[e];
      const float t2 = op_multiply(t0, t1);
      const float t4 = op_add(t2, s0);
      const float t5 = op_tanh(t4);
      const float t6 = op_abs(t0);
      const float t7 = op_neg(t6);
      const float t8 = op_exp_nonpos(t7);
      const float t9 = op_multiply(t5, t8);
      const float t10 = op_multiply(t0, t0);
      const float t11 = op_log1p_nonneg(t10);
      const float t12 = op_subtract(t9, t11);
      acc += (double)t12;
      x[e] = op_add(t0, dx);
    }
  }
  out[t] = acc;
}
"""


def c5_valu_ceiling(cp, be, reps=10):
    """ms of the VALU-only C5 loop at C5's grid (8192 x 256 threads, 8
    steps of 4 elements: 8192^2 elements) and Gelem/s of its long form."""
    from macmetalpy_amd import _fusion
    k = cp.RawKernel(_fusion._ops_header() + _C5_VALU_SRC, "c5_valu",
                     options="-ffp-contract=off -Xclang -target-feature -Xclang -packed-fp32-ops")
    out = cp.zeros(8192 * 256, dtype=np.float64)
    out._ensure_gpu()
    res = {}
    for name, nwg, iters in (("c5_grid", 8192, 8), ("long", 2048, 32)):
        k((nwg * 256,), (out, np.int32(iters), np.float32(1e-5)))
        cp.synchronize()
        timer = EventTimer(be)
        for _ in range(reps):
            timer.run(name, lambda: k((nwg * 256,), (out, np.int32(iters), np.float32(1e-5))))
        cp.synchronize()
        ms, _ = timer.ms(name)
        timer.close()
        elems = nwg * 256 * iters * 4
        res[name] = {"ms": round(ms, 4), "gelem_s": round(elems / ms / 1e6, 1)}
    return res


def bench_c5(cp, be, reps=10):
    from macmetalpy_amd.workloads import c5_inputs
    x_np, r_np = c5_inputs()
    x, r = cp.array(x_np), cp.array(r_np)
    x._ensure_gpu()
    r._ensure_gpu()
    nbytes = 4 * x.size + 4 * r.size + 4 * x.shape[0]

    def chain():
        return cp.sum(cp.tanh(x * r + 1.0) * cp.exp(-cp.abs(x)) - cp.log1p(x * x), axis=1)

    res = {}
    for mode in ("fused", "fused_fast_math", "unfused"):
        try:
            cp.set_config(fusion=(mode != "unfused"), fast_math=(mode == "fused_fast_math"))
            chain()
            cp.synchronize()
            t = time.perf_counter()
            ms = _launch_ms(cp, be, chain, reps)
            wall = (time.perf_counter() - t) / reps * 1e3
            res[mode] = {"ms": round(ms, 4), "wall_ms": round(wall, 4)}
        except Exception as e:
            res[mode] = {"error": f"{type(e).__name__}: {e}"[:300]}
        finally:
            cp.set_config(fusion=True, fast_math=False)
    if "ms" in res.get("fused_fast_math", {}):
        ms = res["fused_fast_math"]["ms"]
        res["fused_fast_math"].update({"gbs": round(nbytes / ms / 1e6, 1),
                                       "frac_of_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)})
    if "ms" in res.get("fused", {}):
        ms = res["fused"]["ms"]
        res["fused"].update({"gbs": round(nbytes / ms / 1e6, 1),
                             "frac_of_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)})
        if "ms" in res.get("unfused", {}):
            res["speedup_vs_unfused"] = round(res["unfused"]["ms"] / ms, 2)
        # the VALU roof: the same chain with no memory traffic, timed now
        try:
            v = c5_valu_ceiling(cp, be)
            v["c5_elements_gelem_s"] = round(x.size / ms / 1e6, 1)
            v["valu_roof_frac"] = round(v["c5_grid"]["ms"] / ms, 4)
            v["valu_roof_frac_sustained"] = round(x.size / ms / 1e6 / v["long"]["gelem_s"], 4)
            res["valu_roof"] = v
        except Exception as e:
            res["valu_roof"] = {"error": f"{type(e).__name__}: {e}"[:300]}
    return res


# ------------------------------------------------------- CPU baseline
def _median_time(fn, reps, warm):
    """Median wall time of ``fn`` over ``reps`` runs after ``warm`` warm-ups
    (the reference's method, benchmarks/bench_vs_numpy.py:30-45)."""
    times = []
    for i in range(warm + reps):
        t = time.perf_counter()
        fn()
        dt = time.perf_counter() - t
        if i >= warm:
            times.append(dt)
    return statistics.median(times)


def _host_info():
    info = {"nproc": os.cpu_count()}
    try:
        with open("/proc/cpuinfo") as f:
            info["cpu_model"] = next((l.split(":", 1)[1].strip() for l in f
                                      if l.startswith("model name")), "")
    except OSError:
        pass
    try:
        from threadpoolctl import threadpool_info
        info["blas"] = [{k: d.get(k) for k in ("internal_api", "version", "num_threads",
                                                 "threading_layer", "architecture")}
                        for d in threadpool_info() if d.get("user_api") == "blas"]
    except Exception as e:  # report, keep going
        info["blas"] = f"unavailable: {type(e).__name__}"
    info["OPENBLAS_NUM_THREADS"] = os.environ.get("OPENBLAS_NUM_THREADS", "unset (all cores)")
    info["numpy"] = np.__version__
    return info


def _cpu_entry(value, unit, cores, sample, extra=None):
    d = {"value": round(value, 3), "unit": unit, "cores": cores, "kind": "port",
         "sample": sample}
    if extra:
        d.update(extra)
    return d


def cpu_baseline(sample_log2=25, reps=10, warm=2):
    """The reference's CPU path -- NumPy, the oracle's restatement
    (oracle/reference_cpu.py) -- timed on this host: the headline C2 step on
    the first 2^sample_log2 elements of the 2^28 inputs, and one bounded
    sample of every other configuration (``per_config``).  NumPy ufuncs
    are single-threaded; np.matmul uses all host cores through BLAS."""
    from macmetalpy_amd import workloads as W
    from oracle import reference_cpu as ref
    n = 1 << sample_log2
    a, b = W.c2_float_inputs(N28)
    a, b = a[:n].copy(), b[:n].copy()
    ai, bi = W.c2_int_inputs(N28)
    ai, bi = ai[:n].copy(), bi[:n].copy()
    ops = [(lambda: ref.binary("add_op", a, b), 12), (lambda: ref.unary("sin_op", a), 8),
           (lambda: ref.floor_divide(ai, bi), 12), (lambda: ref.mod(ai, bi), 12)]
    total_bytes = sum(bpe for _, bpe in ops) * n
    med = _median_time(lambda: [fn() for fn, _ in ops], reps, warm)
    out = _cpu_entry(total_bytes / med / 1e9, "GB/s", 1,
                     f"a+b, sin(a) float32 and floor_divide, mod int32 on the first 2^{sample_log2} "
                     f"elements of the 2^28 inputs; NumPy {np.__version__} single-threaded "
                     f"ufuncs; median of {reps} after {warm} warm-ups ({med:.3f} s/step)")
    del a, b, ai, bi
    per = {}
    # C1 at its full size, 2^20
    x = W.c1_inputs(1 << 20)
    t = _median_time(lambda: ref.fused_elementwise(x), reps, warm)
    per["c1_fused_elementwise_2^20"] = _cpu_entry(
        8 * x.size / t / 1e9, "GB/s", 1, "full 2^20 config, op by op in float32",
        {"call_us": round(t * 1e6, 1)})
    # C2 per op (same sample as the headline)
    per["c2_binary"] = {k: v for k, v in out.items()}
    # C3: reductions on the first 4096 rows of the 16384^2 matrix, scans on 2^25
    A = W.c3_matrix(4096, 16384)
    nb = A.nbytes
    c3 = {}
    for name, fn in (("sum_all", lambda: ref.sum(A)), ("mean_all", lambda: ref.mean(A)),
                     ("sum_axis1", lambda: ref.sum(A, axis=1)),
                     ("mean_axis1", lambda: ref.mean(A, axis=1)),
                     ("argmax_all", lambda: ref.argmax(A)),
                     ("argmax_axis1", lambda: ref.argmax(A, axis=1))):
        t = _median_time(fn, reps, warm)
        c3[name] = _cpu_entry(nb / t / 1e9, "GB/s", 1, "4096 x 16384 float32 (first quarter of "
                              "the 16384^2 config)", {"ms": round(t * 1e3, 2)})
    del A
    ci, cf = W.c3_scan_inputs(1 << 25)
    for name, arr, bpe in (("cumsum_i32_to_i64", ci, 12), ("cumsum_f32", cf, 8)):
        t = _median_time(lambda arr=arr: ref.cumsum(arr), reps, warm)
        c3[name] = _cpu_entry(bpe * arr.size / t / 1e9, "GB/s", 1,
                              "2^25 elements (1/8 of the 2^28 config)", {"ms": round(t * 1e3, 2)})
    # NumPy's float32 cumsum accumulates in float32: its error against the
    # float64-accumulated prefix sums, under the 1e-5 relative bar the
    # device scan is held to
    exact = np.cumsum(cf, dtype=np.float64)
    rel = float(np.max(np.abs(ref.cumsum(cf).astype(np.float64) - exact) / np.maximum(exact, 1e-30)))
    c3["cumsum_f32"].update({"max_rel_err_vs_f64": rel, "within_1e-5": rel <= 1e-5})
    per["c3_reduce_scan"] = c3
    del ci, cf
    # C4: BLAS float32 at full size (all host cores), float16 scaled down
    c4 = {}
    for kind, label in (("f32", "4096^3 float32"), ("batched", "64 x 1024^3 float32")):
        p, q = W.c4_inputs(kind)
        flops = 2.0 * p.shape[-2] * p.shape[-1] * q.shape[-1] * (p.shape[0] if p.ndim == 3 else 1)
        t = _median_time(lambda p=p, q=q: ref.matmul(p, q), 3, 1)
        c4[kind] = _cpu_entry(flops / t / 1e9, "GFLOP/s", os.cpu_count(),
                              f"full {label}, np.matmul (BLAS, all host cores); median of 3 after 1",
                              {"ms": round(t * 1e3, 1)})
        del p, q
    p, q = W.c4_inputs("f16", 2048)
    t = _median_time(lambda: ref.matmul(p, q), 1, 0)
    c4["f16"] = _cpu_entry(2.0 * 2048 ** 3 / t / 1e9, "GFLOP/s", 1,
                           "scaled: 2048^3 float16 (NumPy's non-BLAS float16 loop; at this rate "
                           f"the 8192^3 config would take ~{t * 64 / 60:.0f} min); one run",
                           {"ms": round(t * 1e3, 1)})
    per["c4_matmul"] = c4
    # C5 on the first 2048 rows
    xx, rr = W.c5_inputs(2048, 8192)
    t = _median_time(lambda: ref.fusion_chain(xx, rr), reps, warm)
    per["c5_fusion_chain"] = _cpu_entry(
        (xx.nbytes + rr.nbytes + 4 * xx.shape[0]) / t / 1e9, "GB/s", 1,
        "2048 x 8192 rows of the 8192^2 config, op by op in float32",
        {"ms": round(t * 1e3, 2)})
    per["small_host_ops"] = _small_host_cpu()
    out["per_config"] = per
    out["host"] = _host_info()
    return out


def _env(be):
    info = {}
    try:
        info.update(be.device_info())
    except Exception:
        pass
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
        info["host_cpu"] = model
    except OSError:
        pass
    info["host_nproc"] = os.cpu_count()
    info["numpy"] = np.__version__
    info["python"] = platform.python_version()
    return info


ONLY_OPS = ("add_f32", "sin_f32", "floor_divide_i32", "mod_i32", "copy_f32", "cumsum_i32",
            "cumsum_f32", "matmul_f16", "sort_f32", "c5_fused", "sum_all", "sum_axis1",
            "argmax_all", "argmax_axis1", "sum_axis0", "argmax_axis0", "c1_2p20",
            "c1_2p28", "matmul_f32", "matmul_batched", "mfma_ceiling")


def run_only(cp, be, name, steps):
    """One op of a benchmark workload, `steps` launches (for counter
    profiling); copy_f32 is a plain strided-copy kernel of 2^28 floats
    (1 GiB read + 1 GiB written) used to calibrate the byte counters."""
    from macmetalpy_amd.workloads import (c1_inputs, c2_float_inputs, c2_int_inputs, c3_matrix,
                                          c3_scan_inputs, c4_inputs, c5_inputs)
    if name == "mfma_ceiling":
        print(json.dumps({"only": name, **mfma_ceiling(cp, be)}), flush=True)
        return
    if name in ("add_f32", "sin_f32", "copy_f32"):
        a, b = (cp.array(x) for x in c2_float_inputs(N28))
    elif name in ("floor_divide_i32", "mod_i32"):
        a, b = (cp.array(x) for x in c2_int_inputs(N28))
    elif name in ("cumsum_i32", "cumsum_f32"):
        ci, cf = c3_scan_inputs()
        a = b = cp.array(ci if name == "cumsum_i32" else cf)
        del ci, cf
    elif name == "sort_f32":
        a = b = cp.array(np.random.default_rng(12).standard_normal(N28, dtype=np.float32))
    elif name == "c5_fused":
        a, b = (cp.array(x) for x in c5_inputs())
    elif name in ("sum_all", "sum_axis1", "argmax_all", "argmax_axis1", "sum_axis0",
                  "argmax_axis0"):
        a = b = cp.array(c3_matrix())
    elif name in ("c1_2p20", "c1_2p28"):
        a = b = cp.array(c1_inputs(1 << 20 if name == "c1_2p20" else N28))
    elif name == "matmul_f32":
        a, b = (cp.array(x) for x in c4_inputs("f32"))
    elif name == "matmul_batched":
        a, b = (cp.array(x) for x in c4_inputs("batched"))
    else:  # matmul_f16
        a, b = (cp.array(x) for x in c4_inputs("f16"))
    a._ensure_gpu()
    b._ensure_gpu()
    fn = {"add_f32": lambda: a + b, "sin_f32": lambda: cp.sin(a),
          "floor_divide_i32": lambda: cp.floor_divide(a, b), "mod_i32": lambda: cp.mod(a, b),
          "copy_f32": lambda: a.copy(), "cumsum_i32": lambda: cp.cumsum(a),
          "cumsum_f32": lambda: cp.cumsum(a), "matmul_f16": lambda: a @ b,
          "matmul_f32": lambda: a @ b, "matmul_batched": lambda: a @ b,
          "sort_f32": lambda: cp.sort(a),
          "c5_fused": lambda: cp.sum(cp.tanh(a * b + 1.0) * cp.exp(-cp.abs(a))
                                     - cp.log1p(a * a), axis=1),
          "sum_all": lambda: cp.sum(a), "sum_axis1": lambda: cp.sum(a, axis=1),
          "argmax_all": lambda: cp.argmax(a, axis=None, keepdims=True),
          "argmax_axis1": lambda: cp.argmax(a, axis=1),
          "sum_axis0": lambda: cp.sum(a, axis=0), "argmax_axis0": lambda: cp.argmax(a, axis=0),
          "c1_2p20": lambda: cp.sqrt(cp.abs(a)) + cp.exp(-a ** 2),
          "c1_2p28": lambda: cp.sqrt(cp.abs(a)) + cp.exp(-a ** 2)}[name]
    timer = EventTimer(be)
    for _ in range(steps):
        timer.run(name, lambda: _mat(fn()))
    cp.synchronize()
    ms, _ = timer.ms(name)
    timer.close()
    print(json.dumps({"only": name, "steps": steps, "kernel_ms": round(ms, 4)}), flush=True)


def bench_linalg(cp, be, reps=3):
    """Dense factorizations (one workgroup per matrix): GFLOP/s counts the
    textbook flops -- LU 2/3 n^3 plus 2 n^2 per right-hand side for solve,
    Cholesky 1/3 n^3, Householder QR 2 m n^2 - 2/3 n^3; the Jacobi methods
    (eigh, SVD) are timed per call.  Batched shapes fill the chip; a single
    large matrix runs on one CU (a blocked multi-workgroup factorization is
    the next step for it)."""
    rng = np.random.default_rng(21)
    LA = cp.linalg

    def mat(shape, dt, spd=False):
        a = rng.standard_normal(shape)
        a = a + np.eye(shape[-1]) * shape[-1] * 0.5
        if spd:
            a = a @ np.swapaxes(a, -1, -2)
        d = cp.array(a.astype(dt))
        d._ensure_gpu()
        return d

    res = {}
    a1k, b1k = mat((1024, 1024), np.float64), cp.array(rng.standard_normal((1024, 1)))
    ab, bb = mat((4096, 64, 64), np.float32), cp.array(rng.standard_normal((4096, 64, 1)).astype(np.float32))
    s1k, sb = mat((1024, 1024), np.float64, spd=True), mat((4096, 32, 32), np.float32, spd=True)
    q = cp.array(rng.standard_normal((1024, 256)))
    e = mat((256, 256), np.float64)
    e = (e + e.T) * 0.5
    eb = cp.array(np.swapaxes(rng.standard_normal((1024, 32, 32)), 1, 2).astype(np.float32))
    eb = (eb + eb.swapaxes(1, 2)) * 0.5
    sv = cp.array(rng.standard_normal((512, 256)))
    cases = {
        "solve_f64_1024": (lambda: LA.solve(a1k, b1k), 2 / 3 * 1024 ** 3 + 2 * 1024 ** 2),
        "solve_f32_4096x64": (lambda: LA.solve(ab, bb), 4096 * (2 / 3 * 64 ** 3 + 2 * 64 ** 2)),
        "inv_f64_1024": (lambda: LA.inv(a1k), 2 / 3 * 1024 ** 3 + 2 * 1024 ** 3),
        "cholesky_f64_1024": (lambda: LA.cholesky(s1k), 1024 ** 3 / 3),
        "cholesky_f32_4096x32": (lambda: LA.cholesky(sb), 4096 * 32 ** 3 / 3),
        "qr_f64_1024x256": (lambda: LA.qr(q), 2 * 1024 * 256 ** 2 - 2 / 3 * 256 ** 3),
        "eigh_f64_256": (lambda: LA.eigh(e), None),
        "eigh_f32_1024x32": (lambda: LA.eigvalsh(eb), None),
        "svd_f64_512x256": (lambda: LA.svd(sv, full_matrices=False), None),
    }
    for name, (f, flops) in cases.items():
        try:
            ms = _time(cp, be, name, f, reps)
            res[name] = {"ms": round(ms, 3)}
            if flops:
                res[name]["gflops"] = round(flops / ms / 1e6, 1)
        except Exception as ex:
            res[name] = {"error": f"{type(ex).__name__}: {ex}"[:300]}
    return res


def bench_routines(cp, be, reps=5):
    """Routines composed of device ops at 2^24-2^26 elements; `gbs` counts
    the bytes of the inputs read and the result written once."""
    rng = np.random.default_rng(22)
    n = 1 << 24
    x = cp.array(rng.standard_normal(n).astype(np.float32))
    x._ensure_gpu()
    t = cp.array(rng.standard_normal(1 << 20).astype(np.float32))
    ints = cp.array(rng.integers(0, 1000, n).astype(np.int32))
    m = x.reshape(4096, 4096)
    xp = cp.array(np.sort(rng.standard_normal(4096)))
    fp = cp.array(rng.standard_normal(4096))
    x64 = x.astype(np.float64)
    cases = {
        "isclose_f32_2^24": (lambda: cp.isclose(x, x * 1.0000001), 9 * n),
        "isin_2^24_in_2^20": (lambda: cp.isin(x, t), 5 * n),
        "histogram_100_2^24": (lambda: cp.histogram(x, bins=100), 4 * n),
        "bincount_int32_2^24": (lambda: cp.bincount(ints), 4 * n),
        "interp_f64_2^24": (lambda: cp.interp(x64, xp, fp), 16 * n),
        "pad_reflect_4096sq_+64": (lambda: cp.pad(m, 64, mode="reflect"), 4 * n + 4 * 4224 ** 2),
        "einsum_bij,bjk_256x128": (lambda: cp.einsum("bij,bjk->bik", m.reshape(256, 128, 512),
                                                      m.reshape(256, 512, 128)), None),
        "cov_64x2^18": (lambda: cp.cov(x.reshape(64, 1 << 18)), None),
    }
    res = {}
    for name, (f, nbytes) in cases.items():
        try:
            ms = _time(cp, be, name, f, reps)
            res[name] = {"kernel_ms": round(ms, 4)}
            if nbytes:
                res[name]["gbs"] = round(nbytes / ms / 1e6, 1)
        except Exception as ex:
            res[name] = {"error": f"{type(ex).__name__}: {ex}"[:300]}
    return res


CONFIG_SECTIONS = {
    "c2_end_to_end": bench_c2_end_to_end,
    "vendor_copy_2p28": vendor_copy,
    "scaling_vs_numpy": bench_scaling_vs_numpy,
    "c1_fused_elementwise": bench_c1, "small_ops_2p20": bench_small_ops,
    "small_host_ops": bench_small_host_ops,
    "scan_shape_copy_2p28": scan_shape_copy,
    "mfma_clock_under_load": mfma_clock_under_load,
    "c3_reduce_scan": bench_c3, "c4_matmul": bench_c4,
    "c5_fusion_chain": bench_c5, "logic_where_clip_2p28": bench_logic,
    "nan_reductions_16384sq": bench_nan, "sort_searchsorted": bench_sort,
    "indexing_manipulation": bench_indexing, "linalg": bench_linalg,
    "routines": bench_routines, "vendor_torch": vendor_torch,
}


def _vendor_ratios(out, cfgs):
    """Beside each C2 op and C4 product, the same run's vendor rate and
    this library's rate over it (vendor_torch: torch / hipBLASLt)."""
    v = cfgs.get("vendor_torch")
    if not isinstance(v, dict) or "gemm" not in v:
        return
    for op, name in (("add_f32", "add"), ("sin_f32", "sin")):
        t = v["elementwise_2p28"].get(name)
        if t and op in out.get("per_op", {}):
            d = out["per_op"][op]
            d["torch_gbs"] = t["gbs"]
            d["vs_torch"] = round(d["gbs"] / t["gbs"], 3)
    c4 = cfgs.get("c4_matmul", {})
    for kind, t in v["gemm"].items():
        if isinstance(c4.get(kind), dict) and "tflops" in c4[kind]:
            c4[kind]["hipblaslt_tflops"] = t["tflops"]
            c4[kind]["vs_hipblaslt"] = round(c4[kind]["tflops"] / t["tflops"], 3)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--suite", choices=["all", "headline"], default="all")
    ap.add_argument("--cpu-sample-log2", type=int, default=25)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=ONLY_OPS, default=None,
                    help="run one headline op `--steps` times and exit (profiling)")
    ap.add_argument("--config", choices=sorted(CONFIG_SECTIONS), default=None,
                    help="run one configuration section, print its JSON and exit (profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the library has no multi-GPU path "
              f"(--gpus {args.gpus} requested).", file=sys.stderr)
        sys.exit(2)

    import macmetalpy_amd as cp
    from macmetalpy_amd._backend import HipBackend
    be = HipBackend()
    if args.only:
        run_only(cp, be, args.only, args.steps)
        return
    if args.config:
        print(json.dumps({args.config: CONFIG_SECTIONS[args.config](cp, be)}), flush=True)
        return

    c2 = bench_c2(cp, be, args.steps, args.warmup)
    per_op = c2["per_op"]
    # a+b: the longest of the four launches (12 B per element), event-timed
    # inside the timed steps
    dominant = "add_f32"
    dom = per_op[dominant]
    value = c2["bytes_per_step"] * args.steps / c2["wall_s"] / 1e9
    kernel_names = {"add_f32": "k_binary<MMP_B_ADD,float>", "sin_f32": "k_unary<MMP_U_SIN,float>",
                    "floor_divide_i32": "k_binary<MMP_B_FLOOR_DIVIDE,int>",
                    "mod_i32": "k_binary<MMP_B_MOD,int>"}
    traffic_table = _traffic_table()
    traffic = traffic_table.get(f"{dominant}@2^28")
    out = {
        "metric": "achieved HBM GB/s (fused elementwise/reduce/cumsum) + matmul TFLOPS, 1xMI355X",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(c2["wall_s"] / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32+i32",
        "data": "synthetic (seeded NumPy default_rng inputs, as cp.random.seed + randn/randint)",
        "config": {"workload": "binary elementwise 2^28: a+b, sin(a) float32 N(0,1); "
                               "floor_divide(a,b), mod(a,b) int32 a~U[-2^30,2^30), "
                               "b~+-U[1,1000]",
                   "elements": N28, "bytes_per_step": c2["bytes_per_step"]},
        "roofline": {"bound": "hbm", "kernel": kernel_names[dominant], "op": dominant,
                     "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_table.get("_source"),
                     "algorithmic_bytes_per_launch": dom["bytes"],
                     "avg_launch_ms": dom["kernel_ms"]},
        "per_op": per_op,
    }
    if args.suite == "all":
        cfgs = {}
        for name, fn in CONFIG_SECTIONS.items():
            t = time.time()
            try:
                cfgs[name] = fn(cp, be)
            except Exception as e:
                cfgs[name] = {"error": f"{type(e).__name__}: {e}"[:300]}
            _log(f"{name} done in {time.time() - t:.1f}s")
        out["configs"] = cfgs
        _vendor_ratios(out, cfgs)
    if not args.no_cpu:
        t = time.time()
        out["cpu_baseline"] = cpu_baseline(args.cpu_sample_log2)
        _log(f"cpu baseline done in {time.time() - t:.1f}s")
        # the CPU path's time of each small host call beside the device's
        small = out.get("configs", {}).get("small_host_ops", {})
        cpu_small = out["cpu_baseline"]["per_config"]["small_host_ops"]
        for label, sec in small.items() if isinstance(small, dict) else ():
            for name, d in sec.items() if isinstance(sec, dict) else ():
                if name in cpu_small.get(label, {}):
                    d["cpu_path_us"] = cpu_small[label][name]["call_us"]
    out["env"] = _env(be)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
