"""mmp_reduce_noalloc against mmp_reduce, through the C ABI.

The allocation-free variant keeps its cross-workgroup partials in a static
device array; it must give mmp_reduce's results (bit for bit where it
splits the same way, within the float32 reduction tolerance of 1e-5
relative where it lowers a strided split to fit) on two calls in a row,
the second smaller, and must leave the allocator untouched.  Captured into
a HIP graph on the library stream (mmp_stream), it must give the eager
call's results on every replay.
"""
import ctypes
import os

import numpy as np
import pytest

from macmetalpy_amd import _abi
from macmetalpy_amd._backend import HipBackend, load_library

pytestmark = pytest.mark.gpu

F32, F64, I32, I64 = (_abi.DTYPE_CODES[np.dtype(t)] for t in
                      (np.float32, np.float64, np.int32, np.int64))


def _dev(be, arr):
    return be.array_to_buffer(np.ascontiguousarray(arr))


def _both(be, lib, op, x, out_dt, outer, length, inner):
    """Run both entry points on the same device input; return host results
    and the allocator's (in_use, cached) around the no-alloc call."""
    buf = _dev(be, x)
    dc = _abi.DTYPE_CODES[x.dtype]
    oc = _abi.DTYPE_CODES[np.dtype(out_dt)]
    n_out = outer * inner
    o1 = be.create_buffer(n_out, out_dt)
    o2 = be.create_buffer(n_out, out_dt)
    assert lib.mmp_reduce(op, dc, oc, outer, length, inner, buf.ptr, o1.ptr) == 0
    be.synchronize()
    stats0 = be.memory_stats()
    st = lib.mmp_reduce_noalloc(op, dc, oc, outer, length, inner, buf.ptr, o2.ptr)
    assert st == 0, lib.mmp_last_error().decode()
    be.synchronize()
    stats1 = be.memory_stats()
    r1 = be.read_buffer(o1, 0, np.empty(n_out, out_dt))
    r2 = be.read_buffer(o2, 0, np.empty(n_out, out_dt))
    return r1, r2, stats0, stats1


CASES = [
    # (op, dtype, out dtype, (outer, len, inner) first, then smaller)
    (_abi.REDUCE_SUM, np.float32, np.float32, (3, 1 << 20, 1), (2, 1 << 18, 1)),
    (_abi.REDUCE_MEAN, np.float32, np.float32, (1, 1 << 22, 1), (1, 100003, 1)),
    (_abi.REDUCE_MAX, np.float32, np.float32, (5, 1 << 19, 1), (1, 1 << 17, 1)),
    (_abi.REDUCE_SUM, np.int32, np.int64, (2, 1 << 21, 1), (1, 70001, 1)),
    (_abi.REDUCE_NANMEAN, np.float64, np.float64, (1, 1 << 20, 1), (3, 1 << 16, 1)),
    (_abi.REDUCE_SUM, np.float32, np.float32, (1, 4096, 300), (2, 1024, 100)),
    (_abi.REDUCE_SUM, np.int32, np.int64, (1, 8192, 257), (1, 1000, 33)),
]


@pytest.mark.parametrize("op,dt,odt,first,second", CASES)
def test_noalloc_matches_reduce_twice(op, dt, odt, first, second):
    be = HipBackend()
    lib = load_library()
    rng = np.random.default_rng(90 + op)
    for shape in (first, second):
        outer, length, inner = shape
        if np.dtype(dt).kind == "f":
            x = rng.standard_normal(outer * length * inner).astype(dt)
            if op == _abi.REDUCE_NANMEAN:
                x[::97] = np.nan
        else:
            x = rng.integers(-1000, 1000, outer * length * inner).astype(dt)
        r1, r2, s0, s1 = _both(be, lib, op, x, odt, outer, length, inner)
        assert s0 == s1, (s0, s1)  # nothing allocated or freed
        assert r1.tobytes() == r2.tobytes(), (shape, r1[:4], r2[:4])


def test_noalloc_lowered_strided_split_within_tolerance():
    """Column sums along axis 0.  (65536, 2047) takes the column-per-thread
    kernel (2047 is not a multiple of 4): 8 column blocks x 128 splits x 256
    columns x 16 bytes of tagged slots is 4 MiB, more than the static
    scratch's 4 MiB - 16 KiB of partials, so the no-alloc variant lowers the
    split count to 127 (float64 partials either way): float32 results
    within 1e-5 relative of the float64 sums, integer sums bit-exact.
    (65536, 2048) takes the column-vector kernel (32 splits, 1 MiB: not
    lowered); then a smaller input."""
    be = HipBackend()
    lib = load_library()
    rng = np.random.default_rng(95)
    for rows, cols in ((65536, 2047), (65536, 2048), (8192, 512)):
        xf = rng.standard_normal((rows, cols)).astype(np.float32)
        r1, r2, s0, s1 = _both(be, lib, _abi.REDUCE_SUM, xf, np.float32, 1, rows, cols)
        assert s0 == s1
        want = xf.astype(np.float64).sum(axis=0)
        scale = np.abs(xf).astype(np.float64).sum(axis=0)
        assert np.all(np.abs(r2 - want) <= 1e-5 * scale)
        assert np.all(np.abs(r1 - want) <= 1e-5 * scale)
        xi = rng.integers(-50, 50, (rows, cols)).astype(np.int32)
        q1, q2, _, _ = _both(be, lib, _abi.REDUCE_SUM, xi, np.int64, 1, rows, cols)
        assert np.array_equal(q1, q2) and np.array_equal(q2, xi.sum(axis=0, dtype=np.int64))


def test_noalloc_lowered_split_nanmean():
    """nanmean along axis 0 of (65536, 3) float32: one column block, 1024
    splits of (sum, count) pairs (32 bytes of tagged slots per column) need
    8 MiB, so the no-alloc variant lowers the split count to 510; results
    within 1e-5 relative of the float64 NaN-skipping means."""
    be = HipBackend()
    lib = load_library()
    rng = np.random.default_rng(96)
    for rows, cols in ((65536, 3), (4096, 5)):
        x = rng.standard_normal((rows, cols)).astype(np.float32)
        x[::89, :] = np.nan
        r1, r2, s0, s1 = _both(be, lib, _abi.REDUCE_NANMEAN, x, np.float32, 1, rows, cols)
        assert s0 == s1
        want = np.nanmean(x.astype(np.float64), axis=0)
        scale = np.nanmean(np.abs(x).astype(np.float64), axis=0)
        assert np.all(np.abs(r2 - want) <= 1e-5 * scale), (r2, want)
        assert np.all(np.abs(r1 - want) <= 1e-5 * scale)


def test_noalloc_rejects_bad_arguments():
    be = HipBackend()
    lib = load_library()
    x = be.create_buffer(16, np.float32)
    o = be.create_buffer(1, np.float32)
    assert lib.mmp_reduce_noalloc(_abi.REDUCE_SUM, F32, F32, 1, 0, 1, x.ptr, o.ptr) == _abi.MMP_E_ARG
    assert lib.mmp_reduce_noalloc(99, F32, F32, 1, 16, 1, x.ptr, o.ptr) == _abi.MMP_E_ARG
    assert lib.mmp_reduce_noalloc(_abi.REDUCE_SUM, F32, F32, 1, 16, 1, None, o.ptr) == _abi.MMP_E_ARG


def _hip_runtime():
    """The HIP runtime's graph-capture entry points through ctypes (the
    process already has the library loaded through libmmp_hip.so)."""
    path = "/opt/rocm/lib/libamdhip64.so"
    hip = ctypes.CDLL(path if os.path.exists(path) else "libamdhip64.so")
    vp = ctypes.c_void_p
    sigs = {
        "hipStreamBeginCapture": [vp, ctypes.c_int],
        "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
        "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, ctypes.c_char_p, ctypes.c_size_t],
        "hipGraphLaunch": [vp, vp],
        "hipGraphExecDestroy": [vp],
        "hipGraphDestroy": [vp],
    }
    for name, argtypes in sigs.items():
        fn = getattr(hip, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    return hip


HIP_STREAM_CAPTURE_MODE_RELAXED = 2

GRAPH_CASES = [
    # (op, dtype, out dtype, (outer, len, inner)): split rows, then column partials
    (_abi.REDUCE_SUM, np.float32, np.float32, (1, 1 << 22, 1)),
    (_abi.REDUCE_SUM, np.int32, np.int64, (2, 1 << 20, 1)),
    (_abi.REDUCE_MEAN, np.float32, np.float32, (1, 4096, 300)),
]


@pytest.mark.parametrize("op,dt,odt,shape", GRAPH_CASES)
def test_noalloc_graph_replays_match_eager(op, dt, odt, shape):
    """mmp_reduce_noalloc captured into a HIP graph on the library stream
    and replayed four times.  Before each replay the input gets new values
    and another no-alloc reduction (another tag, the same scratch words)
    runs eagerly.  Every replay must give, bit for bit, what an eager
    mmp_reduce_noalloc call on the same input gives afterwards, and the
    float64 / exact reference of that input."""
    be = HipBackend()
    lib = load_library()
    hip = _hip_runtime()
    rng = np.random.default_rng(97 + op)
    outer, length, inner = shape
    n, n_out = outer * length * inner, outer * inner
    dc, oc = _abi.DTYPE_CODES[np.dtype(dt)], _abi.DTYPE_CODES[np.dtype(odt)]

    def draw():
        if np.dtype(dt).kind == "f":
            return rng.standard_normal(n).astype(dt)
        return rng.integers(-1000, 1000, n).astype(dt)

    x = be.create_buffer(n, dt)
    out_graph = be.create_buffer(n_out, odt)
    out_eager = be.create_buffer(n_out, odt)
    other_x = _dev(be, rng.standard_normal(1 << 20).astype(np.float32))
    other_out = be.create_buffer(1, np.float32)
    be.write_buffer(x, 0, draw())
    be.synchronize()

    stream = ctypes.c_void_p()
    assert lib.mmp_stream(ctypes.byref(stream)) == 0 and stream.value
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipStreamBeginCapture(stream, HIP_STREAM_CAPTURE_MODE_RELAXED) == 0
    try:
        st = lib.mmp_reduce_noalloc(op, dc, oc, outer, length, inner, x.ptr, out_graph.ptr)
    finally:
        end = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
    assert st == 0, lib.mmp_last_error().decode()
    assert end == 0 and graph.value
    try:
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        for rep in range(4):
            data = draw()
            be.write_buffer(x, 0, data)
            assert lib.mmp_reduce_noalloc(_abi.REDUCE_MAX, F32, F32, 1, 1 << 20, 1,
                                          other_x.ptr, other_out.ptr) == 0
            assert hip.hipGraphLaunch(exe, stream) == 0
            be.synchronize()
            got = be.read_buffer(out_graph, 0, np.empty(n_out, odt))
            assert lib.mmp_reduce_noalloc(op, dc, oc, outer, length, inner, x.ptr,
                                          out_eager.ptr) == 0
            be.synchronize()
            want = be.read_buffer(out_eager, 0, np.empty(n_out, odt))
            assert got.tobytes() == want.tobytes(), (rep, got[:4], want[:4])
            v = data.reshape(outer, length, inner)
            if np.dtype(dt).kind == "f":
                ref = v.astype(np.float64).sum(axis=1).reshape(-1)
                if op == _abi.REDUCE_MEAN:
                    ref /= length
                scale = np.abs(v).astype(np.float64).sum(axis=1).reshape(-1) / (
                    length if op == _abi.REDUCE_MEAN else 1)
                assert np.all(np.abs(got - ref) <= 1e-5 * scale), rep
            else:
                assert np.array_equal(got, v.sum(axis=1, dtype=np.int64).reshape(-1)), rep
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
