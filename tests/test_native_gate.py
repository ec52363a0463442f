"""The native dispatch gate on the CPU, against the Python path.

The gate (macmetalpy_amd/csrc/native_gate.cpp) is bound to a host-only stub
of the five library entry points it calls (tests/native_stub/stub_mmp.c,
built here with gcc); the stub records calls and copies the parameter
block of each generated-kernel launch.  Checked: the gate builds the same
lazy DAGs and result dtypes as the Python path, hands back what it does not
handle, calls the precompiled kernels with the right codes and pointers,
and packs exactly the parameter block the Python path packs (_fill_params)
for the same program -- what the generated kernel reads on the device.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd import _abi, _backend, _elementwise as ew, _fusion, _gate
from macmetalpy_amd.ndarray import ndarray

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def stub(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("stub") / "libstub_mmp.so")
    subprocess.run(["gcc", "-O1", "-shared", "-fPIC", "-std=c11",
                    os.path.join(HERE, "native_stub", "stub_mmp.c"), "-o", out], check=True)
    lib = ctypes.CDLL(out)
    lib.stub_call.restype = ctypes.c_int64
    lib.stub_params.restype = ctypes.c_void_p
    lib.stub_live.restype = ctypes.c_longlong
    lib.mmp_last_error.restype = ctypes.c_char_p
    # the library's own ctypes signatures, for the entry points the stub has
    for name in ("mmp_rtc_compile", "mmp_alloc", "mmp_free", "mmp_h2d", "mmp_d2h",
                 "mmp_rtc_launch", "mmp_reduce", "mmp_argreduce", "mmp_unary", "mmp_binary",
                 "mmp_binary_scalar"):
        getattr(lib, name).argtypes = _backend._SIGNATURES[name]
        getattr(lib, name).restype = ctypes.c_int
    saved = (_backend.HipBackend._instance, _backend._lib)
    _gate.unbind_library()
    inst = object.__new__(_backend.HipBackend)
    inst._lib = lib
    inst._exec_cache = {}
    _backend.HipBackend._instance = inst
    _backend._lib = lib
    _gate.bind_library(lib)
    # generated-kernel compiles only produce a handle (nothing runs)
    saved_compile = _backend.HipBackend.compile
    _backend.HipBackend.compile = lambda self, src, name, opts="": 0x4000
    yield lib
    _backend.HipBackend.compile = saved_compile
    # forget the stand-in's handles and pointers; rebind a real device, if any
    _gate.unbind_library()
    _backend.HipBackend._instance, _backend._lib = saved
    if saved[0] is not None:
        _gate.bind_library(saved[0]._lib)


def _dev(stub, a):
    """A device-resident ndarray over stub host memory holding ``a``."""
    a = np.ascontiguousarray(a)
    p = ctypes.c_void_p()
    assert stub.mmp_alloc(max(a.nbytes, 1), ctypes.byref(p)) == 0
    ctypes.memmove(p.value, a.ctypes.data, a.nbytes)
    buf = _backend.DeviceBuffer(p.value, a.nbytes)
    return ndarray(buf, a.shape, a.dtype)


def _same_dag(x, y):
    if type(x) is not type(y):
        return False
    if x._dtype != y._dtype or x._shape != y._shape or x._depth != y._depth \
            or x._nleaves != y._nleaves or x._buffers != y._buffers:
        return False
    t = type(x)
    if t is _fusion.InputNode:
        return (x._buffer is y._buffer and x._offset == y._offset and x._strides == y._strides)
    if t is _fusion.ScalarNode:
        return x._bits == y._bits
    if t is _fusion.CastNode:
        return _same_dag(x._input, y._input)
    if t is _fusion.UnaryOpNode:
        return x._op_name == y._op_name and _same_dag(x._input, y._input)
    if t is _fusion.BinaryOpNode:
        return (x._op_name == y._op_name and _same_dag(x._lhs, y._lhs)
                and _same_dag(x._rhs, y._rhs))
    return False


def test_gate_builds_the_python_dags(stub):
    g = np.random.default_rng(1)
    a = _dev(stub, g.standard_normal((4, 6)).astype(np.float32))
    b = _dev(stub, g.standard_normal((4, 6)).astype(np.float32))
    i = _dev(stub, g.integers(-9, 9, (4, 6)).astype(np.int32))
    row = _dev(stub, g.standard_normal((1, 6)).astype(np.float32))
    col = _dev(stub, g.standard_normal((4, 1)).astype(np.float32))
    cases = [
        ("unary", "sin_op", a), ("unary", "neg_op", i), ("unary", "sqrt_op", i),
        ("unary", "isnan_op", a), ("binary", "add_op", a, b), ("binary", "mul_op", i, a),
        ("binary", "div_op", i, i), ("binary", "lt_op", a, b), ("binary", "sub_op", a, 2.5),
        ("binary", "sub_op", 2.5, a), ("binary", "mul_op", i, 3), ("binary", "add_op", i, 1.5),
        ("binary", "floor_divide_op", i, -7), ("binary", "pow_op", a, 2.0),
        ("binary", "mul_op", a, row), ("binary", "add_op", col, row),
        ("binary", "sub_op", i, row),
    ]
    before = _gate.stats()["native_ops"]
    for kind, op, *args in cases:
        if kind == "unary":
            got, want = _gate._native.unary(op, *args), ew._unary_py(op, *args)
        else:
            got, want = _gate._native.binary(op, *args), ew._binary_py(op, *args)
        assert type(got) is ndarray and got._dtype == want._dtype, (op, got._dtype, want._dtype)
        assert got._shape == want._shape and got._strides == want._strides
        assert _same_dag(got._fusion_node, want._fusion_node), op
        # the result is registered with the buffers it reads
        for buf in got._fusion_node._buffers:
            assert any(r() is got for r in buf.lazy_dependents)
    assert _gate.stats()["native_ops"] - before == len(cases)
    # chains: a lazy operand is extended, not re-read
    c = _gate._native.binary("add_op", _gate._native.unary("abs_op", a), b)
    assert c._fusion_node._lhs._op_name == "abs_op" and c._fusion_node._depth == 2


def test_gate_hands_back_what_it_does_not_handle(stub):
    g = np.random.default_rng(2)
    a = _dev(stub, g.standard_normal((4, 6)).astype(np.float32))
    row = _dev(stub, g.standard_normal((1, 6)).astype(np.float32))
    i16 = _dev(stub, g.integers(-9, 9, (4, 6)).astype(np.int16))
    bad = _dev(stub, g.standard_normal((5, 6)).astype(np.float32))
    before = _gate.stats()["fallbacks"]
    with pytest.raises(ValueError):                           # shapes do not broadcast
        _gate._native.binary("add_op", a, bad)
    with pytest.raises(OverflowError):                        # NumPy's error, from Python
        _gate._native.binary("add_op", i16, 100000)
    strided = cp.asarray(g.standard_normal((4, 12)).astype(np.float32)[:, ::2])
    assert strided._np_data is not None and not strided._np_data.flags.c_contiguous
    h = _gate._native.binary("mul_op", strided, 2.0)          # strided host data: Python copies
    assert h._fusion_node is not None and strided._np_data is None
    assert _gate._native.binary("add_op", a, np.float32(1)) is not None  # NumPy scalar
    assert _gate._native.binary("pow_op", i16, 2) is not None            # int power check
    assert _gate.stats()["fallbacks"] - before >= 5


def test_gate_uploads_host_resident_operands(stub):
    """Arrays made from NumPy data start host-resident; the gate uploads
    contiguous data itself (mmp_h2d into a new buffer) and builds the same
    DAG the Python path builds after its own upload."""
    g = np.random.default_rng(5)
    x_np = g.standard_normal(1000).astype(np.float32)
    y_np = g.standard_normal(1000).astype(np.float32)
    s0 = _gate.stats()
    x, y = cp.array(x_np), cp.array(y_np)
    assert x._np_data is not None and x._buffer is None
    z = _gate._native.binary("add_op", x, y)
    s1 = _gate.stats()
    assert s1["native_uploads"] - s0["native_uploads"] == 2
    assert s1["native_ops"] - s0["native_ops"] == 1 and s1["fallbacks"] == s0["fallbacks"]
    for arr, ref in ((x, x_np), (y, y_np)):
        assert arr._np_data is None and arr._buffer is not None and arr._offset == 0
        assert arr._strides == (1,)
        got = np.empty_like(ref)
        ctypes.memmove(got.ctypes.data, arr._buffer.ptr, ref.nbytes)
        assert np.array_equal(got, ref)
    node = z._fusion_node
    assert node._lhs._buffer is x._buffer and node._rhs._buffer is y._buffer
    # the Python path over the now device-resident operands builds the same DAG
    assert _same_dag(node, ew._binary_py("add_op", x, y)._fusion_node)
    # unary and scalar forms, and a whole-array reduction of host data
    u = cp.array(x_np.reshape(10, 100))
    assert _gate._native.unary("sin_op", u)._fusion_node._input._buffer is u._buffer
    w = cp.array(x_np)
    assert _gate._native.binary("mul_op", 3.0, w)._fusion_node._rhs._buffer is w._buffer
    r = cp.array(x_np.reshape(10, 100))
    stub.stub_reset(0)
    out = _gate._native.reduce(_abi.REDUCE_SUM, r, -1)
    assert out is not None and out._shape == (10,) and r._np_data is None
    call = [stub.stub_call(0, j) for j in range(8)]
    assert call[:7] == [5, _abi.REDUCE_SUM, _abi.DTYPE_CODES[np.dtype(np.float32)],
                        _abi.DTYPE_CODES[np.dtype(np.float32)], 10, 100, 1]
    assert _gate.stats()["native_uploads"] - s0["native_uploads"] == 5


def _expected_block(root, out_ptr):
    """The parameter block the Python path packs for ``root``."""
    prog = _fusion._Program(root)
    shape = root._shape
    cshape, outer, cols, leaf_str, kinds = _fusion._plan(prog, shape, keep_last=False)
    vec = _fusion._vec_ok(prog, kinds, leaf_str, outer, cols, out_ptr, root._dtype.itemsize, "map")
    tile = _fusion._map_tile(kinds)
    colblocks = -(-cols // tile)
    P = _fusion._param_struct(len(prog.arrays), len(prog.scalars), len(outer))
    p, rows = _fusion._fill_params(prog, P, outer, cols, leaf_str, out_ptr, colblocks, 1.0)
    return bytes(p), rows * colblocks, vec


@pytest.mark.parametrize("case", ["c1", "chain_scalars", "strided", "int_cast", "where_like",
                                  "c5_broadcast"])
def test_gate_packs_the_python_parameter_block(stub, case):
    g = np.random.default_rng(3)
    x = _dev(stub, g.standard_normal(5000).astype(np.float32))
    m = _dev(stub, g.standard_normal((64, 48)).astype(np.float32))
    i = _dev(stub, g.integers(-5, 5, 5000).astype(np.int32))
    n = _gate._native
    if case == "c1":
        y = n.binary("add_op", n.unary("sqrt_op", n.unary("abs_op", x)),
                     n.unary("exp_op", n.unary("neg_op", n.unary("square_op", x))))
    elif case == "chain_scalars":
        y = n.binary("sub_op", n.binary("mul_op", x, 3.0), n.binary("add_op", x, -1.25))
    elif case == "strided":
        mt = m.transpose()
        y = n.binary("add_op", n.unary("sin_op", mt), mt)
    elif case == "int_cast":
        y = n.binary("add_op", n.binary("mul_op", i, 2), x)  # int32 -> float64 cast leaves
    elif case == "where_like":
        y = n.binary("mul_op", n.binary("gt_op", x, 0.0), x)
    else:  # tanh(x*r + 1.0) * exp(-abs(x)) - log1p(x*x) with a (1, 48) row r
        r = _dev(stub, g.uniform(0.5, 2.0, (1, 48)).astype(np.float32))
        y = n.binary("sub_op",
                     n.binary("mul_op", n.unary("tanh_op", n.binary("add_op", n.binary("mul_op", m, r), 1.0)),
                              n.unary("exp_op", n.unary("neg_op", n.unary("abs_op", m)))),
                     n.unary("log1p_op", n.binary("mul_op", m, m)))
    root = y._fusion_node
    out_probe = ctypes.c_void_p()
    # the block holds the output pointer, which the gate allocates itself:
    # compare everything else, then check that field against the new buffer
    want, nblocks, vec = _expected_block(root, 0)
    stub.stub_reset(len(want))
    n.materialize(y)
    assert y._fusion_node is None and y._buffer is not None
    calls = [[stub.stub_call(k, j) for j in range(8)] for k in range(stub.stub_ncalls())]
    assert len(calls) == 1 and calls[0][0] == 4, calls
    assert calls[0][2] == nblocks and calls[0][5] == 256
    got = ctypes.string_at(stub.stub_params(), len(want))
    nin = len(_fusion._Program(root).arrays)
    off = 8 * max(1, nin)  # outp follows ptr[nin]
    assert got[:off] == want[:off] and got[off + 8:] == want[off + 8:]
    assert int.from_bytes(got[off:off + 8], "little") == y._buffer.ptr
    del out_probe


def test_gate_calls_precompiled_kernels(stub):
    g = np.random.default_rng(4)
    a = _dev(stub, g.standard_normal(1000).astype(np.float32))
    b = _dev(stub, g.standard_normal(1000).astype(np.float32))
    n = _gate._native
    f32 = _abi.DTYPE_CODES[np.dtype(np.float32)]
    for y, expect in ((n.unary("sin_op", a), (1, _abi.UNARY_OPS["sin_op"][0], f32, 1000, a._ptr)),
                      (n.binary("add_op", a, b),
                       (2, _abi.BINARY_OPS["add_op"][0], f32, 1000, a._ptr, b._ptr)),
                      (n.binary("mul_op", a, 2.0),
                       (3, _abi.BINARY_OPS["mul_op"][0], f32, 1000, a._ptr,
                        int.from_bytes(np.float32(2.0).tobytes(), "little"), 1)),
                      (n.binary("sub_op", 0.5, b),
                       (3, _abi.BINARY_OPS["sub_op"][0], f32, 1000, b._ptr,
                        int.from_bytes(np.float32(0.5).tobytes(), "little"), 0))):
        stub.stub_reset(0)
        n.materialize(y)
        call = tuple(stub.stub_call(0, j) for j in range(len(expect)))
        assert stub.stub_ncalls() == 1 and call == expect, (call, expect)
    # fast_math: a fast-form op skips the precompiled kernel
    cp.set_config(fast_math=True)
    try:
        y = n.unary("exp_op", a)
        stub.stub_reset(8)
        n.materialize(y)
        assert stub.stub_call(0, 0) == 4
    finally:
        cp.set_config(fast_math=False)


def test_buffers_are_freed(stub):
    live = stub.stub_live()
    x = _dev(stub, np.ones(100, np.float32))
    y = _gate._native.unary("neg_op", x)
    _gate._native.materialize(y)
    assert stub.stub_live() == live + 2
    del x, y
    assert stub.stub_live() == live


def _record(stub, fn, nbytes):
    stub.stub_reset(nbytes)
    keep = fn()
    calls = [[stub.stub_call(k, j) for j in range(8)] for k in range(stub.stub_ncalls())]
    return calls, ctypes.string_at(stub.stub_params(), nbytes), keep


@pytest.mark.parametrize("shape,axis_last,mean", [((64, 48), True, False), ((2, 20000), True, True),
                                                  ((64, 48), False, False), ((3, 7, 40), True, False)])
def test_gate_run_sum_matches_python(stub, shape, axis_last, mean):
    g = np.random.default_rng(5)
    x = _dev(stub, g.standard_normal(shape).astype(np.float32))
    r = _dev(stub, g.uniform(0.5, 2.0, (1,) * (len(shape) - 1) + (shape[-1],)).astype(np.float32))
    n = _gate._native
    y = n.binary("sub_op", n.unary("tanh_op", n.binary("mul_op", x, r)), n.unary("log1p_op", x))
    root = y._fusion_node
    f32 = np.dtype(np.float32)
    out = _dev(stub, np.zeros(64, np.float32))
    prog = _fusion._Program(root)
    nin, nsc = len(prog.arrays), len(prog.scalars)
    _, outer, _, _, _ = _fusion._plan(prog, root._shape, keep_last=axis_last)
    nbytes = ctypes.sizeof(_fusion._param_struct(nin, nsc, len(outer)))
    want = _record(stub, lambda: _fusion._run_sum_py(root, axis_last, f32, out._ptr, mean), nbytes)
    got = _record(stub, lambda: n.run_sum(root, axis_last, f32, out._ptr, mean), nbytes)
    assert len(got[0]) == len(want[0]) and got[0][0][0] == 4
    assert got[0][0][1:] == want[0][0][1:]  # kernel, grid, block
    off = 8 * max(1, nin)
    assert got[1][:off] == want[1][:off] and got[1][off + 8:] == want[1][off + 8:]
    if len(want[0]) == 2:  # partials, then the reduction over them into out
        assert got[0][1][:7] == want[0][1][:7] and got[0][1][7] == want[0][1][7] == out._ptr
        assert int.from_bytes(got[1][off:off + 8], "little") == got[2].ptr
    else:
        assert int.from_bytes(got[1][off:off + 8], "little") == out._ptr


def test_native_dispatch_switch():
    from macmetalpy_amd._config import set_config
    assert ew.unary is _gate._native.unary
    set_config(native_dispatch=False)
    try:
        assert ew.unary is ew._unary_py and _fusion.materialize is _fusion._materialize_py
        assert _fusion.run_sum is _fusion._run_sum_py
    finally:
        set_config(native_dispatch=True)
    assert ew.binary is _gate._native.binary and _fusion.run_sum is _gate._native.run_sum


def test_gate_reductions_call_the_library_directly(stub):
    """sum / mean / max / argmax of a device-resident contiguous array, over
    everything or the last axis: one mmp_reduce / mmp_argreduce call with the
    Python path's output dtype; anything else is handed back (None)."""
    g = np.random.default_rng(6)
    x = _dev(stub, g.standard_normal((6, 10)).astype(np.float32))
    i = _dev(stub, g.integers(-5, 5, (6, 10)).astype(np.int32))
    n = _gate._native
    f32, i32 = _abi.DTYPE_CODES[np.dtype(np.float32)], _abi.DTYPE_CODES[np.dtype(np.int32)]
    i64 = _abi.DTYPE_CODES[np.dtype(np.int64)]
    f64 = _abi.DTYPE_CODES[np.dtype(np.float64)]
    for code, arr, axis, want_call, shape, dt in (
            (_abi.REDUCE_SUM, x, None, (5, _abi.REDUCE_SUM, f32, f32, 1, 60, 1), (), np.float32),
            (_abi.REDUCE_SUM, i, -1, (5, _abi.REDUCE_SUM, i32, i64, 6, 10, 1), (6,), np.int64),
            (_abi.REDUCE_MEAN, i, None, (5, _abi.REDUCE_MEAN, i32, f64, 1, 60, 1), (), np.float64),
            (_abi.REDUCE_MAX, x, 1, (5, _abi.REDUCE_MAX, f32, f32, 6, 10, 1), (6,), np.float32),
            (_abi.REDUCE_ARGMAX, x, 1, (6, _abi.REDUCE_ARGMAX, f32, 6, 10, 1), (6,), np.int64)):
        stub.stub_reset(0)
        r = n.reduce(code, arr, axis)
        call = tuple(stub.stub_call(0, j) for j in range(len(want_call)))
        assert stub.stub_ncalls() == 1 and call == want_call, (call, want_call)
        assert type(r) is ndarray and r._shape == shape and r._dtype == np.dtype(dt)
        assert r._fusion_node is None and r._buffer is not None
    stub.stub_reset(0)
    assert n.reduce(_abi.REDUCE_ARGMAX, x, None) == 7  # a Python int, read back
    assert stub.stub_ncalls() == 1
    # handed back: other axes, lazy input, non-contiguous views, strided host data
    assert n.reduce(_abi.REDUCE_SUM, x, 0) is None
    assert n.reduce(_abi.REDUCE_SUM, n.unary("neg_op", x), None) is None
    assert n.reduce(_abi.REDUCE_SUM, x.transpose(), None) is None
    assert n.reduce(_abi.REDUCE_SUM, cp.asarray(np.ones((4, 6), np.float32)[:, ::2]), None) is None
    # contiguous host data is uploaded and reduced here
    h = cp.array(np.ones(4, np.float32))
    stub.stub_reset(0)
    r = n.reduce(_abi.REDUCE_SUM, h, None)
    assert type(r) is ndarray and h._np_data is None and stub.stub_call(0, 0) == 5


def test_gate_leaks_no_references(stub):
    """Thousands of gate calls (elementwise ops with arrays and Python
    scalars, materialisation through the precompiled and the generated
    paths, reductions, host-resident operands uploaded by the gate, calls
    handed back to Python, errors) leave the
    reference counts of the shared objects they touch, the number of live
    Python objects and the stub's live allocations where they were."""
    import gc
    import sys
    n = _gate._native
    g = np.random.default_rng(9)
    x = _dev(stub, g.standard_normal((8, 16)).astype(np.float32))
    w = _dev(stub, g.standard_normal((8, 16)).astype(np.float32))
    i = _dev(stub, g.integers(-5, 5, (8, 16)).astype(np.int32))
    f32, i64 = np.dtype(np.float32), np.dtype(np.int64)
    watched = [f32, i64, np.dtype(np.int32), np.dtype(np.float64), ndarray, "add_op", "neg_op",
               "mul_op", "tanh_op", x, w, i, x._buffer, w._buffer, None, True, False]

    def work():
        a = n.binary("add_op", x, w)
        n.materialize(a)                                   # precompiled binary kernel
        b = n.unary("neg_op", n.binary("mul_op", x, 2.5))  # generated kernel
        n.materialize(b)
        c = n.binary("add_op", i, 3)                       # int array + Python int
        n.materialize(c)
        d = n.unary("tanh_op", n.binary("mul_op", x, w))
        n.run_sum(d._fusion_node, True, f32, x._ptr, False)
        r = n.reduce(_abi.REDUCE_SUM, x, None)
        r2 = n.reduce(_abi.REDUCE_MAX, i, -1)
        h = n.binary("add_op", x, cp.array(np.ones((8, 16), np.float32)))  # host: uploaded here
        hu = n.unary("sin_op", cp.array(np.ones(16, np.float32)))
        hr = n.reduce(_abi.REDUCE_SUM, cp.array(np.ones((8, 16), np.float32)), -1)
        hs = n.binary("mul_op", cp.asarray(np.ones((8, 32), np.float32)[:, ::2]), 2.0)  # handed back
        assert n.reduce(_abi.REDUCE_SUM, x, 0) is None
        try:
            n.binary("add_op", x, _dev(stub, np.ones((3, 5), np.float32)))
        except ValueError:
            pass
        return a, b, c, r, r2, h, hu, hr, hs

    for _ in range(20):  # warm the caches, result-dtype tables and kernel table
        work()
    gc.collect()
    refs = [sys.getrefcount(o) for o in watched]
    nobj = len(gc.get_objects())
    live = stub.stub_live()
    for _ in range(2000):
        work()
    gc.collect()
    assert [sys.getrefcount(o) for o in watched] == refs
    assert len(gc.get_objects()) <= nobj + 50
    assert stub.stub_live() == live


def test_gate_result_dtypes_follow_the_float64_policy(stub):
    """The gate's result-dtype tables are filled on first use from the
    Python rules, which depend on float64_behavior: switching the policy
    mid-session must re-resolve them (the reference's tests switch to
    "downcast" per test, and its test_config toggles it at run time)."""
    import warnings
    from macmetalpy_amd._config import set_config
    g = np.random.default_rng(12)
    i = _dev(stub, g.integers(1, 9, (4, 6)).astype(np.int32))
    n = _gate._native
    assert n.binary("div_op", i, i)._dtype == np.dtype(np.float64)
    assert n.unary("sqrt_op", i)._dtype == np.dtype(np.float64)
    assert n.binary("div_op", i, 2)._dtype == np.dtype(np.float64)
    assert cp.mean(i).dtype == np.dtype(np.float64)
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", UserWarning)
        set_config(float64_behavior="downcast")
        assert n.binary("div_op", i, i)._dtype == np.dtype(np.float32)
        assert n.unary("sqrt_op", i)._dtype == np.dtype(np.float32)
        assert n.binary("div_op", i, 2)._dtype == np.dtype(np.float32)
        assert n.reduce(_abi.REDUCE_MEAN, i, None)._dtype == np.dtype(np.float32)
        # and back
        set_config(float64_behavior="cpu_fallback")
    assert n.binary("div_op", i, i)._dtype == np.dtype(np.float64)
    assert n.reduce(_abi.REDUCE_MEAN, i, None)._dtype == np.dtype(np.float64)
