"""Host-side logic on the CPU (no device): dtype resolution against NumPy
for every op and dtype pair, weak-scalar rules, broadcasting, reduction
layouts and result dtypes, op-table consistency.  These are the decisions
the Python layer makes before any kernel runs (reference:
ndarray._binary_op / _unary_op, ndarray.py:960-1243; _dtypes.py:77-146;
_broadcasting.py:8-76; reductions.py:74-163)."""
import itertools
import os
import warnings

import numpy as np
import pytest

from macmetalpy_amd import _abi, _dtypes, reductions
from macmetalpy_amd._broadcasting import broadcast_shapes, broadcast_strides
from macmetalpy_amd._config import set_config

DTYPES = [np.dtype(d) for d in (np.bool_, np.int16, np.uint16, np.int32, np.uint32, np.int64,
                                np.uint64, np.float16, np.float32, np.float64)]


_NARROW = {np.dtype(np.int8): np.dtype(np.int16), np.dtype(np.uint8): np.dtype(np.uint16)}


def _numpy_dtype(ufunc, *ops):
    """NumPy's result dtype, with int8 / uint8 mapped as the device maps them."""
    d = _raw_numpy_dtype(ufunc, *ops)
    return _NARROW.get(d, d)


def _raw_numpy_dtype(ufunc, *ops):
    args = [np.empty(0, dtype=o) if isinstance(o, np.dtype) else o for o in ops]
    with np.errstate(all="ignore"), warnings.catch_warnings():
        warnings.simplefilter("ignore")
        return ufunc(*args).dtype


@pytest.mark.parametrize("name", sorted(set(_abi.UNARY_OPS) | set(_abi.EXPR_UNARY_OPS)))
def test_unary_result_dtypes_match_numpy(name):
    ufunc = (_abi.UNARY_OPS.get(name) or (None, None))[1] or _abi.EXPR_UNARY_OPS[name][0]
    for dt in DTYPES:
        try:
            want = _numpy_dtype(ufunc, dt)
        except TypeError:
            with pytest.raises(TypeError):
                _dtypes.ufunc_result_dtype(ufunc, dt)
            continue
        assert _dtypes.ufunc_result_dtype(ufunc, dt) == want, (name, dt)


@pytest.mark.parametrize("name", sorted(set(_abi.BINARY_OPS) | set(_abi.EXPR_BINARY_OPS)))
def test_binary_result_dtypes_match_numpy(name):
    ufunc = (_abi.BINARY_OPS.get(name) or (None, None))[1] or _abi.EXPR_BINARY_OPS[name][0]
    for a, b in itertools.product(DTYPES, DTYPES):
        try:
            want = _numpy_dtype(ufunc, a, b)
        except TypeError:
            with pytest.raises(TypeError):
                _dtypes.ufunc_result_dtype(ufunc, a, b)
            continue
        assert _dtypes.ufunc_result_dtype(ufunc, a, b) == want, (name, a, b)


@pytest.mark.parametrize("scalar", [2, -3, 2.5, True])
def test_weak_python_scalars(scalar):
    """NEP 50: a Python scalar takes the array's dtype where it fits."""
    for dt in DTYPES:
        for ufunc in (np.add, np.multiply, np.maximum, np.less):
            try:
                want = _numpy_dtype(ufunc, dt, scalar)
            except (TypeError, OverflowError):
                continue
            assert _dtypes.ufunc_result_dtype(ufunc, dt, scalar) == want, (ufunc, dt, scalar)
            # cached second lookup agrees
            assert _dtypes.ufunc_result_dtype(ufunc, dt, scalar) == want


def test_integer_scalar_out_of_range_raises():
    with pytest.raises(OverflowError):
        _dtypes.ufunc_result_dtype(np.add, np.dtype(np.int16), 1 << 40)


def test_float64_policy_and_narrow_ints():
    assert _dtypes.resolve_dtype(np.int8) == np.int16
    assert _dtypes.resolve_dtype(np.uint8) == np.uint16
    assert _dtypes.resolve_dtype(None) == np.float32
    assert _dtypes.resolve_dtype(np.float64) == np.float64
    with pytest.raises(TypeError):
        _dtypes.resolve_dtype(np.complex128)
    set_config(float64_behavior="downcast", warn_on_downcast=True)
    with pytest.warns(UserWarning):
        assert _dtypes.resolve_dtype(np.float64) == np.float32
    set_config(warn_on_downcast=False)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert _dtypes.resolve_dtype(np.float64) == np.float32


@pytest.mark.parametrize("shapes", [((3, 1, 5), (4, 1)), ((), (7,)), ((2, 3), (1, 3), (2, 1)),
                                    ((0, 3), (1, 3)), ((1,), (5, 0))])
def test_broadcast_shapes_match_numpy(shapes):
    assert broadcast_shapes(*shapes) == np.broadcast_shapes(*shapes)


def test_broadcast_shapes_mismatch_and_strides():
    with pytest.raises(ValueError):
        broadcast_shapes((3,), (4,))
    # a (1, 5) row viewed as (4, 5): rows have stride 0
    assert tuple(broadcast_strides((1, 5), (4, 5), (5, 1))) == (0, 1)
    assert tuple(broadcast_strides((5,), (2, 3, 5), (1,))) == (0, 0, 1)


@pytest.mark.parametrize("kind", ["sum", "prod", "mean", "cumsum", "cumprod", "var"])
def test_reduction_result_dtypes_match_numpy(kind):
    fn = {"sum": np.sum, "prod": np.prod, "mean": np.mean, "cumsum": np.cumsum,
          "cumprod": np.cumprod, "var": np.var}[kind]
    for dt in DTYPES:
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            want = fn(np.zeros(1, dtype=dt)).dtype
        assert reductions._np_out_dtype(kind, dt) == want, (kind, dt)


def test_reduction_layouts_and_shapes():
    assert reductions._axes(None, 3) is None
    assert reductions._axes(-1, 3) == (2,)
    assert reductions._axes((2, 0), 3) == (0, 2)
    assert reductions._out_shape((4, 5, 6), (1,), False) == (4, 6)
    assert reductions._out_shape((4, 5, 6), (1,), True) == (4, 1, 6)
    assert reductions._out_shape((4, 5, 6), None, True) == (1, 1, 1)
    # (outer, len, inner) views of a contiguous array; None = not one run
    assert reductions._layout((4, 5, 6), None) == (1, 120, 1)
    assert reductions._layout((4, 5, 6), (1,)) == (4, 5, 6)
    assert reductions._layout((4, 5, 6), (1, 2)) == (4, 30, 1)
    assert reductions._layout((4, 5, 6), (0, 2)) is None


def test_op_tables_are_consistent():
    """Every op the dispatcher may emit has a device function, and codes of
    precompiled ops are unique."""
    for name, (code, ufunc, fn) in _abi.UNARY_OPS.items():
        assert _abi.UNARY_FN[name] == fn and isinstance(ufunc, np.ufunc)
    for name, (code, ufunc, fn) in _abi.BINARY_OPS.items():
        assert _abi.BINARY_FN[name] == fn and isinstance(ufunc, np.ufunc)
    codes = [c for n, (c, _, _) in _abi.BINARY_OPS.items()]
    assert len(set(codes)) == len(codes)
    assert set(_abi.EXPR_UNARY_OPS).isdisjoint(_abi.UNARY_OPS)
    assert set(_abi.EXPR_BINARY_OPS).isdisjoint(_abi.BINARY_OPS)
    assert _abi.BOOL_RESULT_OPS <= set(_abi.EXPR_UNARY_OPS) | set(_abi.EXPR_BINARY_OPS)


def test_jacobi_convergence_check():
    """A batch member that used every allowed Jacobi sweep raises NumPy's
    LinAlgError message; fewer sweeps pass."""
    from macmetalpy_amd import linalg as LA
    LA._check_converged(np.array([3, 59, 12]), "SVD did not converge")
    with pytest.raises(np.linalg.LinAlgError, match="SVD did not converge"):
        LA._check_converged(np.array([3, LA._MAX_SWEEPS, 12]), "SVD did not converge")
    src = open(os.path.join(os.path.dirname(LA.__file__), "csrc", "linalg.hip")).read()
    assert f"constexpr int kMaxSweeps = {LA._MAX_SWEEPS};" in src


@pytest.mark.parametrize("grid", [(1,), (7,), (64,), (1000,), (100_000,), (1_000_003,), (65537,),
                                  (37, 23), (1009, 7), (7, 11, 13), (4, 1, 1), (2, 3, 5),
                                  (1 << 20, 3), (97, 89, 83)])
def test_dispatch_shape_covers_exactly_the_grid(grid):
    """RawKernel / execute_kernel launch shape: uniform workgroups of at
    least one wave64 that divide the grid when such a divisor exists (or a
    single workgroup), else full workgroups with a partial last one; the
    workgroup never exceeds 256 threads and, in the uniform case, tiles the
    grid exactly."""
    from macmetalpy_amd._backend import dispatch_shape
    uniform, block = dispatch_shape(grid)
    g = tuple(grid) + (1,) * (3 - len(grid))
    assert len(block) == 3 and all(b >= 1 for b in block)
    assert block[0] * block[1] * block[2] <= 256
    assert all(b <= x for b, x in zip(block, g))
    if uniform:
        assert all(x % b == 0 for x, b in zip(g, block))
        assert block[0] * block[1] * block[2] >= 64 or block == g
    else:
        # a partial last workgroup only where no uniform wave-sized split exists
        assert block[0] * block[1] * block[2] >= 64
        assert any(x % b for x, b in zip(g, block))


def test_dispatch_shape_prime_counts_use_full_workgroups():
    from macmetalpy_amd._backend import dispatch_shape
    assert dispatch_shape((1_000_003,)) == (False, (256, 1, 1))
    assert dispatch_shape((1000,)) == (True, (250, 1, 1))
    with pytest.raises(ValueError):
        dispatch_shape((1 << 32,))


@pytest.mark.parametrize("dt", [np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64])
def test_out_of_range_int_comparisons_are_constant(dt):
    """Comparing an integer array with a Python int outside its dtype's
    range: NumPy compares by value, so every element gives the same answer
    (the library fills the result instead of converting the int)."""
    from macmetalpy_amd._elementwise import _out_of_range_compare
    info = np.iinfo(dt)
    a = np.array([info.min, info.min + 1, 0, info.max - 1, info.max], dt)
    ops = {"lt_op": np.less, "le_op": np.less_equal, "gt_op": np.greater,
           "ge_op": np.greater_equal, "eq_op": np.equal, "ne_op": np.not_equal}
    for s in (info.max + 1, info.min - 1, 2 ** 70, -2 ** 70, 0, info.max):
        for name, uf in ops.items():
            for left in (True, False):
                c = _out_of_range_compare(name, s, np.dtype(dt), left)
                if info.min <= s <= info.max:
                    assert c is None
                    continue
                want = uf(a, s) if left else uf(s, a)
                assert np.all(want == c), (s, name, left)
    assert _out_of_range_compare("lt_op", 2.5, np.dtype(dt), True) is None


def test_logical_ops_read_int_scalars_as_truth_values():
    from macmetalpy_amd._elementwise import _logical_int_scalar
    arr = object()
    assert _logical_int_scalar(arr, 300000, np.dtype(np.int16), 300000, False)[1] is True
    assert _logical_int_scalar(0, arr, 0, np.dtype(np.int16), True)[0] is False
    # beyond int64 NumPy raises OverflowError; the int is left for the
    # conversion to raise it
    assert _logical_int_scalar(arr, 2 ** 64, np.dtype(np.int16), 2 ** 64, False)[1] == 2 ** 64
    with pytest.raises(OverflowError):
        np.logical_or(np.zeros(2, np.int16), 2 ** 64)
    assert np.logical_or(np.zeros(2, np.int16), 300000).tolist() == [True, True]
