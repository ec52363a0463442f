"""Elementwise dispatch: dtype resolution, lazy DAG construction, eager path.

Reference: ndarray._binary_op / _unary_op (src/macmetalpy/ndarray.py:960-1243).
The reference's order of steps is kept -- wrap scalar, resolve the result
dtype, cast, broadcast, fusion intercept, launch -- with three changes:

* no CPU path: every op runs on the GPU whatever the size (the reference
  sends arrays below 8K/256K/4M elements to NumPy, ndarray.py:41-44);
* the result dtype is NumPy's own type resolution for the ufunc
  (``np.sin(int32)`` is float64, ``int32 // int32`` is int32, ...), then the
  float64 policy; the reference's GPU kernels instead compute in the input
  dtype;
* with fusion on (default) every op returns a lazy array; scalars become
  kernel arguments and broadcasts stride-0 leaves.  With fusion off, ops run
  one by one on precompiled kernels after materialising broadcasts and
  casts, as the reference's GPU path does.
"""
from __future__ import annotations

import numbers
import weakref

import numpy as np

from . import _abi
from ._broadcasting import broadcast_shapes
from ._config import get_config
from ._dtypes import resolve_dtype, ufunc_result_dtype
from ._fusion import (
    _MAX_DEPTH, _MAX_LEAVES, BinaryOpNode, CastNode, InputNode, ScalarNode, UnaryOpNode,
    WhereNode, materialize,
)

__all__ = ["unary", "binary", "where", "is_scalar", "flush_lazy", "track_lazy"]


def is_scalar(x) -> bool:
    return isinstance(x, (numbers.Number, np.generic, bool)) and not isinstance(x, np.ndarray)


_mods = {}


def _ndarray():
    cls = _mods.get("ndarray")
    if cls is None:  # imported lazily: ndarray imports this module
        from .ndarray import ndarray as cls
        _mods["ndarray"] = cls
    return cls


def _creation():
    mod = _mods.get("creation")
    if mod is None:
        from . import creation as mod
        _mods["creation"] = mod
    return mod


def _asarray(x):
    return _creation().asarray(x)


# ----------------------------------------------------- lazy dependents
_PRUNE_AT = 64


def track_lazy(arr) -> None:
    """Register lazy ``arr`` with every device buffer its DAG reads, so an
    in-place write to one of those buffers first evaluates ``arr``.  The
    entries are plain weak references: ``flush_lazy`` skips dead and
    already evaluated arrays, and a buffer's list is pruned of them when it
    grows past ``_PRUNE_AT`` entries."""
    ref = weakref.ref(arr)
    for buf in arr._fusion_node._buffers:
        deps = buf.lazy_dependents
        if deps is None:
            buf.lazy_dependents = [ref]
            continue
        deps.append(ref)
        if len(deps) > _PRUNE_AT:
            _prune_deps(deps)


def _prune_deps(deps) -> None:
    """Drop dead and already evaluated arrays from a buffer's dependents
    list, in place."""
    deps[:] = [r for r in deps if _pending(r) is not None]


def _pending(ref):
    arr = ref()
    return arr if arr is not None and arr._fusion_node is not None else None


def flush_lazy(buffer) -> None:
    """Evaluate pending lazy arrays that read ``buffer`` (before an in-place
    write to it).  NumPy evaluates eagerly, so they must see the old data."""
    if buffer is None:
        return
    deps = buffer.lazy_dependents
    if not deps:
        return
    buffer.lazy_dependents = None
    for ref in deps:
        arr = _pending(ref)
        if arr is not None:
            materialize(arr)


# ----------------------------------------------------------- node helpers
def _node_of(x, dtype):
    """Fusion node reading ndarray ``x`` as ``dtype``."""
    node = x._fusion_node
    if node is None:
        x._ensure_gpu()
        node = InputNode(x._buffer, x._shape, x._dtype, x._strides, x._offset)
    if node._dtype != dtype:
        node = CastNode(node, dtype)
    return node


def _limit(x, node, dtype, extra_depth=1):
    """Materialise ``x`` first when fusing would exceed the depth or leaf
    caps (reference: _MAX_DEPTH, ndarray.py:1218-1224)."""
    if x._fusion_node is not None and (node._depth + extra_depth > _MAX_DEPTH
                                       or node._nleaves > _MAX_LEAVES):
        materialize(x)
        return _node_of(x, dtype)
    return node


def _lazy_result(node):
    arr = _ndarray()._lazy(node)
    track_lazy(arr)
    return arr


def _empty(shape, dtype):
    return _creation().empty(shape, dtype=dtype)


def _materialise_operand(x, shape, dtype):
    """Unfused mode: contiguous, full-shape, result-dtype copy of ``x``
    (the reference's astype + _gpu_broadcast_to, ndarray.py:1058-1065)."""
    x._materialize_if_lazy()
    if x._shape == tuple(shape) and x._dtype == dtype and x._is_device_contiguous():
        return x
    return x._broadcast_copy(shape, dtype)


# ------------------------------------------------------------------ ops
_UNARY_DTYPES: dict = {}


def _unary_dtypes(op_name, dt):
    """(result dtype, dtype the operand is read as) of a unary op."""
    key = (op_name, dt)
    hit = _UNARY_DTYPES.get(key)
    if hit is None:
        ent = _abi.UNARY_OPS.get(op_name)
        ufunc = ent[1] if ent is not None else _abi.EXPR_UNARY_OPS[op_name][0]
        rdt = ufunc_result_dtype(ufunc, dt)
        # predicates read the operand as it is; other ops compute in the result dtype
        own = op_name in _abi.BOOL_RESULT_OPS or op_name in _abi.OWN_INPUT_OPS
        hit = _UNARY_DTYPES[key] = (rdt, dt if own else rdt)
    return hit


def _unary_py(op_name: str, x):
    """The Python path of a unary op (the native gate calls it for every
    case it does not handle itself)."""
    if type(x) is not _ndarray():
        x = _asarray(x)
    rdt, idt = _unary_dtypes(op_name, x._dtype)
    if x.size == 0:
        return _empty(x._shape, rdt)
    if not get_config().fusion:
        xin = _materialise_operand(x, x._shape, idt)
        node = UnaryOpNode(op_name, _node_of(xin, idt), x._shape, rdt)
        out = _lazy_result(node)
        materialize(out)
        return out
    node = _limit(x, _node_of(x, idt), idt)
    return _lazy_result(UnaryOpNode(op_name, node, x._shape, rdt))


def _scalar_operand(v):
    """Python / NumPy scalar for dtype resolution (NEP 50: Python scalars
    are weak, NumPy scalars strong)."""
    if isinstance(v, np.generic):
        return v
    if isinstance(v, bool):
        return bool(v)
    return v


_BINARY_DTYPES: dict = {}
_LOGICAL_OPS = frozenset({"logical_and_op", "logical_or_op", "logical_xor_op"})
# (array OP scalar) when the scalar exceeds every value of the array's
# integer dtype; below every value the answers flip except == / !=
_ABOVE = {"lt_op": True, "le_op": True, "gt_op": False, "ge_op": False, "eq_op": False,
          "ne_op": True}
_FLIP = {"lt_op": "gt_op", "le_op": "ge_op", "gt_op": "lt_op", "ge_op": "le_op",
         "eq_op": "eq_op", "ne_op": "ne_op"}


def _out_of_range_compare(op_name, s, dtype, array_left):
    """The constant result of comparing an integer array with a Python int
    outside its dtype's range (NumPy compares by value), or None when the
    int is in range or not an int."""
    if type(s) is not int:
        return None
    info = np.iinfo(dtype)
    if info.min <= s <= info.max:
        return None
    op = op_name if array_left else _FLIP[op_name]
    if s > info.max:
        return _ABOVE[op]
    return op in ("gt_op", "ge_op", "ne_op")


def _logical_int_scalar(a, b, ka, kb, b_arr):
    """Replace a Python int operand of a logical op by its truth value when
    it fits int64 (NumPy then accepts it whatever the array's dtype; beyond
    int64 NumPy raises OverflowError, which the conversion below keeps)."""
    s = a if b_arr else b
    if -2 ** 63 <= s < 2 ** 63:
        s = bool(s)
        if b_arr:
            a, ka = s, s
        else:
            b, kb = s, s
    return a, b, ka, kb


def _binary_dtypes(op_name, ka, kb):
    """(result dtype, dtype both operands are read as) of a binary op on
    operand dtypes / Python scalars ``ka``, ``kb``."""
    if op_name in _abi.COMPARE_OPS or op_name in _abi.BOOL_RESULT_OPS:
        # NumPy compares (and tests truth) in the operands' common dtype and
        # returns bool
        ufunc = (_abi.COMPARE_OPS.get(op_name) or _abi.EXPR_BINARY_OPS[op_name])[0]
        ufunc_result_dtype(ufunc, ka, kb)  # raises for invalid operands
        return np.dtype(np.bool_), resolve_dtype(np.result_type(ka, kb))
    ent = _abi.BINARY_OPS.get(op_name)
    ufunc = ent[1] if ent is not None else _abi.EXPR_BINARY_OPS[op_name][0]
    rdt = ufunc_result_dtype(ufunc, ka, kb)
    return rdt, rdt


def _binary_py(op_name: str, a, b):
    """The Python path of a binary op (the native gate calls it for every
    case it does not handle itself)."""
    nd = _ndarray()
    a_arr = isinstance(a, nd)
    b_arr = isinstance(b, nd)
    if not a_arr and not is_scalar(a):
        a = _asarray(a)
        a_arr = True
    if not b_arr and not is_scalar(b):
        b = _asarray(b)
        b_arr = True
    if not a_arr and not b_arr:
        a = _asarray(a)
        a_arr = True
    ka = a._dtype if a_arr else _scalar_operand(a)
    kb = b._dtype if b_arr else _scalar_operand(b)
    if a_arr and b_arr:
        key = (op_name, ka, kb)
        hit = _BINARY_DTYPES.get(key)
        if hit is None:
            hit = _BINARY_DTYPES[key] = _binary_dtypes(op_name, ka, kb)
        rdt, odt = hit
    else:
        if type(a if b_arr else b) is int and op_name in _LOGICAL_OPS:
            # only the truth of an int counts; NumPy accepts any int64 value
            a, b, ka, kb = _logical_int_scalar(a, b, ka, kb, b_arr)
        rdt, odt = _binary_dtypes(op_name, ka, kb)
    sa = a._shape if a_arr else ()
    sb = b._shape if b_arr else ()
    shape = broadcast_shapes(sa, sb)
    size = 1
    for s in shape:
        size *= s
    if size == 0:
        return _empty(shape, rdt)
    if not (a_arr and b_arr) and op_name in _abi.COMPARE_OPS and odt.kind in "iu":
        const = _out_of_range_compare(op_name, b if a_arr else a, odt, a_arr)
        if const is not None:
            return _creation().full(shape, const, dtype=np.bool_)
    if op_name == "pow_op" and rdt.kind in "iu":
        _check_int_power(b if b_arr else None, None if b_arr else b)

    if not get_config().fusion:
        an = (_node_of(_materialise_operand(a, shape, odt), odt) if a_arr
              else ScalarNode(a, odt))
        bn = (_node_of(_materialise_operand(b, shape, odt), odt) if b_arr
              else ScalarNode(b, odt))
        out = _lazy_result(BinaryOpNode(op_name, an, bn, shape, rdt))
        materialize(out)
        return out

    an = _node_of(a, odt) if a_arr else ScalarNode(a, odt)
    bn = _node_of(b, odt) if b_arr else ScalarNode(b, odt)
    if a_arr:
        an = _limit(a, an, odt)
    if b_arr:
        bn = _limit(b, bn, odt)
    if an._nleaves + bn._nleaves > _MAX_LEAVES:
        if a_arr and a._fusion_node is not None:
            materialize(a)
            an = _node_of(a, odt)
        if b_arr and b._fusion_node is not None:
            materialize(b)
            bn = _node_of(b, odt)
    return _lazy_result(BinaryOpNode(op_name, an, bn, shape, rdt))


def where(cond, x, y):
    """``x`` where ``cond`` is true, else ``y``, broadcast together
    (reference math_ops.py:106-155).  The result dtype is NumPy's
    ``result_type(x, y)`` (Python scalars weak); ``cond`` is read as its
    truth value.  Lazy like the other elementwise ops."""
    nd = _ndarray()
    cond = cond if isinstance(cond, nd) else _asarray(cond)
    ops = []
    for v in (x, y):
        if not isinstance(v, nd) and not is_scalar(v):
            v = _asarray(v)
        ops.append(v)
    x, y = ops
    x_arr, y_arr = isinstance(x, nd), isinstance(y, nd)
    kx = x._dtype if x_arr else _scalar_operand(x)
    ky = y._dtype if y_arr else _scalar_operand(y)
    rdt = resolve_dtype(np.result_type(kx, ky))
    shape = broadcast_shapes(cond._shape, x._shape if x_arr else (), y._shape if y_arr else ())
    size = 1
    for s in shape:
        size *= s
    if size == 0:
        return _empty(shape, rdt)
    bdt = np.dtype(np.bool_)
    unfused = not get_config().fusion

    def leaf(v, is_arr, dt):
        if not is_arr:
            if type(v) is int and dt.kind in "biu":
                # np.where converts a Python int with a plain cast, which
                # wraps (and warns) where the strict conversion would raise
                v = np.asarray(v).astype(dt)
            return ScalarNode(v, dt)
        if unfused:
            return _node_of(_materialise_operand(v, shape, dt), dt)
        return _limit(v, _node_of(v, dt), dt)

    cn = leaf(cond, True, bdt)
    xn = leaf(x, x_arr, rdt)
    yn = leaf(y, y_arr, rdt)
    if cn._nleaves + xn._nleaves + yn._nleaves > _MAX_LEAVES:
        for v, is_arr in ((cond, True), (x, x_arr), (y, y_arr)):
            if is_arr and v._fusion_node is not None:
                materialize(v)
        cn = leaf(cond, True, bdt)
        xn = leaf(x, x_arr, rdt)
        yn = leaf(y, y_arr, rdt)
    out = _lazy_result(WhereNode(cn, xn, yn, shape, rdt))
    if unfused:
        materialize(out)
    return out


def _check_int_power(exp_arr, exp_scalar):
    """NumPy raises for integer powers with negative integer exponents."""
    msg = "Integers to negative integer powers are not allowed."
    if exp_arr is None:
        if exp_scalar < 0:
            raise ValueError(msg)
        return
    if exp_arr._dtype.kind == "i" and exp_arr.size:
        from . import reductions
        if int(reductions.min(exp_arr)) < 0:
            raise ValueError(msg)


def power(a, b):
    """``a ** b`` with NumPy's scalar-exponent shortcuts for inexact arrays:
    ``**2`` -> square, ``**0.5`` -> sqrt, ``**-1`` -> reciprocal (NumPy's
    fast_scalar_power), which round differently from pow()."""
    nd = _ndarray()
    if isinstance(a, nd) and a._dtype.kind == "f" and is_scalar(b) and not isinstance(b, np.generic):
        if isinstance(b, int) and not isinstance(b, bool):
            if b == 2:
                return unary("square_op", a)
            if b == -1:
                return unary("reciprocal_op", a)
        elif isinstance(b, float):
            if b == 2.0:
                return unary("square_op", a)
            if b == 0.5:
                return unary("sqrt_op", a)
            if b == -1.0:
                return unary("reciprocal_op", a)
    return binary("pow_op", a, b)


def resolve(dtype):
    return resolve_dtype(dtype)


# The native gate (macmetalpy_amd._native) takes over these names when the
# package is set up; until then (and for what it hands back) the Python
# paths run.
unary = _unary_py
binary = _binary_py
