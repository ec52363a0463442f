"""NumPy ufunc -> device function map for ``ndarray.__array_ufunc__``
(reference ndarray.py:2681-2720 looks names up on the package)."""
from __future__ import annotations

import numpy as np

_TABLE = None


def lookup(ufunc):
    global _TABLE
    if _TABLE is None:
        from . import ufunc_ops
        t = {}
        for name in ufunc_ops.__all__:
            u = getattr(np, name, None)
            if isinstance(u, np.ufunc):
                t[u] = getattr(ufunc_ops, name)
        from .linalg_top import matmul
        t[np.matmul] = matmul
        _TABLE = t
    return _TABLE.get(ufunc)


# ufunc.reduce / ufunc.accumulate on the device
_REDUCE = {"add": "sum", "multiply": "prod", "maximum": "max", "minimum": "min",
           "logical_and": "all", "logical_or": "any", "fmax": "nanmax", "fmin": "nanmin"}
_ACCUMULATE = {"add": "cumsum", "multiply": "cumprod"}
_IGNORED = ("order", "subok")


def _write_out(out, res, casting, where=True):
    from .ndarray import ndarray
    from . import _elementwise as ew
    outs = out if isinstance(out, tuple) else (out,)
    if len(outs) != 1 or not isinstance(outs[0], ndarray):
        return NotImplemented
    o = outs[0]
    rd = res.dtype if isinstance(res, ndarray) else np.asarray(res).dtype
    if not np.can_cast(rd, o.dtype, casting=casting):
        raise TypeError(f"Cannot cast ufunc output from {rd} to {o.dtype} with casting rule "
                        f"{casting!r}")
    if where is True:
        o[...] = res
    else:
        o[...] = ew.where(where, res, o)
    return o


def dispatch(ufunc, method, inputs, kwargs):
    """Device evaluation of ``ufunc.method(*inputs, **kwargs)`` or
    NotImplemented."""
    from . import creation, reductions, nan_ops
    kwargs = dict(kwargs)
    for k in _IGNORED:
        kwargs.pop(k, None)
    casting = kwargs.pop("casting", "same_kind")
    out = kwargs.pop("out", None)
    if method == "__call__":
        fn = lookup(ufunc)
        where = kwargs.pop("where", True)
        dtype = kwargs.pop("dtype", None)
        if fn is None or kwargs:
            return NotImplemented
        if dtype is not None:
            inputs = tuple(creation.asarray(x).astype(dtype) if not np.isscalar(x) else x
                           for x in inputs)
        res = fn(*inputs)
        if out is None:
            if where is True:
                return res
            # NumPy leaves the outputs outside ``where`` undefined: here they
            # are whatever a new array holds
            out = creation.empty(res.shape, dtype=res.dtype)
        return _write_out(out, res, casting, where)
    name = ufunc.__name__
    if method == "reduce" and name in _REDUCE and len(inputs) == 1:
        axis = kwargs.pop("axis", 0)
        kw = {k: kwargs.pop(k) for k in ("keepdims", "initial", "where", "dtype") if k in kwargs}
        if kwargs:
            return NotImplemented
        fname = _REDUCE[name]
        fn = getattr(nan_ops, fname) if fname.startswith("nan") else getattr(reductions, fname)
        if fname in ("all", "any") and "initial" in kw:
            return NotImplemented
        if fname in ("max", "min", "nanmax", "nanmin", "all", "any"):
            kw.pop("dtype", None)
        if fname.startswith("nan"):
            kw.pop("initial", None)
            kw.pop("where", None)
        res = fn(inputs[0], axis=axis, **kw)
        return res if out is None else _write_out(out, res, casting)
    if method == "accumulate" and name in _ACCUMULATE and len(inputs) == 1:
        axis = kwargs.pop("axis", 0)
        dtype = kwargs.pop("dtype", None)
        if kwargs:
            return NotImplemented
        res = getattr(reductions, _ACCUMULATE[name])(inputs[0], axis=axis, dtype=dtype)
        return res if out is None else _write_out(out, res, casting)
    return NotImplemented
