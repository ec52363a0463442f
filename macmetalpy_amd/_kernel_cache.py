"""Kernel source by category and dtype (reference: src/macmetalpy/_kernel_cache.py).

The reference keeps a singleton ``KernelCache`` whose ``get_shader(category,
dtype)`` returns Metal source for a family of one-thread-per-element kernels
(``add_op``, ``sin_op``, ``lt_op``, ``where_op`` ...; _kernel_cache.py:192-229,
_kernels.py:21-1017), keyed by ``(category, dtype, fast_math)``; callers hand
that source and a kernel name to ``MetalBackend.execute_kernel`` with one
buffer per argument and a grid of one thread per element
(_fusion.py:457-460, math_ops.py:155-157, bitwise_ops.py:52-54).

Here the source is HIP C++ for gfx950 built from the same per-element
functions as the library's own kernels (csrc/mmp_ops.h), so a kernel taken
from this cache computes exactly what the corresponding ``cp`` op computes
(NumPy semantics, not the reference's Metal approximations).  Kernel names,
argument order and output conventions are the reference's: elementwise
kernels read and write ``dtype``; comparison kernels write int32 0 / 1
(``comparison_bool``: bool); ``where_op`` takes an int32 condition.  Every
kernel also takes a trailing element count, which ``execute_kernel`` passes
as the grid's thread count, and bounds-checks against it.  Categories whose
reference kernels implement a multi-pass protocol of the Metal backend
(reductions, scans, matmul) are served by the device library's entry points
instead (``cp.sum``, ``cp.cumsum``, ``@``) and raise NotImplementedError.
"""
from __future__ import annotations

import threading
from typing import Dict, Tuple

import numpy as np

from . import _abi
from ._config import get_config
from ._dtypes import ctype_name

__all__ = ["KernelCache"]

_LIBRARY_CATEGORIES = {
    "reduction": "cp.sum / cp.prod / cp.max / cp.min (mmp_reduce)",
    "axis_reduction": "cp.sum(axis=...) and friends (mmp_reduce)",
    "parallel_reduction": "cp.sum / cp.argmax (mmp_reduce, mmp_argreduce)",
    "parallel_scan": "cp.cumsum / cp.cumprod (mmp_scan)",
    "matmul": "the @ operator / cp.matmul (mmp_matmul)",
    "nan_reduction": "cp.nansum / cp.nanmax ... (mmp_reduce with MMP_R_NAN*)",
    "nan_elementwise": "cp.isnan / cp.nan_to_num",
    "boolean": "the bitwise operators on device arrays",
    "bool_logic": "cp.logical_and / logical_or / logical_xor",
    "predicate": "cp.isnan / cp.isinf / cp.isfinite / cp.signbit",
}

_CMP = (("lt_op", "<"), ("le_op", "<="), ("gt_op", ">"), ("ge_op", ">="), ("eq_op", "=="),
        ("ne_op", "!="))

# Ops that keep an integer dtype (NumPy's integer loops); the rest are
# floating-point only.
_INT_UNARY = ("neg_op", "negative_op", "positive_op", "abs_op", "sign_op", "square_op",
              "floor_op", "ceil_op", "rint_op", "trunc_op")
_INT_BINARY = ("add_op", "sub_op", "mul_op", "floor_divide_op", "mod_op", "pow_op", "max_op",
               "min_op")

_IDX = "  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;\n  if (i >= n) return;\n"


def _header() -> str:
    from ._fusion import _ops_header
    return _ops_header()


def _elementwise_source(dtype: np.dtype, fast: bool) -> str:
    from ._fusion import _op_fn
    t = ctype_name(dtype)
    is_float = dtype.kind == "f"
    out = [_header()]
    unary = _abi.UNARY_OPS if is_float else {k: _abi.UNARY_OPS[k] for k in _INT_UNARY}
    binary = _abi.BINARY_OPS if is_float else {k: _abi.BINARY_OPS[k] for k in _INT_BINARY}
    for name in unary:
        fn = _op_fn(_abi.UNARY_FN, name, dtype, fast)
        out.append(f'extern "C" __global__ void {name}(const {t}* __restrict__ a, '
                   f'{t}* __restrict__ out, long long n) {{\n{_IDX}  out[i] = {fn}(a[i]);\n}}\n')
    for name in binary:
        fn = _op_fn(_abi.BINARY_FN, name, dtype, fast)
        out.append(f'extern "C" __global__ void {name}(const {t}* __restrict__ a, '
                   f'const {t}* __restrict__ b, {t}* __restrict__ out, long long n) {{\n'
                   f'{_IDX}  out[i] = {fn}(a[i], b[i]);\n}}\n')
    out.append(f'extern "C" __global__ void fill_scalar({t}* __restrict__ out, '
               f'const {t}* __restrict__ val, long long n) {{\n{_IDX}  out[i] = val[0];\n}}\n')
    return "".join(out)


def _comparison_source(dtype: np.dtype, out_t: str) -> str:
    t = ctype_name(dtype)
    out = [_header()]
    for name, op in _CMP:
        out.append(f'extern "C" __global__ void {name}(const {t}* __restrict__ a, '
                   f'const {t}* __restrict__ b, {out_t}* __restrict__ out, long long n) {{\n'
                   f'{_IDX}  out[i] = ({out_t})(a[i] {op} b[i]);\n}}\n')
    return "".join(out)


def _where_source(dtype: np.dtype) -> str:
    t = ctype_name(dtype)
    return (_header() + f'extern "C" __global__ void where_op(const int* __restrict__ cond, '
            f'const {t}* __restrict__ x, const {t}* __restrict__ y, {t}* __restrict__ out, '
            f'long long n) {{\n{_IDX}  out[i] = cond[i] ? x[i] : y[i];\n}}\n')


def _clip_source(dtype: np.dtype) -> str:
    t = ctype_name(dtype)
    return (_header() + f'extern "C" __global__ void clip_op(const {t}* __restrict__ a, '
            f'const {t}* __restrict__ lo, const {t}* __restrict__ hi, {t}* __restrict__ out, '
            f'long long n) {{\n{_IDX}  out[i] = op_minimum(op_maximum(a[i], lo[i]), hi[i]);\n}}\n')


class KernelCache:
    """Singleton cache of generated kernel source, keyed by
    ``(category, dtype, fast_math)`` as the reference's."""

    _instance: "KernelCache | None" = None
    _lock = threading.Lock()

    def __new__(cls) -> "KernelCache":
        with cls._lock:
            if cls._instance is None:
                inst = super().__new__(cls)
                inst._cache: Dict[Tuple[str, np.dtype, bool], str] = {}
                cls._instance = inst
            return cls._instance

    def get_shader(self, category: str, dtype) -> str:
        """HIP source of the kernels of ``category`` for ``dtype``."""
        dtype = np.dtype(dtype)
        fast = bool(get_config().fast_math) if category == "elementwise" else False
        key = (category, dtype, fast)
        src = self._cache.get(key)
        if src is not None:
            return src
        if dtype not in _abi.CTYPE_NAMES:
            raise TypeError(f"no device kernels for dtype {dtype}")
        if category == "elementwise":
            src = _elementwise_source(dtype, fast)
        elif category == "comparison":
            src = _comparison_source(dtype, "int")
        elif category == "comparison_bool":
            src = _comparison_source(dtype, "bool")
        elif category == "where":
            src = _where_source(dtype)
        elif category == "clip":
            src = _clip_source(dtype)
        elif category in _LIBRARY_CATEGORIES:
            raise NotImplementedError(
                f"shader category {category!r} is a multi-pass Metal protocol; on the MI355X "
                f"use {_LIBRARY_CATEGORIES[category]}")
        else:
            raise ValueError(f"Unknown shader category: {category!r}")
        self._cache[key] = src
        return src

    def clear(self) -> None:
        """Empty the source cache."""
        self._cache.clear()
