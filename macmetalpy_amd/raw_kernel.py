"""User-written kernels (reference: src/macmetalpy/raw_kernel.py:15-62).

``RawKernel(source, func_name)(grid, args)`` keeps the reference's call
shape: ``grid`` is the TOTAL number of threads (int or 1-3 tuple), as in
Metal's ``dispatchThreads``, and ``args`` are arrays bound in order.  The
source is HIP C++ (compiled by hiprtc for gfx950) instead of MSL; the
kernel reads its index as ``blockIdx.x * blockDim.x + threadIdx.x`` and,
because exactly ``grid`` threads are launched, needs no bounds check.

Exactly ``grid`` threads run.  When a divisor of the thread count that
holds at least one wave64 fits the block budget (256 threads), workgroups
of that extent tile the grid uniformly; otherwise (a prime count, say)
workgroups of up to 256 threads are used and the last one in each
dimension is partial: its missing threads do not run, and ``blockDim``
still reports the full extent, so ``blockIdx * blockDim + threadIdx`` is
the global index either way.  Scalars (NumPy scalar objects, Python
int/float) may be passed by value.
"""
from __future__ import annotations

import ctypes
from typing import Sequence, Union

import numpy as np

from . import _elementwise as ew
from ._backend import DISPATCH_OPTIONS, DISPATCH_PRELUDE, HipBackend, dispatch_shape
from .ndarray import ndarray

__all__ = ["RawKernel"]

_CTYPES = {
    np.dtype(np.float32): ctypes.c_float, np.dtype(np.float64): ctypes.c_double,
    np.dtype(np.int32): ctypes.c_int32, np.dtype(np.uint32): ctypes.c_uint32,
    np.dtype(np.int64): ctypes.c_int64, np.dtype(np.uint64): ctypes.c_uint64,
    np.dtype(np.int16): ctypes.c_int16, np.dtype(np.uint16): ctypes.c_uint16,
    np.dtype(np.bool_): ctypes.c_bool,
}

class RawKernel:
    def __init__(self, source: str, func_name: str, options: str = "") -> None:
        if "metal_stdlib" in source or "[[buffer(" in source:
            raise TypeError("RawKernel takes HIP C++ source on the MI355X; Metal Shading "
                            "Language kernels must be rewritten as extern \"C\" __global__ "
                            "HIP functions")
        self._source = source
        self._func_name = func_name
        self._options = options
        self._kernel = None

    @property
    def kernel(self) -> int:
        if self._kernel is None:
            self._kernel = HipBackend().compile(
                DISPATCH_PRELUDE + self._source, self._func_name,
                ("-O3 -std=c++17 " + DISPATCH_OPTIONS + " " + self._options).strip())
        return self._kernel

    def __call__(self, grid: Union[int, tuple], args: Sequence, shared_mem: int = 0) -> None:
        if isinstance(grid, (int, np.integer)):
            grid = (int(grid),)
        grid = tuple(int(g) for g in grid)
        if not 1 <= len(grid) <= 3:
            raise ValueError("grid tuple must have 1-3 elements")
        if any(g <= 0 for g in grid):
            return
        uniform, block = dispatch_shape(grid)
        cargs = []
        arrays = []
        for a in args:
            if isinstance(a, ndarray):
                a._ensure_gpu()
                arrays.append(a)
                cargs.append(ctypes.c_void_p(a._ptr))
            elif isinstance(a, np.generic) and a.dtype in _CTYPES:
                cargs.append(_CTYPES[a.dtype](a.item()))
            elif isinstance(a, float):
                cargs.append(ctypes.c_float(a))
            elif isinstance(a, int):
                cargs.append(ctypes.c_int32(a))
            else:
                raise TypeError(f"unsupported RawKernel argument type {type(a).__name__}")
        for a in arrays:  # the kernel may write any of them
            ew.flush_lazy(a._buffer)
        if uniform:
            HipBackend().launch(self.kernel, tuple(g // b for g, b in zip(grid + (1, 1), block)),
                                block, cargs, shared_mem)
        else:
            HipBackend().launch_threads(self.kernel, grid, block, cargs, shared_mem)
