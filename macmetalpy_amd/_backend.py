"""ctypes binding of libmmp_hip.so -- the HIP counterpart of MetalBackend.

Reference: src/macmetalpy/_metal_backend.py.  There, a ``MetalBackend``
singleton loads the metalgpu dylib through ctypes (:108-118, 197-263), owns
a buffer pool (:23-77) and exposes ``create_buffer`` / ``array_to_buffer`` /
``execute_kernel`` / ``synchronize`` (:269-372).  ``HipBackend`` keeps those
method names and meanings, but

* buffers are device allocations (HBM is not host-visible), so reading one
  is an explicit device-to-host copy;
* the library's own work goes through typed C entry points (``unary``,
  ``binary``, ``reduce`` ...); ``execute_kernel(source, name, grid,
  buffers)`` keeps the reference's "compile this source, pick a function,
  run it" for HIP source (``compile`` / ``launch`` underneath);
* every call checks the C status and raises with the library's message.

There is no CPU fallback: if the library is missing or no GPU is present
the first device operation raises ``HipError``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional, Sequence

import numpy as np

from . import _abi

__all__ = ["HipBackend", "DeviceBuffer", "HipError", "HipWaitTimeoutError", "lib_path",
           "load_library", "block_for_grid"]

_HERE = os.path.dirname(os.path.abspath(__file__))


def lib_path() -> str:
    return os.environ.get("MMP_HIP_LIB", os.path.join(_HERE, "libmmp_hip.so"))


class HipError(RuntimeError):
    """A libmmp_hip.so call failed."""


class HipUnsupportedError(HipError, TypeError):
    """Op/dtype combination the device library does not implement."""


class HipArgumentError(HipError, ValueError):
    """Invalid argument rejected by the device library."""


class HipOutOfMemoryError(HipError, MemoryError):
    """Device allocation failed."""


class HipWaitTimeoutError(HipError):
    """A device-side bounded wait of a split reduction or scan ran out, so a
    result computed since the last synchronisation may be wrong."""


_ERR_CLASSES = {
    _abi.MMP_E_WAIT: HipWaitTimeoutError,
    _abi.MMP_E_UNSUPPORTED: HipUnsupportedError,
    _abi.MMP_E_ARG: HipArgumentError,
    _abi.MMP_E_OOM: HipOutOfMemoryError,
}

_c_i64 = ctypes.c_int64
_c_vp = ctypes.c_void_p
_c_int = ctypes.c_int
_c_sz = ctypes.c_size_t
_c_u32p = ctypes.POINTER(ctypes.c_uint32)
_c_i64p = ctypes.POINTER(ctypes.c_int64)

_SIGNATURES = {
    "mmp_init": [_c_int],
    "mmp_device_count": [ctypes.POINTER(_c_int)],
    "mmp_device_info": [ctypes.c_char_p, _c_int, ctypes.POINTER(_c_int), _c_i64p,
                        ctypes.POINTER(_c_int), ctypes.POINTER(_c_int)],
    "mmp_alloc": [_c_sz, ctypes.POINTER(_c_vp)],
    "mmp_free": [_c_vp],
    "mmp_empty_cache": [],
    "mmp_memory_stats": [ctypes.POINTER(_c_sz), ctypes.POINTER(_c_sz)],
    "mmp_h2d": [_c_vp, _c_vp, _c_sz],
    "mmp_d2h": [_c_vp, _c_vp, _c_sz],
    "mmp_d2d": [_c_vp, _c_vp, _c_sz],
    "mmp_host_alloc": [_c_sz, ctypes.POINTER(_c_vp)],
    "mmp_host_free": [_c_vp],
    "mmp_sync": [],
    "mmp_stream": [ctypes.POINTER(_c_vp)],
    "mmp_event_create": [ctypes.POINTER(_c_vp)],
    "mmp_event_record": [_c_vp],
    "mmp_event_elapsed_ms": [_c_vp, _c_vp, ctypes.POINTER(ctypes.c_float)],
    "mmp_event_destroy": [_c_vp],
    "mmp_unary": [_c_int, _c_int, _c_i64, _c_vp, _c_vp],
    "mmp_binary": [_c_int, _c_int, _c_i64, _c_vp, _c_vp, _c_vp],
    "mmp_binary_scalar": [_c_int, _c_int, _c_i64, _c_vp, _c_vp, _c_int, _c_vp],
    "mmp_copy": [_c_int, _c_int, _c_int, _c_i64p, _c_vp, _c_i64p, _c_vp],
    "mmp_copy_strided": [_c_int, _c_int, _c_int, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p],
    "mmp_fill": [_c_int, _c_i64, _c_vp, _c_vp],
    "mmp_reduce": [_c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp],
    "mmp_reduce_noalloc": [_c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp],
    "mmp_argreduce": [_c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp],
    "mmp_scan": [_c_int, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp],
    "mmp_sort": [_c_int, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_int],
    "mmp_searchsorted": [_c_int, _c_i64, _c_vp, _c_i64, _c_vp, _c_int, _c_vp],
    "mmp_take": [_c_int, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp],
    "mmp_gather": [_c_int, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp],
    "mmp_scatter": [_c_int, _c_vp, _c_i64, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64],
    "mmp_nonzero": [_c_i64, _c_vp, _c_i64, _c_vp],
    "mmp_mask_tile_counts": [_c_i64, _c_vp, _c_vp],
    "mmp_mask_positions": [_c_i64, _c_vp, _c_vp, _c_vp],
    "mmp_mask_compact": [_c_int, _c_i64, _c_vp, _c_vp, _c_vp, _c_vp],
    "mmp_bincount": [_c_int, _c_i64, _c_vp, _c_i64, _c_vp],
    "mmp_histogram": [_c_int, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp],
    "mmp_lu": [_c_int, _c_vp, _c_i64, _c_i64, _c_vp, _c_vp],
    "mmp_lu_solve": [_c_int, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64],
    "mmp_cholesky": [_c_int, _c_vp, _c_i64, _c_i64, _c_vp],
    "mmp_qr": [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64],
    "mmp_qr_q": [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp],
    "mmp_eigh": [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_vp],
    "mmp_svd": [_c_int, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp],
    "mmp_matmul": [_c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64,
                   _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64],
    "mmp_rtc_compile": [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_c_vp)],
    "mmp_rtc_build": [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _c_vp, _c_sz,
                      ctypes.POINTER(_c_sz)],
    "mmp_rtc_launch": [_c_vp, _c_u32p, _c_u32p, ctypes.c_uint32, ctypes.POINTER(_c_vp)],
    "mmp_rtc_launch_threads": [_c_vp, _c_u32p, _c_u32p, ctypes.c_uint32, ctypes.POINTER(_c_vp)],
    "mmp_wait_status": [ctypes.POINTER(ctypes.c_uint32)],
    "mmp_debug_fail_next": [_c_int, _c_int],
}

_lib = None
_lib_lock = threading.Lock()


def load_library():
    """Load libmmp_hip.so (no device needed) and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not os.path.exists(path):
            raise HipError(
                f"{path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python macmetalpy_amd/csrc/build.py`")
        lib = ctypes.CDLL(path)
        for name, argtypes in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _c_int
        lib.mmp_last_error.argtypes = []
        lib.mmp_last_error.restype = ctypes.c_char_p
        _lib = lib
        return lib


def _check(status: int, what: str) -> None:
    if status != 0:
        msg = _lib.mmp_last_error().decode(errors="replace")
        raise _ERR_CLASSES.get(status, HipError)(f"{what}: {msg} (status {status})")


def _i64_array(vals: Sequence[int]):
    arr = (ctypes.c_int64 * max(1, len(vals)))(*vals)
    return arr


# Owning handle to one device allocation (the reference's ``_Buffer``,
# _metal_backend.py:121-165), implemented in the native gate: attributes
# ``ptr``, ``nbytes``, ``lazy_dependents``; freed to the stream-ordered pool
# (mmp_free) when the last reference goes.
from ._native import DeviceBuffer  # noqa: E402


_U32x3 = ctypes.c_uint32 * 3

# Results of 32 KiB .. 1 GiB come back into page-locked host blocks (below
# 32 KiB the library copies through its own mapped block).
_PINNED_MIN = 32 << 10
_PINNED_MAX = 1 << 30


class _PinnedBlock:
    """Owner of one page-locked host block, exposed to NumPy as bytes; the
    block goes back to the library's cache when the last array viewing it
    is released."""

    __slots__ = ("_lib", "_ptr", "__array_interface__", "__weakref__")

    def __init__(self, lib, ptr: int, nbytes: int) -> None:
        self._lib = lib
        self._ptr = ptr
        self.__array_interface__ = {"data": (ptr, False), "shape": (nbytes,), "typestr": "|u1",
                                    "version": 3}

    def __del__(self) -> None:
        ptr, self._ptr = self._ptr, 0
        if ptr:
            try:
                self._lib.mmp_host_free(ptr)
            except Exception:  # interpreter shutdown
                pass

_BLOCK_BUDGET = 256


def _largest_divisor(n: int, limit: int) -> int:
    """Largest d <= limit dividing n, preferring multiples of 64."""
    limit = max(1, min(limit, n))
    best = 1
    for d in range(limit, 0, -1):
        if n % d == 0:
            if d % 64 == 0:
                return d
            if best == 1:
                best = d
    return best


def block_for_grid(grid) -> tuple:
    """Uniform workgroup extents dividing the thread grid exactly (x first),
    so that a kernel launched with exactly ``grid`` threads needs no bounds
    check (Metal's dispatchThreads semantics)."""
    bx = _largest_divisor(grid[0], _BLOCK_BUDGET)
    by = _largest_divisor(grid[1], _BLOCK_BUDGET // bx) if len(grid) > 1 else 1
    bz = _largest_divisor(grid[2], _BLOCK_BUDGET // (bx * by)) if len(grid) > 2 else 1
    return (bx, by, bz)


# User kernels (RawKernel, execute_kernel) run exactly the requested number
# of threads.  When no uniform workgroup tiles that count well, the last
# workgroup of a dimension is partial; a kernel marked uniform-workgroup
# (hiprtc's default) may not be dispatched that way, so these sources are
# compiled without that mark, and blockDim is read from the dispatch's
# workgroup size, which is the full extent in every workgroup, so that
# blockIdx * blockDim + threadIdx stays the global index (HIP's own
# blockDim reports the partial extent in a partial workgroup).
DISPATCH_OPTIONS = "-fno-offload-uniform-block"
DISPATCH_PRELUDE = (
    "#define blockDim (dim3(__builtin_amdgcn_workgroup_size_x(), "
    "__builtin_amdgcn_workgroup_size_y(), __builtin_amdgcn_workgroup_size_z()))\n"
    "#define hipBlockDim_x (__builtin_amdgcn_workgroup_size_x())\n"
    "#define hipBlockDim_y (__builtin_amdgcn_workgroup_size_y())\n"
    "#define hipBlockDim_z (__builtin_amdgcn_workgroup_size_z())\n"
    "#line 1\n")


def dispatch_shape(grid) -> tuple:
    """(uniform, block) for a launch of exactly ``grid`` threads (1-3
    dims).  Uniform workgroups dividing the grid are used when they hold at
    least one wave64; otherwise (a prime thread count would get one-thread
    workgroups) full workgroups with a partial last one per dimension."""
    g = tuple(grid) + (1,) * (3 - len(grid))
    if any(x > 0xFFFFFFFF for x in g):
        raise ValueError("grid dimension exceeds 2^32 - 1 threads")
    block = block_for_grid(g)
    if block[0] * block[1] * block[2] >= 64 or g[0] * g[1] * g[2] <= block[0] * block[1] * block[2]:
        return True, block
    bx = min(g[0], _BLOCK_BUDGET)
    by = min(g[1], _BLOCK_BUDGET // bx)
    bz = min(g[2], _BLOCK_BUDGET // (bx * by))
    return False, (bx, by, bz)


def _grid3(grid_size) -> tuple:
    """int, 1-3 tuple or an object with width / height / depth (the
    reference's MetalSize) -> a 3-tuple of thread counts."""
    if isinstance(grid_size, (int, np.integer)):
        return (int(grid_size), 1, 1)
    if hasattr(grid_size, "width"):
        return (int(grid_size.width), int(getattr(grid_size, "height", 1)),
                int(getattr(grid_size, "depth", 1)))
    g = tuple(int(v) for v in grid_size)
    if not 1 <= len(g) <= 3:
        raise ValueError("grid must have 1-3 dimensions")
    return g + (1,) * (3 - len(g))


class HipBackend:
    """Process-wide device context (one GPU, one stream)."""

    _instance: Optional["HipBackend"] = None
    _lock = threading.Lock()

    def __new__(cls) -> "HipBackend":
        inst = cls._instance
        if inst is not None:
            return inst
        with cls._lock:
            if cls._instance is None:
                inst = super().__new__(cls)
                inst._lib = load_library()
                inst._exec_cache = {}
                _check(inst._lib.mmp_init(int(os.environ.get("MMP_DEVICE", "0"))), "mmp_init")
                from ._gate import bind_library
                bind_library(inst._lib)
                cls._instance = inst
            return cls._instance

    # ------------------------------------------------------------ device
    def device_info(self) -> dict:
        arch = ctypes.create_string_buffer(64)
        cus, waves, mt = _c_int(), _c_int(), _c_int()
        mem = _c_i64()
        _check(self._lib.mmp_device_info(arch, 64, ctypes.byref(cus), ctypes.byref(mem),
                                         ctypes.byref(waves), ctypes.byref(mt)),
               "mmp_device_info")
        return {"arch": arch.value.decode(), "cu_count": cus.value,
                "total_mem": mem.value, "wave_size": waves.value,
                "max_threads_per_block": mt.value}

    def maxThreadsPerGroup(self) -> int:  # reference name, _metal_backend.py:259
        return self.device_info()["max_threads_per_block"]

    def threadExecutionWidth(self) -> int:  # reference name, _metal_backend.py:261
        return self.device_info()["wave_size"]

    # ----------------------------------------------------------- buffers
    def create_buffer(self, n: int, dtype) -> DeviceBuffer:
        """Uninitialised device buffer of ``n`` elements of ``dtype``."""
        nbytes = int(n) * np.dtype(dtype).itemsize
        p = _c_vp()
        _check(self._lib.mmp_alloc(max(nbytes, 1), ctypes.byref(p)), "mmp_alloc")
        return DeviceBuffer(p.value, nbytes)

    def array_to_buffer(self, arr: np.ndarray) -> DeviceBuffer:
        """Upload a host array (made C-contiguous) into a new buffer."""
        arr = np.ascontiguousarray(arr)
        buf = self.create_buffer(arr.size, arr.dtype)
        if arr.nbytes:
            _check(self._lib.mmp_h2d(buf.ptr, arr.ctypes.data, arr.nbytes), "mmp_h2d")
        return buf

    def write_buffer(self, buf: DeviceBuffer, byte_offset: int, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes:
            _check(self._lib.mmp_h2d(buf.ptr + byte_offset, arr.ctypes.data, arr.nbytes),
                   "mmp_h2d")

    def read_buffer(self, buf: DeviceBuffer, byte_offset: int, out: np.ndarray) -> np.ndarray:
        """Copy ``out.nbytes`` bytes starting at ``byte_offset`` into ``out``."""
        if out.nbytes:
            _check(self._lib.mmp_d2h(out.ctypes.data, buf.ptr + byte_offset, out.nbytes),
                   "mmp_d2h")
        return out

    def host_empty(self, shape, dtype) -> np.ndarray:
        """A C-contiguous NumPy array in page-locked host memory (a cached
        block, returned to the cache when the array is released), or an
        ordinary array when the size is outside the pinned range or the
        pinned budget is used up.  Copies from the device into it run at
        the link rate."""
        dtype = np.dtype(dtype)
        nbytes = int(np.prod(shape, dtype=np.int64)) * dtype.itemsize
        if not _PINNED_MIN <= nbytes <= _PINNED_MAX:
            return np.empty(shape, dtype)
        p = _c_vp()
        if self._lib.mmp_host_alloc(nbytes, ctypes.byref(p)) or not p.value:
            return np.empty(shape, dtype)
        block = _PinnedBlock(self._lib, p.value, nbytes)
        return np.asarray(block).view(dtype).reshape(shape)

    def copy_buffer(self, dst: int, src: int, nbytes: int) -> None:
        if nbytes:
            _check(self._lib.mmp_d2d(dst, src, nbytes), "mmp_d2d")

    def synchronize(self) -> None:
        _check(self._lib.mmp_sync(), "mmp_sync")

    def wait_status(self) -> int:
        """Flags of device-side bounded waits that ran out since the last
        call (bit 0 a scan row tail found no prefix, bit 1 reduction combine),
        then cleared.
        Non-zero means a scan or reduction result may be wrong."""
        f = ctypes.c_uint32()
        _check(self._lib.mmp_wait_status(ctypes.byref(f)), "mmp_wait_status")
        return f.value

    def debug_fail_next(self, kind: int, count: int = 1) -> None:
        """Test hook: make the ``count``-th next call of ``kind`` fail (1
        allocation, 2 runtime compile, 3 kernel launch) or, for kind 4, make
        the ``count``-th next split reduction or scan give up its bounded
        wait at once (reported as HipWaitTimeoutError by the next
        synchronize / get)."""
        _check(self._lib.mmp_debug_fail_next(int(kind), int(count)), "mmp_debug_fail_next")

    def memory_stats(self) -> tuple[int, int]:
        a, b = _c_sz(), _c_sz()
        _check(self._lib.mmp_memory_stats(ctypes.byref(a), ctypes.byref(b)), "mmp_memory_stats")
        return a.value, b.value

    def empty_cache(self) -> None:
        _check(self._lib.mmp_empty_cache(), "mmp_empty_cache")

    # ------------------------------------------------------------ events
    def event(self) -> int:
        e = _c_vp()
        _check(self._lib.mmp_event_create(ctypes.byref(e)), "mmp_event_create")
        return e.value

    def record(self, ev: int) -> None:
        _check(self._lib.mmp_event_record(ev), "mmp_event_record")

    def elapsed_ms(self, start: int, end: int) -> float:
        ms = ctypes.c_float()
        _check(self._lib.mmp_event_elapsed_ms(start, end, ctypes.byref(ms)),
               "mmp_event_elapsed_ms")
        return float(ms.value)

    def destroy_event(self, ev: int) -> None:
        _check(self._lib.mmp_event_destroy(ev), "mmp_event_destroy")

    # ----------------------------------------------------------- kernels
    def unary(self, op: int, dcode: int, n: int, x: int, out: int) -> None:
        _check(self._lib.mmp_unary(op, dcode, n, x, out), "mmp_unary")

    def binary(self, op: int, dcode: int, n: int, a: int, b: int, out: int) -> None:
        _check(self._lib.mmp_binary(op, dcode, n, a, b, out), "mmp_binary")

    def binary_scalar(self, op: int, dcode: int, n: int, arr: int, scalar: np.ndarray,
                      scalar_side: int, out: int) -> None:
        _check(self._lib.mmp_binary_scalar(op, dcode, n, arr, scalar.ctypes.data,
                                           scalar_side, out), "mmp_binary_scalar")

    def copy(self, src_code: int, dst_code: int, shape, x: int, x_strides, out: int) -> None:
        nd = len(shape)
        _check(self._lib.mmp_copy(src_code, dst_code, nd, _i64_array(shape), x,
                                  _i64_array(x_strides), out), "mmp_copy")

    def copy_strided(self, src_code: int, dst_code: int, shape, src: int, src_strides,
                     dst: int, dst_strides) -> None:
        nd = len(shape)
        _check(self._lib.mmp_copy_strided(src_code, dst_code, nd, _i64_array(shape), src,
                                          _i64_array(src_strides), dst,
                                          _i64_array(dst_strides)), "mmp_copy_strided")

    def fill(self, dcode: int, n: int, value: np.ndarray, out: int) -> None:
        _check(self._lib.mmp_fill(dcode, n, value.ctypes.data, out), "mmp_fill")

    def reduce(self, op: int, dcode: int, out_code: int, outer: int, length: int,
               inner: int, x: int, out: int) -> None:
        _check(self._lib.mmp_reduce(op, dcode, out_code, outer, length, inner, x, out),
               "mmp_reduce")

    def argreduce(self, op: int, dcode: int, outer: int, length: int, inner: int,
                  x: int, out: int) -> None:
        _check(self._lib.mmp_argreduce(op, dcode, outer, length, inner, x, out),
               "mmp_argreduce")

    def scan(self, op: int, dcode: int, out_code: int, outer: int, length: int,
             inner: int, x: int, out: int) -> None:
        _check(self._lib.mmp_scan(op, dcode, out_code, outer, length, inner, x, out),
               "mmp_scan")

    def sort(self, dcode: int, rows: int, length: int, x: int, out_values, out_indices,
             stable: bool) -> None:
        _check(self._lib.mmp_sort(dcode, rows, length, x, out_values, out_indices,
                                  1 if stable else 0), "mmp_sort")

    def searchsorted(self, dcode: int, n: int, sorted_ptr: int, m: int, values: int,
                     side_right: bool, out: int) -> None:
        _check(self._lib.mmp_searchsorted(dcode, n, sorted_ptr, m, values,
                                          1 if side_right else 0, out), "mmp_searchsorted")

    def take(self, itemsize: int, nsrc: int, src: int, n: int, indices: int, out: int) -> None:
        _check(self._lib.mmp_take(itemsize, nsrc, src, n, indices, out), "mmp_take")

    def gather(self, word: int, src: int, src_bytes: int, offsets: int, unit: int, n: int,
               row_words: int, out: int, wrap: int = 0, flag: int = 0) -> None:
        _check(self._lib.mmp_gather(word, src, src_bytes, offsets, unit, wrap, flag or None, n,
                                    row_words, out), "mmp_gather")

    def scatter(self, word: int, dst: int, dst_bytes: int, offsets: int, unit: int, n: int,
                row_words: int, src: int, src_rows: int) -> None:
        _check(self._lib.mmp_scatter(word, dst, dst_bytes, offsets, unit, n, row_words, src,
                                     src_rows), "mmp_scatter")

    def nonzero(self, n: int, incl: int, count: int, out: int) -> None:
        _check(self._lib.mmp_nonzero(n, incl, count, out), "mmp_nonzero")

    def mask_tile_counts(self, n: int, mask: int, tile_incl: int) -> None:
        _check(self._lib.mmp_mask_tile_counts(n, mask, tile_incl), "mmp_mask_tile_counts")

    def mask_positions(self, n: int, mask: int, tile_incl: int, out: int) -> None:
        _check(self._lib.mmp_mask_positions(n, mask, tile_incl, out), "mmp_mask_positions")

    def mask_compact(self, word: int, n: int, mask: int, tile_incl: int, src: int, out: int) -> None:
        _check(self._lib.mmp_mask_compact(word, n, mask, tile_incl, src, out), "mmp_mask_compact")

    def bincount(self, dcode, n, x, nbins, counts) -> None:
        _check(self._lib.mmp_bincount(dcode, n, x, nbins, counts), "mmp_bincount")

    def histogram(self, dcode, n, x, nedges, edges, counts) -> None:
        _check(self._lib.mmp_histogram(dcode, n, x, nedges, edges, counts), "mmp_histogram")

    def lu(self, dcode, a, batch, n, piv, info) -> None:
        _check(self._lib.mmp_lu(dcode, a, batch, n, piv, info), "mmp_lu")

    def lu_solve(self, dcode, lu, piv, b, batch, n, nrhs) -> None:
        _check(self._lib.mmp_lu_solve(dcode, lu, piv, b, batch, n, nrhs), "mmp_lu_solve")

    def cholesky(self, dcode, a, batch, n, info) -> None:
        _check(self._lib.mmp_cholesky(dcode, a, batch, n, info), "mmp_cholesky")

    def qr(self, dcode, a, tau, batch, m, n) -> None:
        _check(self._lib.mmp_qr(dcode, a, tau, batch, m, n), "mmp_qr")

    def qr_q(self, dcode, a, tau, batch, m, n, qcols, q) -> None:
        _check(self._lib.mmp_qr_q(dcode, a, tau, batch, m, n, qcols, q), "mmp_qr_q")

    def eigh(self, dcode, a, v, batch, n, sweeps) -> None:
        _check(self._lib.mmp_eigh(dcode, a, v, batch, n, sweeps), "mmp_eigh")

    def svd(self, dcode, w, vt, batch, rows, length, sweeps) -> None:
        _check(self._lib.mmp_svd(dcode, w, vt, batch, rows, length, sweeps), "mmp_svd")

    def matmul(self, dcode: int, batch: int, M: int, N: int, K: int,
               A: int, lda: int, sA: int, B: int, ldb: int, sB: int,
               C: int, ldc: int, sC: int) -> None:
        _check(self._lib.mmp_matmul(dcode, batch, M, N, K, A, lda, sA, B, ldb, sB,
                                    C, ldc, sC), "mmp_matmul")

    # ------------------------------------------ reference kernel interface
    def execute_kernel(self, shader_src: str, func_name, grid_size, buffers) -> None:
        """Compile (cached), select and launch one kernel of ``shader_src``
        with one thread per grid point (reference:
        _metal_backend.py:313-357).  ``shader_src`` is HIP C++ (e.g. from
        ``KernelCache().get_shader``); ``grid_size`` counts threads (int,
        tuple or a MetalSize-like object); ``buffers`` are DeviceBuffers
        (an ndarray's ``_buffer``), device ndarrays or None, bound in order.
        The total thread count is passed as one extra trailing ``long long``
        argument, which the cache's kernels bounds-check against and other
        kernels may ignore.  Asynchronous, like the reference's
        ``runFunction(wait=False)``; ``synchronize()`` waits."""
        from ._fusion import RTC_OPTIONS
        name = func_name.decode() if isinstance(func_name, bytes) else str(func_name)
        key = (shader_src, name)
        kern = self._exec_cache.get(key)
        if kern is None:
            kern = self.compile(DISPATCH_PRELUDE + shader_src, name,
                                RTC_OPTIONS + " " + DISPATCH_OPTIONS)
            self._exec_cache[key] = kern
        g = _grid3(grid_size)
        total = g[0] * g[1] * g[2]
        if total <= 0:
            return
        uniform, block = dispatch_shape(g)
        from ._elementwise import flush_lazy
        args = []
        for b in buffers:
            if isinstance(b, DeviceBuffer):
                dev = b
                args.append(_c_vp(b.ptr))
            elif hasattr(b, "_ensure_gpu"):  # an ndarray: upload / evaluate first
                b._ensure_gpu()
                dev = b._buffer
                args.append(_c_vp(b._ptr))
            elif b is None:
                # the reference binds no buffer (-1); a kernel reading it here
                # would fault, so refuse instead
                raise ValueError("execute_kernel: buffer is None (the _buffer of a host-resident "
                                 "array?); pass the array itself or a DeviceBuffer")
            else:
                raise TypeError(f"execute_kernel: unsupported buffer {type(b).__name__}")
            if not dev.ptr:
                raise ValueError("execute_kernel: buffer has been freed")
            flush_lazy(dev)  # pending expressions reading it see the old data
        args.append(_c_i64(total))
        if uniform:
            self.launch(kern, tuple(gi // bi for gi, bi in zip(g, block)), block, args)
        else:
            self.launch_threads(kern, g, block, args)

    # -------------------------------------------------- runtime compile
    def compile(self, source: str, name: str, options: str = "") -> int:
        """hiprtc-compile ``source`` and return a kernel handle (cached)."""
        k = _c_vp()
        _check(self._lib.mmp_rtc_compile(source.encode(), name.encode(), options.encode(),
                                         ctypes.byref(k)), f"mmp_rtc_compile({name})")
        return k.value

    def launch(self, kernel: int, grid: Sequence[int], block: Sequence[int],
               args: Sequence, shared: int = 0) -> None:
        """Launch a compiled kernel on the library stream; ``grid`` counts
        workgroups, ``args`` are ctypes scalars/structs in kernel-parameter
        order."""
        g = _U32x3(*grid) if len(grid) == 3 else _U32x3(*(tuple(grid) + (1, 1, 1))[:3])
        b = _U32x3(*block) if len(block) == 3 else _U32x3(*(tuple(block) + (1, 1, 1))[:3])
        ptrs = (_c_vp * max(1, len(args)))(*[ctypes.addressof(a) for a in args])
        st = self._lib.mmp_rtc_launch(kernel, g, b, shared, ptrs)
        if st:
            _check(st, "mmp_rtc_launch")

    def launch_threads(self, kernel: int, threads: Sequence[int], block: Sequence[int],
                       args: Sequence, shared: int = 0) -> None:
        """Launch exactly ``threads`` work-items (per dimension) in
        workgroups of ``block``; a dimension that ``block`` does not divide
        ends in a partial workgroup (Metal's dispatchThreads)."""
        t = _U32x3(*(tuple(threads) + (1, 1, 1))[:3])
        b = _U32x3(*(tuple(block) + (1, 1, 1))[:3])
        ptrs = (_c_vp * max(1, len(args)))(*[ctypes.addressof(a) for a in args])
        st = self._lib.mmp_rtc_launch_threads(kernel, t, b, shared, ptrs)
        if st:
            _check(st, "mmp_rtc_launch_threads")


def rtc_build(source: str, options: str = "", arch: str = "gfx950") -> bytes:
    """Compile HIP source to a code object without touching a device."""
    lib = load_library()
    size = _c_sz()
    _check(lib.mmp_rtc_build(source.encode(), options.encode(), arch.encode(), None, 0,
                             ctypes.byref(size)), "mmp_rtc_build")
    buf = ctypes.create_string_buffer(size.value)
    _check(lib.mmp_rtc_build(source.encode(), options.encode(), arch.encode(), buf,
                             size.value, ctypes.byref(size)), "mmp_rtc_build")
    return buf.raw
