"""Matrix products (reference: ndarray.__matmul__ ndarray.py:1398-1450,
linalg_top.matmul linalg_top.py:94-111, math_ops.dot math_ops.py:70-103).

All products run on the device through ``mmp_matmul`` (MFMA kernels for
float32 / float16 / float64, exact wrapping integer kernels).  NumPy
semantics: 1-D operands are promoted and squeezed, N-D operands broadcast
their batch dimensions -- the reference raises for 3-D ``@``
(ndarray.py:1422-1423) and sends batched ``cp.matmul`` to the CPU
(linalg_top.py:105-106).  A core-dimension mismatch raises ValueError with
the reference's "matmul shape mismatch" text.
"""
from __future__ import annotations

import numpy as np

from ._backend import HipBackend
from ._broadcasting import broadcast_shapes
from ._dtypes import dtype_code, ufunc_result_dtype
from .ndarray import ndarray, _prod

__all__ = ["matmul", "dot", "vdot", "inner"]


def _asarray(a):
    from . import creation
    return creation.asarray(a)


def _batch_operand(x, batch_shape, mat_shape):
    """Contiguous operand and its batch stride (0 when broadcast)."""
    xb = x._shape[:-2]
    if xb == tuple(batch_shape):
        return x._ensure_contiguous(), _prod(mat_shape)
    if _prod(xb) == 1:
        return x._ensure_contiguous(), 0
    return x._broadcast_copy(tuple(batch_shape) + tuple(mat_shape), x._dtype), _prod(mat_shape)


_SPLITK_MAX_OUT = 128 * 128   # outputs too few to fill the device with tiles
_SPLITK_MIN_K = 16384
_SPLITK_CHUNK = 2048


def _matmul_split_k(rdt, M, N, K, A, B, res):
    """A small output with a long sum (e.g. X @ X.T of a wide X): the K
    range is cut into chunks that run as one batched matmul, so that every
    chunk gets its own workgroups, and the partial products are summed
    (float64 accumulation) into the result."""
    from .reductions import sum as _sum
    kc = _SPLITK_CHUNK
    nb = K // kc
    rem = K - nb * kc
    isz = rdt.itemsize
    part = ndarray._empty_device((nb + (1 if rem else 0), M, N), rdt)
    be = HipBackend()
    be.matmul(dtype_code(rdt), nb, M, N, kc, A._ptr, K, kc, B._ptr, N, kc * N, part._ptr, N, M * N)
    if rem:
        be.matmul(dtype_code(rdt), 1, M, N, rem, A._ptr + nb * kc * isz, K, 0,
                  B._ptr + nb * kc * N * isz, N, 0, part._ptr + nb * M * N * isz, N, M * N)
    res[...] = _sum(part, axis=0)


def matmul(x1, x2, out=None, **kwargs):
    a, b = _asarray(x1), _asarray(x2)
    if a.ndim == 0 or b.ndim == 0:
        raise ValueError("matmul: Input operand does not have enough dimensions")
    rdt = ufunc_result_dtype(np.matmul, a._dtype, b._dtype)
    a1, b1 = a.ndim == 1, b.ndim == 1
    if a1 and b1:
        if a._shape[0] != b._shape[0]:
            raise ValueError(f"matmul shape mismatch: ({a._shape[0]},) @ ({b._shape[0]},)")
        from .reductions import sum as _sum
        r = _sum(a.astype(rdt) * b.astype(rdt)).astype(rdt)
        return out._inplace(r) if out is not None else r
    A = a.reshape(1, -1) if a1 else a
    B = b.reshape(-1, 1) if b1 else b
    M, K = A._shape[-2:]
    K2, N = B._shape[-2:]
    if K != K2:
        raise ValueError(f"matmul shape mismatch: ({M},{K}) @ ({K2},{N})")
    batch_shape = broadcast_shapes(A._shape[:-2], B._shape[:-2])
    batch = _prod(batch_shape)
    if A._dtype != rdt:
        A = A.astype(rdt)
    if B._dtype != rdt:
        B = B.astype(rdt)
    A, sA = _batch_operand(A, batch_shape, (M, K))
    B, sB = _batch_operand(B, batch_shape, (K, N))
    res = ndarray._empty_device(tuple(batch_shape) + (M, N), rdt)
    if res.size:
        if K == 0:
            res.fill(0)
        elif (batch == 1 and M * N <= _SPLITK_MAX_OUT and K >= _SPLITK_MIN_K
              and rdt in (np.float32, np.float64)):
            _matmul_split_k(rdt, M, N, K, A, B, res)
        else:
            HipBackend().matmul(dtype_code(rdt), batch, M, N, K, A._ptr, K, sA, B._ptr, N, sB,
                                res._ptr, N, M * N)
    if a1:
        res = res.reshape(tuple(batch_shape) + (N,))
    elif b1:
        res = res.reshape(tuple(batch_shape) + (M,))
    return out._inplace(res) if out is not None else res


def dot(a, b, out=None):
    a, b = _asarray(a), _asarray(b)
    if a.ndim == 0 or b.ndim == 0:
        r = a * b
    elif a.ndim <= 2 and b.ndim <= 2:
        r = matmul(a, b)
    else:
        raise NotImplementedError("dot of arrays with more than 2 dimensions; use matmul")
    return out._inplace(r) if out is not None else r


def vdot(a, b):
    a, b = _asarray(a).reshape(-1), _asarray(b).reshape(-1)
    return matmul(a, b)


def inner(a, b):
    a, b = _asarray(a), _asarray(b)
    if a.ndim == 1 and b.ndim == 1:
        return matmul(a, b)
    return matmul(a, b.swapaxes(-1, -2))
