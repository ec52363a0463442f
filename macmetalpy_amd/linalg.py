"""``cp.linalg`` on the device.

The reference's linalg.py wraps NumPy / LAPACK on the host for every
function but matmul.  Here the factorizations run as HIP kernels
(csrc/linalg.hip: LU with partial pivoting, Cholesky, Householder QR,
cyclic Jacobi for symmetric eigenproblems, one-sided Jacobi SVD), one
workgroup per matrix of a batch, and everything built on them (solve,
inv, det, slogdet, lstsq, pinv, matrix_rank, cond, norms, matrix_power,
multi_dot, tensorsolve, tensorinv) composes those kernels with device
matmuls, reductions and fused expressions.

Results agree with NumPy's to rounding (LAPACK blocks its algorithms and
orders its sums differently); singular vectors and eigenvectors are unique
only up to sign, so they agree through reconstruction, not entry by entry.
float32 stays float32, integers and bool compute in float64, float16 is
refused (as NumPy's linalg refuses it).  ``eig`` / ``eigvals`` serve
exactly symmetric matrices (real eigenpairs); general matrices, whose
eigenpairs can be complex, raise NotImplementedError.
"""
from __future__ import annotations

import builtins
from collections import namedtuple

import numpy as np

from . import _elementwise as ew
from ._backend import HipBackend
from ._dtypes import dtype_code
from .linalg_top import matmul
from .ndarray import ndarray, _prod

__all__ = ["LinAlgError", "matmul", "solve", "inv", "det", "slogdet", "cholesky", "qr", "eigh",
           "eigvalsh", "svd", "svdvals", "matrix_rank", "pinv", "lstsq", "cond", "norm",
           "vector_norm", "matrix_norm", "matrix_power", "multi_dot", "tensorsolve",
           "tensorinv", "cross", "diagonal", "matrix_transpose", "outer", "tensordot", "trace",
           "vecdot", "eig", "eigvals"]

LinAlgError = np.linalg.LinAlgError
SlogdetResult = namedtuple("SlogdetResult", ["sign", "logabsdet"])
QRResult = namedtuple("QRResult", ["Q", "R"])
EighResult = namedtuple("EighResult", ["eigenvalues", "eigenvectors"])
SVDResult = namedtuple("SVDResult", ["U", "S", "Vh"])
EigResult = namedtuple("EigResult", ["eigenvalues", "eigenvectors"])


def _asarray(a):
    from .creation import asarray
    return asarray(a)


def _ftype(*dts):
    """NumPy linalg's computation dtype: float32 stays, float64 / integers /
    bool go to float64, float16 is refused."""
    out = np.dtype(np.float32)
    for d in dts:
        d = np.dtype(d)
        if d == np.float16:
            raise TypeError("array type float16 is unsupported in linalg")
        if d != np.float32:
            out = np.dtype(np.float64)
    return out


def _square(a, name="Last 2 dimensions of the array must be square"):
    if a.ndim < 2:
        raise LinAlgError(f"{a.ndim}-dimensional array given. Array must be at least "
                          "two-dimensional")
    if a.shape[-1] != a.shape[-2]:
        raise LinAlgError(name)


def _stack(a, dt):
    """Contiguous device copy (batch, m, n) in dtype dt, and the batch shape."""
    bshape = tuple(a.shape[:-2])
    m, n = a.shape[-2], a.shape[-1]
    c = a.astype(dt) if a.dtype != dt else a.copy()
    return c._ensure_contiguous().reshape((_prod(bshape), m, n)), bshape


def _ints(shape):
    return ndarray._empty_device(shape, np.int32)


def _lu(a3):
    """In-place LU of a (batch, n, n) array; (pivots, info) device arrays."""
    b, n = a3.shape[0], a3.shape[1]
    piv, info = _ints((b, n)), _ints((b,))
    if b and n:
        HipBackend().lu(dtype_code(a3.dtype), a3._ptr, b, n, piv._ptr, info._ptr)
    return piv, info


def _any_positive(info):
    from .reductions import max as _max
    return info.size > 0 and int(_max(info)) > 0


# ------------------------------------------------------------ solve family
def solve(a, b):
    A, B = _asarray(a), _asarray(b)
    _square(A)
    dt = _ftype(A.dtype, B.dtype)
    n = A.shape[-1]
    vec = B.ndim == 1
    Bm = B.reshape(tuple(B.shape) + (1,)) if vec else B
    if Bm.shape[-2] != n:
        raise ValueError(f"solve: Input operand 1 has a mismatch in its core dimension 0 "
                         f"(size {Bm.shape[-2]} is different from {n})")
    from ._broadcasting import broadcast_shapes
    from .manipulation import broadcast_to
    bs = broadcast_shapes(tuple(A.shape[:-2]), tuple(Bm.shape[:-2]))
    if tuple(A.shape[:-2]) != bs:
        A = broadcast_to(A, bs + (n, n))
    if tuple(Bm.shape[:-2]) != bs:
        Bm = broadcast_to(Bm, bs + tuple(Bm.shape[-2:]))
    lu, _ = _stack(A, dt)
    x, _ = _stack(Bm, dt)
    piv, info = _lu(lu)
    if _any_positive(info):
        raise LinAlgError("Singular matrix")
    nrhs = x.shape[2]
    if lu.shape[0] and n and nrhs:
        HipBackend().lu_solve(dtype_code(dt), lu._ptr, piv._ptr, x._ptr, lu.shape[0], n, nrhs)
    x = x.reshape(bs + (n, nrhs))
    return x.reshape(bs + (n,)) if vec else x


def inv(a):
    from .creation import eye
    from .manipulation import broadcast_to
    A = _asarray(a)
    _square(A)
    dt = _ftype(A.dtype)
    n = A.shape[-1]
    lu, bshape = _stack(A, dt)
    piv, info = _lu(lu)
    if _any_positive(info):
        raise LinAlgError("Singular matrix")
    x = broadcast_to(eye(n, dtype=dt), (lu.shape[0], n, n)).copy()
    if lu.shape[0] and n:
        HipBackend().lu_solve(dtype_code(dt), lu._ptr, piv._ptr, x._ptr, lu.shape[0], n, n)
    return x.reshape(bshape + (n, n))


def _lu_diag_sign(a):
    from .manipulation import diagonal
    from .creation import arange
    from .reductions import sum as _sum
    A = _asarray(a)
    _square(A)
    dt = _ftype(A.dtype)
    n = A.shape[-1]
    lu, bshape = _stack(A, dt)
    piv, _ = _lu(lu)
    d = diagonal(lu, 0, 1, 2)
    swaps = _sum(piv != arange(n, dtype=np.int32), axis=-1)
    sign = ew.where(swaps % 2 == 1, dt.type(-1), dt.type(1))
    return d, sign, bshape, dt


def det(a):
    """Product of U's diagonal with the sign of the row permutation."""
    from .reductions import prod
    d, sign, bshape, dt = _lu_diag_sign(a)
    r = (sign * prod(d, axis=-1)).astype(dt)
    return r.reshape(bshape) if bshape else r.reshape(())


def slogdet(a):
    from .reductions import sum as _sum, prod
    d, sign, bshape, dt = _lu_diag_sign(a)
    s = sign * prod(ew.unary("sign_op", d), axis=-1)
    logabs = _sum(ew.unary("log_op", ew.unary("abs_op", d)), axis=-1)
    logabs = ew.where(s == 0, dt.type(-np.inf), logabs)
    s, logabs = s.astype(dt), logabs.astype(dt)
    shp = bshape if bshape else ()
    return SlogdetResult(s.reshape(shp), logabs.reshape(shp))


def cholesky(a, /, *, upper=False):
    A = _asarray(a)
    _square(A)
    dt = _ftype(A.dtype)
    n = A.shape[-1]
    c, bshape = _stack(A, dt)
    info = _ints((c.shape[0],))
    if c.shape[0] and n:
        HipBackend().cholesky(dtype_code(dt), c._ptr, c.shape[0], n, info._ptr)
    if _any_positive(info):
        raise LinAlgError("Matrix is not positive definite")
    L = c.reshape(bshape + (n, n))
    return L.swapaxes(-1, -2).copy() if upper else L


# ---------------------------------------------------------------------- QR
def _qr_factor(A, dt):
    a3, bshape = _stack(A, dt)
    b, m, n = a3.shape
    k = builtins.min(m, n)
    tau = ndarray._empty_device((b, k), dt)
    if b and m and n:
        HipBackend().qr(dtype_code(dt), a3._ptr, tau._ptr, b, m, n)
    return a3, tau, bshape


def _qr_q(a3, tau, qcols, dt):
    b, m, n = a3.shape
    q = ndarray._empty_device((b, m, qcols), dt)
    if b and m and qcols:
        HipBackend().qr_q(dtype_code(dt), a3._ptr, tau._ptr, b, m, n, qcols, q._ptr)
    return q


def qr(a, mode="reduced"):
    """Householder QR (LAPACK's reflector signs, so R's diagonal matches
    NumPy's signs); modes 'reduced', 'complete' and 'r'."""
    from .manipulation import triu
    A = _asarray(a)
    if A.ndim < 2:
        raise LinAlgError(f"{A.ndim}-dimensional array given. Array must be at least "
                          "two-dimensional")
    if mode not in ("reduced", "complete", "r", "raw"):
        raise ValueError(f"Unrecognized mode '{mode}'")
    if mode == "raw":
        raise NotImplementedError("qr(mode='raw') is not supported on the device")
    dt = _ftype(A.dtype)
    a3, tau, bshape = _qr_factor(A, dt)
    b, m, n = a3.shape
    k = builtins.min(m, n)
    rows = m if mode == "complete" else k
    R = triu(a3[:, :rows, :]).reshape(bshape + (rows, n))
    if mode == "r":
        return R
    Q = _qr_q(a3, tau, m if mode == "complete" else k, dt)
    return QRResult(Q.reshape(bshape + (m, Q.shape[2])), R)


# ------------------------------------------------------ symmetric eigen
def _sym_from(A, UPLO):
    from .manipulation import tril, triu
    if UPLO not in ("L", "U"):
        raise ValueError("UPLO argument must be 'L' or 'U'")
    if UPLO == "L":
        lo = tril(A)
        return lo + tril(A, -1).swapaxes(-1, -2)
    up = triu(A)
    return up + triu(A, 1).swapaxes(-1, -2)


def _eigh(a, UPLO, want_vectors):
    from .manipulation import diagonal
    from .sorting import argsort
    from .indexing import take_along_axis
    A = _asarray(a)
    _square(A)
    dt = _ftype(A.dtype)
    n = A.shape[-1]
    S = _sym_from(A.astype(dt), UPLO)
    a3, bshape = _stack(S, dt)
    b = a3.shape[0]
    v = ndarray._empty_device((b, n, n), dt)
    sweeps = _ints((b,))
    if b and n:
        HipBackend().eigh(dtype_code(dt), a3._ptr, v._ptr, b, n, sweeps._ptr)
        _check_converged(sweeps, "Eigenvalues did not converge")
    w = diagonal(a3, 0, 1, 2).copy()
    order = argsort(w, axis=-1)
    w = take_along_axis(w, order, axis=-1)
    if not want_vectors:
        return w.reshape(bshape + (n,)), None
    V = take_along_axis(v, order.reshape((b, 1, n)), axis=-1)
    return w.reshape(bshape + (n,)), V.reshape(bshape + (n, n))


def eigh(a, UPLO="L"):
    w, v = _eigh(a, UPLO, True)
    return EighResult(w, v)


def eigvalsh(a, UPLO="L"):
    return _eigh(a, UPLO, False)[0]


# Sweep cap of the device Jacobi kernels (csrc/linalg.hip, kMaxSweeps): a
# matrix whose rotations have not died out by then reports that count.
_MAX_SWEEPS = 60


def _check_converged(sweeps, msg):
    """Raise LinAlgError (NumPy's message) when a Jacobi solve of the batch
    used every allowed sweep without converging."""
    if int(sweeps.max()) >= _MAX_SWEEPS:
        raise LinAlgError(msg)


def _all_finite(A):
    from .reductions import all as _all
    return bool(_all(ew.unary("isfinite_op", A)))


def _exactly_symmetric(A):
    from .reductions import all as _all
    return bool(_all(A == A.swapaxes(-1, -2)))


def eig(a):
    """Exactly symmetric matrices: their eigenpairs are real, which NumPy
    returns as real arrays too (ascending here, LAPACK's geev order there;
    vectors unit length, sign arbitrary).  A general matrix can have
    complex eigenpairs, which device arrays cannot hold."""
    A = _asarray(a)
    _square(A)
    if A.size and not _all_finite(A):
        raise LinAlgError("Array must not contain infs or NaNs")
    if not _exactly_symmetric(A):
        raise NotImplementedError("eig of a non-symmetric matrix (complex eigenpairs) is not "
                                  "supported on the device")
    w, v = _eigh(A, "L", True)
    return EigResult(w, v)


def eigvals(a):
    A = _asarray(a)
    _square(A)
    if A.size and not _all_finite(A):
        raise LinAlgError("Array must not contain infs or NaNs")
    if not _exactly_symmetric(A):
        raise NotImplementedError("eigvals of a non-symmetric matrix (complex eigenvalues) is "
                                  "not supported on the device")
    return _eigh(A, "L", False)[0]


# -------------------------------------------------------------------- SVD
def _svd(A, dt, compute_uv):
    """(u, s, vh) reduced, s descending, through one-sided Jacobi on the
    rows of A^T (m >= n) or of A (m < n)."""
    from .reductions import sum as _sum
    from .sorting import argsort
    from .indexing import take_along_axis
    a3, bshape = _stack(A, dt)
    b, m, n = a3.shape
    tall = m >= n
    W = a3.swapaxes(1, 2).copy() if tall else a3
    r, L = W.shape[1], W.shape[2]
    vt = ndarray._empty_device((b, r, r), dt)
    sweeps = _ints((b,))
    if b and r:
        if not _all_finite(W):  # LAPACK's gesdd does not converge on NaN / inf
            raise LinAlgError("SVD did not converge")
        HipBackend().svd(dtype_code(dt), W._ptr, vt._ptr, b, r, L, sweeps._ptr)
        _check_converged(sweeps, "SVD did not converge")
    s = ew.unary("sqrt_op", _sum(W * W, axis=-1))
    order = argsort(-s, axis=-1)
    s = take_along_axis(s, order, axis=-1)
    if not compute_uv:
        return None, s.reshape(bshape + (r,)), None, bshape
    W = take_along_axis(W, order.reshape((b, r, 1)), axis=1)
    vt = take_along_axis(vt, order.reshape((b, r, 1)), axis=1)
    safe = ew.where(s == 0, dt.type(1), s)
    Wn = W / safe.reshape((b, r, 1))
    if tall:
        u, vh = Wn.swapaxes(1, 2).copy(), vt
    else:
        u, vh = vt.swapaxes(1, 2).copy(), Wn
    return u, s, vh, bshape


def _complete(q_reduced, dt):
    """Orthonormal columns appended to q (b, m, k) up to m: the complete Q of
    its QR decomposition spans them."""
    from .manipulation import concatenate
    b, m, k = q_reduced.shape
    if k == m:
        return q_reduced
    a3, tau, _ = _qr_factor(q_reduced, dt)
    Q = _qr_q(a3, tau, m, dt)
    return concatenate([q_reduced, Q[:, :, k:]], axis=2)


def svd(a, full_matrices=True, compute_uv=True, hermitian=False):
    A = _asarray(a)
    if A.ndim < 2:
        raise LinAlgError(f"{A.ndim}-dimensional array given. Array must be at least "
                          "two-dimensional")
    dt = _ftype(A.dtype)
    m, n = A.shape[-2], A.shape[-1]
    u, s, vh, bshape = _svd(A, dt, compute_uv)
    if not compute_uv:
        return s
    if full_matrices and m != n:
        if m > n:
            u = _complete(u, dt)
        else:
            vh = _complete(vh.swapaxes(1, 2).copy(), dt).swapaxes(1, 2).copy()
    return SVDResult(u.reshape(bshape + tuple(u.shape[1:])), s.reshape(bshape + (s.shape[-1],)),
                     vh.reshape(bshape + tuple(vh.shape[1:])))


def svdvals(x, /):
    return svd(x, compute_uv=False)


def matrix_rank(A, tol=None, hermitian=False, *, rtol=None):
    from .reductions import max as _max, sum as _sum, all as _all
    M = _asarray(A)
    if M.ndim < 2:
        return int(not bool(_all(M == 0)))
    S = svd(M, compute_uv=False)
    if tol is None:
        if rtol is None:
            rtol = builtins.max(M.shape[-2:]) * np.finfo(S.dtype).eps
        tol = _max(S, axis=-1, keepdims=True) * rtol
    else:
        tol = _asarray(np.asarray(tol))[..., None] if np.ndim(tol) else tol
    r = _sum(S > tol, axis=-1)
    return int(r) if r.ndim == 0 else r


def pinv(a, rcond=None, hermitian=False, *, rtol=np._NoValue):
    from .reductions import max as _max
    A = _asarray(a)
    dt = _ftype(A.dtype)
    m, n = A.shape[-2], A.shape[-1]
    if rcond is None:
        rcond = 1e-15 if rtol is np._NoValue else (
            builtins.max(m, n) * np.finfo(dt).eps if rtol is None else rtol)
    u, s, vh, bshape = _svd(A, dt, True)
    cut = dt.type(rcond) * _max(s, axis=-1, keepdims=True)
    sinv = ew.where(s > cut, dt.type(1) / ew.where(s == 0, dt.type(1), s), dt.type(0))
    k = s.shape[-1]
    res = matmul(vh.swapaxes(1, 2).copy(), sinv.reshape((-1, k, 1)) * u.swapaxes(1, 2))
    return res.reshape(bshape + (n, m))


def lstsq(a, b, rcond=None):
    """Minimum-norm least squares through the SVD (as LAPACK's gelsd):
    (x, residuals, rank, singular values)."""
    from .reductions import max as _max, sum as _sum
    A, B = _asarray(a), _asarray(b)
    if A.ndim != 2:
        raise LinAlgError(f"{A.ndim}-dimensional array given. Array must be two-dimensional")
    vec = B.ndim == 1
    Bm = B.reshape((B.shape[0], 1)) if vec else B
    m, n = A.shape
    if Bm.shape[0] != m:
        raise LinAlgError("Incompatible dimensions")
    dt = _ftype(A.dtype, B.dtype)
    if rcond is None:
        rcond = np.finfo(dt).eps * builtins.max(m, n)
    u, s, vh, _ = _svd(A.reshape((1, m, n)), dt, True)
    u, s, vh = u[0], s[0], vh[0]
    smax = float(_max(s)) if s.size else 0.0
    cut = rcond * smax
    keep = s > cut
    rank = int(_sum(keep))
    sinv = ew.where(keep, dt.type(1) / ew.where(s == 0, dt.type(1), s), dt.type(0))
    Bd = Bm.astype(dt)
    uTb = matmul(u.T.copy(), Bd)
    x = matmul(vh.T.copy(), sinv.reshape((s.size, 1)) * uTb)
    if rank == n and m > n:
        r = matmul(A.astype(dt), x) - Bd
        resid = _sum(r * r, axis=0)
    else:
        resid = ndarray._empty_device((0,), dt)
    if vec:
        x = x.reshape((n,))
    return x, resid, rank, s


# ------------------------------------------------------------------ norms
def _fdt(x):
    return x.astype(np.float64) if x.dtype.kind in "iub" else x


def vector_norm(x, /, *, axis=None, keepdims=False, ord=2):
    from . import reductions
    a = _fdt(_asarray(x))
    if axis is None:
        a2 = a.ravel()
        ax = 0
    else:
        a2, ax = a, axis
    absx = ew.unary("abs_op", a2)
    if ord == np.inf:
        r = reductions.max(absx, axis=ax, keepdims=keepdims)
    elif ord == -np.inf:
        r = reductions.min(absx, axis=ax, keepdims=keepdims)
    elif ord == 0:
        r = reductions.sum((a2 != 0).astype(a2.dtype), axis=ax, keepdims=keepdims)
    elif ord == 1:
        r = reductions.sum(absx, axis=ax, keepdims=keepdims)
    elif ord is None or ord == 2:
        r = ew.unary("sqrt_op", reductions.sum(a2 * a2, axis=ax, keepdims=keepdims))
    else:
        p = float(ord)
        r = reductions.sum(absx ** p, axis=ax, keepdims=keepdims) ** (1.0 / p)
    r = _asarray(r)
    if axis is None and keepdims:
        r = r.reshape((1,) * a.ndim)
    return r


def matrix_norm(x, /, *, keepdims=False, ord="fro"):
    return norm(x, ord=ord, axis=(-2, -1), keepdims=keepdims)


def norm(x, ord=None, axis=None, keepdims=False):
    from . import reductions
    a = _fdt(_asarray(x))
    if axis is None:
        if ord is None or (ord in ("f", "fro") and a.ndim == 2) or (ord == 2 and a.ndim == 1):
            r = ew.unary("sqrt_op", reductions.sum(a * a))
            r = _asarray(r)
            return r.reshape((1,) * a.ndim) if keepdims else r
        axis = tuple(builtins.range(a.ndim))
    if isinstance(axis, (int, np.integer)):
        axis = (int(axis),)
    axis = tuple(axis)
    if len(axis) == 1:
        if isinstance(ord, str):
            raise ValueError(f"Invalid norm order '{ord}' for vectors")
        return vector_norm(a, axis=axis[0], keepdims=keepdims, ord=2 if ord is None else ord)
    if len(axis) != 2:
        raise ValueError("Improper number of dimensions to norm.")
    r0, c0 = (ax % a.ndim for ax in axis)
    if r0 == c0:
        raise ValueError("Duplicate axes given.")
    absx = ew.unary("abs_op", a)
    if ord in (2, -2, "nuc"):
        from .manipulation import moveaxis
        m = moveaxis(a, (r0, c0), (-2, -1))
        s = svd(m, compute_uv=False)
        if ord == 2:
            r = reductions.max(s, axis=-1)
        elif ord == -2:
            r = reductions.min(s, axis=-1)
        else:
            r = reductions.sum(s, axis=-1)
    elif ord in (None, "fro", "f"):
        r = ew.unary("sqrt_op", reductions.sum(a * a, axis=axis))
    elif ord in (1, -1):
        col = reductions.sum(absx, axis=r0)
        c1 = c0 - 1 if c0 > r0 else c0
        r = (reductions.max if ord == 1 else reductions.min)(col, axis=c1)
    elif ord in (np.inf, -np.inf):
        row = reductions.sum(absx, axis=c0)
        r1 = r0 - 1 if r0 > c0 else r0
        r = (reductions.max if ord == np.inf else reductions.min)(row, axis=r1)
    else:
        raise ValueError("Invalid norm order for matrices.")
    r = _asarray(r)
    if keepdims:
        shp = list(a.shape)
        shp[r0] = 1
        shp[c0] = 1
        r = r.reshape(tuple(shp))
    return r


def cond(x, p=None):
    from .reductions import max as _max, min as _min
    A = _asarray(x)
    if p is None or p == 2 or p == -2:
        s = svd(A, compute_uv=False)
        if p == -2:
            return _min(s, axis=-1) / _max(s, axis=-1)
        return _max(s, axis=-1) / _min(s, axis=-1)
    return norm(A, p, axis=(-2, -1)) * norm(inv(A), p, axis=(-2, -1))


# -------------------------------------------------------- products, misc
def matrix_power(a, n):
    """NumPy's binary decomposition (squarings and products in its order)."""
    from .creation import eye
    from .manipulation import broadcast_to
    A = _asarray(a)
    _square(A)
    try:
        n = int(n) if int(n) == n else None
    except (TypeError, ValueError):
        n = None
    if n is None:
        raise TypeError("exponent must be an integer")
    if n == 0:
        return broadcast_to(eye(A.shape[-1], dtype=A.dtype), tuple(A.shape)).copy()
    if n < 0:
        A = inv(A)
        n = abs(n)
    if n == 1:
        return A.copy()
    if n == 2:
        return matmul(A, A)
    if n == 3:
        return matmul(matmul(A, A), A)
    z = result = None
    while n > 0:
        z = A if z is None else matmul(z, z)
        n, bit = divmod(n, 2)
        if bit:
            result = z if result is None else matmul(result, z)
    return result


def _chain_order(shapes):
    """Optimal parenthesization of a matrix chain (classic O(n^3) dynamic
    program on the scalar-multiplication counts), as NumPy's multi_dot."""
    n = len(shapes)
    p = [shapes[0][0]] + [s[1] for s in shapes]
    m = [[0] * n for _ in builtins.range(n)]
    s = [[0] * n for _ in builtins.range(n)]
    for ln in builtins.range(1, n):
        for i in builtins.range(n - ln):
            j = i + ln
            m[i][j] = np.inf
            for k in builtins.range(i, j):
                q = m[i][k] + m[k + 1][j] + p[i] * p[k + 1] * p[j + 1]
                if q < m[i][j]:
                    m[i][j] = q
                    s[i][j] = k
    return s


def multi_dot(arrays, *, out=None):
    arrs = [_asarray(a) for a in arrays]
    n = len(arrs)
    if n < 2:
        raise ValueError("Expecting at least two arrays.")
    first_1d, last_1d = arrs[0].ndim == 1, arrs[-1].ndim == 1
    if first_1d:
        arrs[0] = arrs[0].reshape((1, arrs[0].shape[0]))
    if last_1d:
        arrs[-1] = arrs[-1].reshape((arrs[-1].shape[0], 1))
    for a in arrs:
        if a.ndim != 2:
            raise ValueError(f"{a.ndim}-dimensional array given. Array must be two-dimensional")
    if n == 2:
        r = matmul(arrs[0], arrs[1])
    elif n == 3:
        a, b, c = arrs
        cost1 = a.shape[0] * a.shape[1] * b.shape[1] + a.shape[0] * b.shape[1] * c.shape[1]
        cost2 = b.shape[0] * b.shape[1] * c.shape[1] + a.shape[0] * a.shape[1] * c.shape[1]
        r = matmul(matmul(a, b), c) if cost1 < cost2 else matmul(a, matmul(b, c))
    else:
        s = _chain_order([tuple(a.shape) for a in arrs])

        def go(i, j):
            if i == j:
                return arrs[i]
            return matmul(go(i, s[i][j]), go(s[i][j] + 1, j))
        r = go(0, n - 1)
    if first_1d and last_1d:
        r = r.reshape(())
    elif first_1d:
        r = r.reshape((r.shape[1],))
    elif last_1d:
        r = r.reshape((r.shape[0],))
    if out is not None:
        out[...] = r
        return out
    return r


def tensorsolve(a, b, axes=None):
    from .manipulation import moveaxis
    A, B = _asarray(a), _asarray(b)
    an = A.ndim
    if axes is not None:
        allaxes = list(builtins.range(an))
        for k in axes:
            allaxes.remove(k)
            allaxes.insert(an, k)
        A = A.transpose(allaxes)
    oldshape = tuple(A.shape[-(an - B.ndim):])
    prod = _prod(oldshape)
    if _prod(A.shape) != prod * prod:
        raise LinAlgError("Input arrays must satisfy the requirement "
                          "prod(a.shape[b.ndim:]) == prod(a.shape[:b.ndim])")
    x = solve(A.reshape((prod, prod)), B.ravel())
    return x.reshape(oldshape)


def tensorinv(a, ind=2):
    A = _asarray(a)
    if ind <= 0:
        raise ValueError("Invalid ind argument.")
    oldshape = tuple(A.shape)
    prod = _prod(oldshape[:ind])
    invshape = oldshape[ind:] + oldshape[:ind]
    if _prod(oldshape[ind:]) != prod:
        raise LinAlgError("Last 2 dimensions of the array must be square")
    return inv(A.reshape((prod, -1 if prod == 0 else _prod(oldshape) // prod))).reshape(invshape)


def cross(x1, x2, /, *, axis=-1):
    from .manipulation import cross as _cross
    a, b = _asarray(x1), _asarray(x2)
    if a.shape[axis] != 3 or b.shape[axis] != 3:
        raise ValueError("Both input arrays must be (arrays of) 3-dimensional vectors")
    return _cross(a, b, axis=axis)


def diagonal(x, /, *, offset=0):
    from .manipulation import diagonal as _diag
    return _diag(_asarray(x), offset, -2, -1)


def matrix_transpose(x, /):
    return _asarray(x).swapaxes(-1, -2)


def outer(x1, x2, /):
    from .manipulation import outer as _outer
    a, b = _asarray(x1), _asarray(x2)
    if a.ndim != 1 or b.ndim != 1:
        raise ValueError("Input arrays must be one-dimensional")
    return _outer(a, b)


def tensordot(x1, x2, /, *, axes=2):
    from .manipulation import tensordot as _td
    return _td(x1, x2, axes=axes)


def trace(x, /, *, offset=0, dtype=None):
    from .reductions import sum as _sum
    return _sum(diagonal(x, offset=offset), axis=-1, dtype=dtype)


def vecdot(x1, x2, /, *, axis=-1):
    from .ufunc_ops import vecdot as _vd
    return _vd(x1, x2, axis=axis)
