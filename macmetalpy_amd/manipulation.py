"""Array manipulation and small array routines, on the device.

The reference implements these as NumPy calls on the host
(manipulation.py:27-668, math_ext.py, set_ops.py, linalg_top.py).  Here
each is a view (shapes and strides over the same device buffer: flips,
splits, broadcasts, axis moves, diagonals) or a composition of the
device's strided copies (``mmp_copy_strided``: concatenate, tile, repeat,
roll), fused elementwise expressions (tril / triu, diff, outer, kron,
cross), reductions, the radix sort (unique, median, percentile, quantile)
and the gather kernels (``repeat`` with per-element counts).  NumPy's
shapes, dtypes and errors.
"""
from __future__ import annotations

import builtins

import numpy as np

from . import _elementwise as ew
from ._broadcasting import broadcast_shapes, broadcast_strides
from ._dtypes import resolve_dtype
from .ndarray import ndarray, _normalize_axis, _prod

__all__ = ["concatenate", "concat", "stack", "vstack", "hstack", "dstack", "column_stack",
           "split", "array_split", "hsplit", "vsplit", "dsplit", "unstack", "tile", "repeat",
           "flip", "fliplr", "flipud", "rot90", "roll", "broadcast_to", "broadcast_arrays",
           "moveaxis", "rollaxis", "swapaxes", "squeeze", "expand_dims", "atleast_1d",
           "atleast_2d", "atleast_3d", "diagonal", "diag", "trace", "tril", "triu", "copy",
           "copyto", "append", "ptp", "diff", "outer", "meshgrid", "cross", "kron", "tensordot",
           "average", "unique", "permute_dims", "matrix_transpose"]


def _asarray(a):
    from .creation import asarray
    return asarray(a)


def _dev(a):
    """Device-resident, evaluated ``a``."""
    a = _asarray(a)
    a._materialize_if_lazy()
    a._ensure_gpu()
    return a


def _view(a, shape, strides, offset):
    base = a._base if a._base is not None else a
    return ndarray(a._buffer, shape, a._dtype, strides=strides, offset=offset, base=base)


# ------------------------------------------------------------- joining
def concatenate(arrays, axis=0, out=None, *, dtype=None, casting="same_kind"):
    """Join arrays along an existing axis (None: flattened); one strided
    copy per input into its slab of the result."""
    arrs = [_asarray(a) for a in arrays]
    if not arrs:
        raise ValueError("need at least one array to concatenate")
    if axis is None:
        arrs = [a.ravel() for a in arrs]
        axis = 0
    nd = arrs[0].ndim
    if nd == 0:
        raise ValueError("zero-dimensional arrays cannot be concatenated")
    for a in arrs[1:]:
        if a.ndim != nd:
            raise ValueError("all the input array dimensions except for the concatenation axis "
                             f"must match exactly, but along dimension 0, the array at index 0 "
                             f"has {nd} dimension(s) and another array has {a.ndim} dimension(s)")
    axis = _normalize_axis(axis, nd)
    shape = list(arrs[0].shape)
    for a in arrs[1:]:
        for d in range(nd):
            if d != axis and a.shape[d] != shape[d]:
                raise ValueError("all the input array dimensions except for the concatenation "
                                 f"axis must match exactly, but along dimension {d}, the array "
                                 f"at index 0 has size {shape[d]} and another has size "
                                 f"{a.shape[d]}")
    shape[axis] = builtins.sum(a.shape[axis] for a in arrs)
    rdt = resolve_dtype(dtype) if dtype is not None else \
        resolve_dtype(np.result_type(*[a.dtype for a in arrs]))
    for a in arrs:
        if not np.can_cast(a.dtype, rdt, casting=casting):
            raise TypeError(f"Cannot cast array data from {a.dtype} to {rdt} according to the "
                            f"rule {casting!r}")
    if out is None:
        out = ndarray._empty_device(tuple(shape), rdt)
    elif tuple(out.shape) != tuple(shape):
        raise ValueError(f"Output array has wrong dimensionality / shape {out.shape}")
    off = 0
    for a in arrs:
        n = a.shape[axis]
        if n and out.size:
            out[(slice(None),) * axis + (slice(off, off + n),)] = a
        off += n
    return out


def concat(arrays, axis=0, *, dtype=None, casting="same_kind"):
    return concatenate(arrays, axis=axis, dtype=dtype, casting=casting)


def stack(arrays, axis=0, out=None, *, dtype=None, casting="same_kind"):
    arrs = [_asarray(a) for a in arrays]
    if not arrs:
        raise ValueError("need at least one array to stack")
    shp = arrs[0].shape
    if any(a.shape != shp for a in arrs):
        raise ValueError("all input arrays must have the same shape")
    axis = _normalize_axis(axis, len(shp) + 1)
    return concatenate([expand_dims(a, axis) for a in arrs], axis=axis, out=out, dtype=dtype,
                       casting=casting)


def vstack(tup, *, dtype=None, casting="same_kind"):
    return concatenate(atleast_2d(*tup) if len(tup) > 1 else [atleast_2d(*tup)], axis=0,
                       dtype=dtype, casting=casting)


def hstack(tup, *, dtype=None, casting="same_kind"):
    arrs = [atleast_1d(a) for a in tup]
    return concatenate(arrs, axis=0 if arrs and arrs[0].ndim == 1 else 1, dtype=dtype,
                       casting=casting)


def dstack(tup):
    return concatenate([atleast_3d(a) for a in tup], axis=2)


def column_stack(tup):
    arrs = []
    for a in tup:
        a = _asarray(a)
        arrs.append(a.reshape((a.size, 1)) if a.ndim < 2 else a)
    return concatenate(arrs, axis=1)


# ------------------------------------------------------------ splitting
def array_split(ary, indices_or_sections, axis=0):
    """Views of ``ary`` between the split points (uneven sections allowed)."""
    a = _asarray(ary)
    axis = _normalize_axis(axis, a.ndim)
    n = a.shape[axis]
    if isinstance(indices_or_sections, (int, np.integer)):
        k = int(indices_or_sections)
        if k <= 0:
            raise ValueError("number sections must be larger than 0.")
        each, extra = divmod(n, k)
        sizes = [each + 1] * extra + [each] * (k - extra)
        bounds = [0]
        for s in sizes:
            bounds.append(bounds[-1] + s)
    else:
        bounds = [0] + [int(i) for i in indices_or_sections] + [n]
    out = []
    for lo, hi in zip(bounds[:-1], bounds[1:]):
        out.append(a[(slice(None),) * axis + (slice(lo, hi),)])
    return out


def split(ary, indices_or_sections, axis=0):
    a = _asarray(ary)
    if isinstance(indices_or_sections, (int, np.integer)):
        if a.shape[_normalize_axis(axis, a.ndim)] % int(indices_or_sections):
            raise ValueError("array split does not result in an equal division")
    return array_split(a, indices_or_sections, axis)


def hsplit(ary, indices_or_sections):
    a = _asarray(ary)
    if a.ndim == 0:
        raise ValueError("hsplit only works on arrays of 1 or more dimensions")
    return split(a, indices_or_sections, 1 if a.ndim > 1 else 0)


def vsplit(ary, indices_or_sections):
    a = _asarray(ary)
    if a.ndim < 2:
        raise ValueError("vsplit only works on arrays of 2 or more dimensions")
    return split(a, indices_or_sections, 0)


def dsplit(ary, indices_or_sections):
    a = _asarray(ary)
    if a.ndim < 3:
        raise ValueError("dsplit only works on arrays of 3 or more dimensions")
    return split(a, indices_or_sections, 2)


def unstack(x, /, *, axis=0):
    a = _asarray(x)
    axis = _normalize_axis(axis, a.ndim)
    return tuple(a[(slice(None),) * axis + (i,)] for i in range(a.shape[axis]))


# ------------------------------------------------- tiling / repetition
def tile(A, reps):
    """One strided copy of a view that repeats ``A`` with stride-0 axes."""
    a = _dev(A)
    reps = (int(reps),) if isinstance(reps, (int, np.integer)) else tuple(int(r) for r in reps)
    d = builtins.max(a.ndim, len(reps))
    a = a.reshape((1,) * (d - a.ndim) + tuple(a.shape))
    reps = (1,) * (d - len(reps)) + reps
    if builtins.any(r < 0 for r in reps):
        raise ValueError("negative dimensions are not allowed")
    shape, strides = [], []
    for r, s, st in zip(reps, a.shape, a._strides):
        shape += [r, s]
        strides += [0, st]
    v = _view(a, tuple(shape), tuple(strides), a._offset)
    return v._contiguous_copy().reshape(tuple(r * s for r, s in zip(reps, a.shape)))


def repeat(a, repeats, axis=None):
    """Each element (slice along ``axis``) repeated; a scalar count is one
    strided copy, per-element counts a gather at searchsorted positions."""
    a = _dev(a)
    if axis is None:
        a, axis = a.ravel(), 0
    axis = _normalize_axis(axis, a.ndim)
    n = a.shape[axis]
    if isinstance(repeats, (int, np.integer)) or (
            not isinstance(repeats, ndarray) and np.ndim(repeats) == 0):
        r = int(repeats)
        if r < 0:
            raise ValueError("negative dimensions are not allowed")
        shape = list(a.shape[:axis + 1]) + [r] + list(a.shape[axis + 1:])
        strides = list(a._strides[:axis + 1]) + [0] + list(a._strides[axis + 1:])
        v = _view(a, tuple(shape), tuple(strides), a._offset)
        out_shape = list(a.shape)
        out_shape[axis] = n * r
        return v._contiguous_copy().reshape(tuple(out_shape))
    from . import reductions
    from .creation import arange
    from .sorting import searchsorted
    from .indexing import take
    rep = _asarray(repeats).astype(np.int64)
    if rep.size == 1:
        return repeat(a, int(rep.reshape(()).get()), axis)
    if rep.shape != (n,):
        raise ValueError(f"operands could not be broadcast together with shape ({n},) "
                         f"{tuple(rep.shape)}")
    if n and int(reductions.min(rep)) < 0:
        raise ValueError("negative dimensions are not allowed")
    ends = reductions.cumsum(rep)
    total = int(ends[n - 1]) if n else 0
    idx = searchsorted(ends, arange(total, dtype=np.int64), side="right")
    return take(a, idx, axis=axis)


# ----------------------------------------------------------------- views
def flip(m, axis=None):
    a = _asarray(m)
    axes = range(a.ndim) if axis is None else (
        (axis,) if isinstance(axis, (int, np.integer)) else tuple(axis))
    key = [slice(None)] * a.ndim
    for ax in axes:
        key[_normalize_axis(ax, a.ndim)] = slice(None, None, -1)
    return a[tuple(key)]


def fliplr(m):
    a = _asarray(m)
    if a.ndim < 2:
        raise ValueError("Input must be >= 2-d.")
    return flip(a, 1)


def flipud(m):
    a = _asarray(m)
    if a.ndim < 1:
        raise ValueError("Input must be >= 1-d.")
    return flip(a, 0)


def rot90(m, k=1, axes=(0, 1)):
    a = _asarray(m)
    ax0, ax1 = (_normalize_axis(x, a.ndim) for x in axes)
    if ax0 == ax1:
        raise ValueError("Axes must be different.")
    k %= 4
    if k == 0:
        return a[(slice(None),) * a.ndim]
    if k == 2:
        return flip(flip(a, ax0), ax1)
    perm = list(range(a.ndim))
    perm[ax0], perm[ax1] = perm[ax1], perm[ax0]
    if k == 1:
        return flip(a, ax1).transpose(perm)
    return flip(a.transpose(perm), ax1)


def roll(a, shift, axis=None):
    """Elements shifted cyclically: two strided copies per rolled axis."""
    x = _dev(a)
    if axis is None:
        return roll(x.ravel(), shift, 0).reshape(tuple(x.shape))
    shifts = (shift,) if isinstance(shift, (int, np.integer)) else tuple(shift)
    axes = (axis,) if isinstance(axis, (int, np.integer)) else tuple(axis)
    if len(shifts) == 1 and len(axes) > 1:
        shifts = shifts * len(axes)
    if len(axes) == 1 and len(shifts) > 1:
        axes = axes * len(shifts)
    if len(shifts) != len(axes):
        raise ValueError("'shift' and 'axis' should be scalars or 1D sequences")
    total = {}
    for sh, ax in zip(shifts, axes):
        ax = _normalize_axis(ax, x.ndim)
        total[ax] = total.get(ax, 0) + int(sh)
    out = x
    for ax, sh in total.items():
        n = out.shape[ax]
        if n == 0 or sh % n == 0:
            continue
        s = sh % n
        res = ndarray._empty_device(tuple(out.shape), out.dtype)
        pre = (slice(None),) * ax
        res[pre + (slice(s, None),)] = out[pre + (slice(0, n - s),)]
        res[pre + (slice(0, s),)] = out[pre + (slice(n - s, None),)]
        out = res
    return out if out is not x else x.copy()


def broadcast_to(array, shape, subok=False):
    a = _dev(array)
    shape = (int(shape),) if isinstance(shape, (int, np.integer)) else tuple(int(s) for s in shape)
    if broadcast_shapes(a.shape, shape) != shape:
        raise ValueError(f"operands could not be broadcast together with remapped shapes "
                         f"[original->remapped]: {a.shape} and requested shape {shape}")
    return _view(a, shape, tuple(broadcast_strides(a.shape, shape, a._strides)), a._offset)


def broadcast_arrays(*args, subok=False):
    arrs = [_asarray(a) for a in args]
    shape = broadcast_shapes(*[a.shape for a in arrs])
    return tuple(broadcast_to(a, shape) for a in arrs)


def moveaxis(a, source, destination):
    a = _asarray(a)
    src = [source] if isinstance(source, (int, np.integer)) else list(source)
    dst = [destination] if isinstance(destination, (int, np.integer)) else list(destination)
    src = [_normalize_axis(s, a.ndim) for s in src]
    dst = [_normalize_axis(d, a.ndim) for d in dst]
    if len(src) != len(dst):
        raise ValueError("`source` and `destination` arguments must have the same number of "
                         "elements")
    order = [n for n in range(a.ndim) if n not in src]
    for d, s in sorted(zip(dst, src)):
        order.insert(d, s)
    return a.transpose(order)


def rollaxis(a, axis, start=0):
    a = _asarray(a)
    axis = _normalize_axis(axis, a.ndim)
    if start < 0:
        start += a.ndim
    if not 0 <= start <= a.ndim:
        raise np.exceptions.AxisError(f"start={start} out of range")
    if axis < start:
        start -= 1
    if axis == start:
        return a[(slice(None),) * a.ndim]
    order = [n for n in range(a.ndim) if n != axis]
    order.insert(start, axis)
    return a.transpose(order)


def swapaxes(a, axis1, axis2):
    return _asarray(a).swapaxes(axis1, axis2)


def permute_dims(a, axes=None):
    return _asarray(a).transpose(axes)


def matrix_transpose(x):
    a = _asarray(x)
    if a.ndim < 2:
        raise ValueError("Input array must be at least 2-dimensional")
    return a.swapaxes(-1, -2)


def squeeze(a, axis=None):
    return _asarray(a).squeeze(axis)


def expand_dims(a, axis):
    a = _asarray(a)
    axes = (axis,) if isinstance(axis, (int, np.integer)) else tuple(axis)
    nd = a.ndim + len(axes)
    axes = sorted(_normalize_axis(x, nd) for x in axes)
    shape = list(a.shape)
    for x in axes:
        shape.insert(x, 1)
    return a.reshape(tuple(shape))


def _atleast(arys, n):
    res = []
    for a in arys:
        a = _asarray(a)
        if a.ndim < n:
            if n == 3:
                shape = {0: (1, 1, 1), 1: (1, a.size, 1), 2: tuple(a.shape) + (1,)}[a.ndim]
            else:
                shape = (1,) * (n - a.ndim) + tuple(a.shape)
            a = a.reshape(shape)
        res.append(a)
    return res[0] if len(res) == 1 else tuple(res)


def atleast_1d(*arys):
    return _atleast(arys, 1)


def atleast_2d(*arys):
    return _atleast(arys, 2)


def atleast_3d(*arys):
    return _atleast(arys, 3)


def diagonal(a, offset=0, axis1=0, axis2=1):
    """View of the diagonal (its own stride is the sum of the two axes')."""
    a = _dev(a)
    if a.ndim < 2:
        raise ValueError("diag requires an array of at least two dimensions")
    ax1, ax2 = _normalize_axis(axis1, a.ndim), _normalize_axis(axis2, a.ndim)
    if ax1 == ax2:
        raise ValueError("axis1 and axis2 cannot be the same")
    n1, n2 = a.shape[ax1], a.shape[ax2]
    s1, s2 = a._strides[ax1], a._strides[ax2]
    off = a._offset
    if offset >= 0:
        length = builtins.max(0, builtins.min(n1, n2 - offset))
        off += offset * s2 if length else 0
    else:
        length = builtins.max(0, builtins.min(n1 + offset, n2))
        off += -offset * s1 if length else 0
    keep = [d for d in range(a.ndim) if d not in (ax1, ax2)]
    return _view(a, tuple(a.shape[d] for d in keep) + (length,),
                 tuple(a._strides[d] for d in keep) + (s1 + s2,), off)


def diag(v, k=0):
    a = _dev(v)
    if a.ndim == 1:
        from .creation import zeros
        n = a.size + builtins.abs(k)
        out = zeros((n, n), dtype=a.dtype)
        if a.size:
            diagonal(out, k)[...] = a
        return out
    if a.ndim == 2:
        return diagonal(a, k).copy()
    raise ValueError("Input must be 1- or 2-d.")


def trace(a, offset=0, axis1=0, axis2=1, dtype=None, out=None):
    from .reductions import sum as _sum
    r = _sum(diagonal(a, offset, axis1, axis2), axis=-1, dtype=dtype)
    if out is not None:
        out[...] = r
        return out
    return r


def _tri_mask(shape, k, lower):
    from .creation import arange
    n, m = shape[-2], shape[-1]
    i = arange(n, dtype=np.int64).reshape((n, 1))
    j = arange(m, dtype=np.int64).reshape((1, m))
    return (j - i) <= k if lower else (j - i) >= k


def tril(m, k=0):
    a = _asarray(m)
    if a.ndim < 2:
        a = atleast_2d(a)
    return ew.where(_tri_mask(a.shape, k, True), a, 0)


def triu(m, k=0):
    a = _asarray(m)
    if a.ndim < 2:
        a = atleast_2d(a)
    return ew.where(_tri_mask(a.shape, k, False), a, 0)


def copy(a, order="K", subok=False):
    return _asarray(a).copy()


def copyto(dst, src, casting="same_kind", where=True):
    s = _asarray(src)
    if not np.can_cast(s.dtype, dst.dtype, casting=casting):
        raise TypeError(f"Cannot cast scalar from {s.dtype} to {dst.dtype} according to the "
                        f"rule {casting!r}")
    if where is True:
        dst[...] = s
    else:
        dst[...] = ew.where(where, s, dst)


def append(arr, values, axis=None):
    a, v = _asarray(arr), _asarray(values)
    if axis is None:
        return concatenate([a.ravel(), v.ravel()], axis=0)
    return concatenate([a, v], axis=axis)


# ------------------------------------------------------- small arithmetic
def ptp(a, axis=None, out=None, keepdims=False):
    from . import reductions
    r = reductions.max(a, axis=axis, keepdims=keepdims) - reductions.min(a, axis=axis,
                                                                          keepdims=keepdims)
    if out is not None:
        out[...] = r
        return out
    return r


def diff(a, n=1, axis=-1, prepend=np._NoValue, append=np._NoValue):
    a = _asarray(a)
    if n < 0:
        raise ValueError(f"order must be non-negative but got {n}")
    if n == 0:
        return a
    axis = _normalize_axis(axis, a.ndim)
    parts = []
    if prepend is not np._NoValue:
        p = _asarray(prepend)
        if p.ndim == 0:
            shp = list(a.shape)
            shp[axis] = 1
            p = broadcast_to(p, tuple(shp))
        parts.append(p)
    parts.append(a)
    if append is not np._NoValue:
        q = _asarray(append)
        if q.ndim == 0:
            shp = list(a.shape)
            shp[axis] = 1
            q = broadcast_to(q, tuple(shp))
        parts.append(q)
    if len(parts) > 1:
        a = concatenate(parts, axis=axis)
    hi = (slice(None),) * axis + (slice(1, None),)
    lo = (slice(None),) * axis + (slice(None, -1),)
    for _ in range(n):
        if a.dtype == np.bool_:
            a = ew.binary("ne_op", a[hi], a[lo])
        else:
            a = a[hi] - a[lo]
        a._materialize_if_lazy()
    return a


def outer(a, b, out=None):
    x, y = _asarray(a).ravel(), _asarray(b).ravel()
    r = x.reshape((x.size, 1)) * y.reshape((1, y.size))
    if out is not None:
        out[...] = r
        return out
    return r


def meshgrid(*xi, copy=True, sparse=False, indexing="xy"):
    """Coordinate arrays: broadcast views of the inputs, copied unless
    ``copy=False`` (NumPy's axis order for 'xy' and 'ij')."""
    if indexing not in ("xy", "ij"):
        raise ValueError("Valid values for `indexing` are 'xy' and 'ij'.")
    nd = len(xi)
    s0 = (1,) * nd
    outs = [_asarray(x).reshape(s0[:i] + (-1,) + s0[i + 1:]) for i, x in enumerate(xi)]
    if indexing == "xy" and nd > 1:
        outs[0] = outs[0].reshape((1, -1) + s0[2:])
        outs[1] = outs[1].reshape((-1, 1) + s0[2:])
    if not sparse:
        outs = list(broadcast_arrays(*outs))
    return tuple(o._contiguous_copy() if copy else o for o in outs)


def cross(a, b, axisa=-1, axisb=-1, axisc=-1, axis=None):
    """Cross product of 2- or 3-vectors along the last axis (fused)."""
    if axis is not None:
        axisa = axisb = axisc = axis
    x, y = moveaxis(_asarray(a), axisa, -1), moveaxis(_asarray(b), axisb, -1)
    if x.shape[-1] not in (2, 3) or y.shape[-1] not in (2, 3):
        raise ValueError("incompatible dimensions for cross product\n(dimension must be 2 or 3)")
    x0, x1 = x[..., 0], x[..., 1]
    y0, y1 = y[..., 0], y[..., 1]
    if x.shape[-1] == 2 and y.shape[-1] == 2:
        return x0 * y1 - x1 * y0
    x2 = x[..., 2] if x.shape[-1] == 3 else None
    y2 = y[..., 2] if y.shape[-1] == 3 else None
    c0 = (x1 * y2 - x2 * y1) if x2 is not None and y2 is not None else (
        x1 * y2 if x2 is None else -(x2 * y1))
    c1 = (x2 * y0 - x0 * y2) if x2 is not None and y2 is not None else (
        -(x0 * y2) if x2 is None else x2 * y0)
    c2 = x0 * y1 - x1 * y0
    r = stack([c0, c1, c2], axis=-1)
    return moveaxis(r, -1, axisc)


def kron(a, b):
    x, y = _asarray(a), _asarray(b)
    nd = builtins.max(x.ndim, y.ndim)
    x = x.reshape((1,) * (nd - x.ndim) + tuple(x.shape))
    y = y.reshape((1,) * (nd - y.ndim) + tuple(y.shape))
    xs = tuple(s for d in x.shape for s in (d, 1))
    ys = tuple(s for d in y.shape for s in (1, d))
    r = x.reshape(xs) * y.reshape(ys)
    return r.reshape(tuple(p * q for p, q in zip(x.shape, y.shape)))


def tensordot(a, b, axes=2):
    """Transposes and reshapes to one matmul (MFMA for float16/32)."""
    from .linalg_top import matmul
    x, y = _asarray(a), _asarray(b)
    if isinstance(axes, (int, np.integer)):
        n = int(axes)
        ax_a = list(range(x.ndim - n, x.ndim))
        ax_b = list(range(n))
    else:
        ax_a, ax_b = axes
        ax_a = [ax_a] if isinstance(ax_a, (int, np.integer)) else list(ax_a)
        ax_b = [ax_b] if isinstance(ax_b, (int, np.integer)) else list(ax_b)
    ax_a = [_normalize_axis(i, x.ndim) for i in ax_a]
    ax_b = [_normalize_axis(i, y.ndim) for i in ax_b]
    if len(ax_a) != len(ax_b) or builtins.any(x.shape[i] != y.shape[j] for i, j in zip(ax_a, ax_b)):
        raise ValueError("shape-mismatch for sum")
    free_a = [i for i in range(x.ndim) if i not in ax_a]
    free_b = [j for j in range(y.ndim) if j not in ax_b]
    k = _prod([x.shape[i] for i in ax_a])
    xa = x.transpose(free_a + ax_a).reshape((_prod([x.shape[i] for i in free_a]), k))
    yb = y.transpose(ax_b + free_b).reshape((k, _prod([y.shape[j] for j in free_b])))
    r = matmul(xa, yb)
    return r.reshape(tuple(x.shape[i] for i in free_a) + tuple(y.shape[j] for j in free_b))


def average(a, axis=None, weights=None, returned=False, *, keepdims=False):
    from . import reductions
    x = _asarray(a)
    if weights is None:
        avg = reductions.mean(x, axis=axis, keepdims=keepdims)
        if not returned:
            return avg
        from .creation import full
        scl = full(tuple(avg.shape), x.size / builtins.max(avg.size, 1), dtype=avg.dtype)
        return avg, scl
    w = _asarray(weights)
    if w.shape != x.shape:
        if axis is None:
            raise TypeError("Axis must be specified when shapes of a and weights differ.")
        if w.ndim != 1:
            raise TypeError("1D weights expected when shapes of a and weights differ.")
        ax = _normalize_axis(axis, x.ndim)
        if w.shape[0] != x.shape[ax]:
            raise ValueError("Length of weights not compatible with specified axis.")
        shp = [1] * x.ndim
        shp[ax] = w.shape[0]
        w = w.reshape(tuple(shp))
    rdt = np.result_type(x.dtype, w.dtype, np.float64 if x.dtype.kind in "iub" else x.dtype)
    wb = broadcast_to(w, x.shape) if w.shape != x.shape else w
    scl = reductions.sum(wb.astype(rdt), axis=axis, keepdims=keepdims)
    avg = reductions.sum(x.astype(rdt) * wb.astype(rdt), axis=axis, keepdims=keepdims) / scl
    return (avg, scl) if returned else avg


# ------------------------------------------------------------ set / stats
_UNIQUE_COUNT_MIN = 1 << 16      # from this size, integer unique may count instead of sort
_UNIQUE_COUNT_RANGE = 1 << 22    # value range counted (32 MiB of int64 counts at most)


def unique(ar, return_index=False, return_inverse=False, return_counts=False, axis=None,
           *, equal_nan=True):
    """Sorted unique elements of the flattened array (device sort, then the
    first element of each run of equal values); NaNs count as one value
    (equal_nan)."""
    if axis is not None:
        raise NotImplementedError("unique(axis=...) is not supported on the device")
    from .sorting import argsort
    from .indexing import _flat_nonzero, take
    from . import reductions
    from .creation import arange
    x = _dev(ar).ravel()
    n = x.size
    if n == 0:
        res = [x.copy()]
        if return_index:
            res.append(ndarray._empty_device((0,), np.int64))
        if return_inverse:
            res.append(ndarray._empty_device(tuple(_asarray(ar).shape), np.int64))
        if return_counts:
            res.append(ndarray._empty_device((0,), np.int64))
        return res[0] if len(res) == 1 else tuple(res)
    if (not return_index and not return_inverse and x.dtype.kind in "iu"
            and n >= _UNIQUE_COUNT_MIN):
        lo, hi = int(reductions.min(x)), int(reductions.max(x))
        if hi - lo < _UNIQUE_COUNT_RANGE:
            # small value range: counts per value (the counting kernel) give
            # the sorted distinct values and their counts exactly
            from .extras import bincount
            # offsets from the minimum: narrow signed inputs are widened
            # first (hi - lo may exceed their range, e.g. full-range int16)
            if x.dtype.kind == "i" and x.dtype.itemsize < 8:
                off = x.astype(np.int64) - lo
            else:
                off = x - lo if lo else x
            counts = bincount(off)
            nz = _flat_nonzero(counts != 0)
            # back in x's dtype: nz + lo fits it, so its wrapping add is exact
            # (and a uint64 minimum above the int64 range stays representable)
            vals = nz.astype(x.dtype)
            if lo:
                vals = vals + x.dtype.type(lo)
            return (vals, take(counts, nz)) if return_counts else vals
    perm = argsort(x, kind="stable")
    s = take(x, perm)
    first = ndarray._empty_device((n,), np.bool_)
    first[0:1] = True
    if n > 1:
        neq = ew.binary("ne_op", s[1:], s[:-1])
        if x.dtype.kind == "f" and equal_nan:
            neq = neq & ~(ew.unary("isnan_op", s[1:]) & ew.unary("isnan_op", s[:-1]))
        first[1:] = neq
    starts = _flat_nonzero(first)
    res = [take(s, starts)]
    if return_index:
        res.append(take(perm, starts))
    if return_inverse:
        run = reductions.cumsum(first) - 1
        inv = ndarray._empty_device((n,), np.int64)
        from .indexing import setitem
        setitem(inv, (perm,), run)
        inv = inv.reshape(tuple(_asarray(ar).shape)) if _asarray(ar).ndim > 1 else inv
        res.append(inv)
    if return_counts:
        ends = concatenate([starts[1:], _asarray(np.array([n], np.int64))]) if starts.size > 1 \
            else _asarray(np.array([n], np.int64))
        res.append(ends - starts)
    return res[0] if len(res) == 1 else tuple(res)
