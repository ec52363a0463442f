"""Advanced indexing and the indexing routines, on the device.

Replaces the reference's host paths: ``ndarray.__getitem__`` /
``__setitem__`` with integer or boolean arrays send the whole array to
NumPy (ndarray.py:874-891, 943-957), and indexing.py's take / put /
putmask / place / compress / extract / nonzero / flatnonzero / argwhere
run NumPy on the host (indexing.py:24-391).

Every advanced index follows NumPy's rules and is reduced to one array of
source offsets, built on the device with fused integer arithmetic:

* boolean arrays become the coordinates of their nonzero elements
  (``mmp_nonzero`` over the mask's inclusive count);
* integers next to index arrays count as 0-d index arrays;
* the index arrays broadcast together; their dimensions replace the
  indexed ones in place when the advanced indices are adjacent in the key,
  and come first otherwise;
* slices contribute ``start + step * arange(len)`` along their own result
  dimension.

Trailing whole, contiguous dimensions are folded into "rows" moved as a
unit, so ``a[idx]`` of a 2-D array moves whole rows.  One gather
(``mmp_gather``) or scatter (``mmp_scatter``) kernel then moves the data.
Indices are range-checked on the device (min / max) and raise IndexError
like NumPy's; negative indices wrap once.
"""
from __future__ import annotations

import math

import numpy as np

from ._backend import HipBackend
from ._dtypes import dtype_code
from . import _elementwise as ew
from .ndarray import ndarray, _prod, _normalize_axis

__all__ = ["take", "put", "take_along_axis", "put_along_axis", "putmask", "place", "compress",
           "extract", "nonzero", "flatnonzero", "argwhere"]

_I64 = np.dtype(np.int64)


def _asarray(x):
    from .creation import asarray
    return asarray(x)


def _is_index_array(k) -> bool:
    return isinstance(k, (ndarray, np.ndarray, list, tuple)) and not isinstance(k, str)


def _int_scalar(k) -> bool:
    return isinstance(k, (int, np.integer)) and not isinstance(k, (bool, np.bool_))


# ------------------------------------------------------------- nonzero
_MASK_TILE = 4096  # elements per tile of mmp_mask_tile_counts / mmp_mask_positions


def _flat_nonzero(mask: ndarray) -> ndarray:
    """int64 positions of the nonzero elements of ``mask`` in C order."""
    m = mask if mask._dtype == np.bool_ else (mask != 0)
    m = m.ravel()._ensure_contiguous()
    n = m.size
    if n == 0:
        return ndarray._empty_device((0,), _I64)
    be = HipBackend()
    tiles = -(-n // _MASK_TILE)
    incl = ndarray._empty_device((tiles,), np.dtype(np.uint64))  # selected count through each tile
    be.mask_tile_counts(n, m._ptr, incl._ptr)
    count = int(incl[tiles - 1])
    out = ndarray._empty_device((count,), _I64)
    if count:
        be.mask_positions(n, m._ptr, incl._ptr, out._ptr)
    return out


def _mask_compact(a: ndarray, mask: ndarray) -> ndarray:
    """``a[mask]`` for a boolean mask of a's shape: the selected elements
    in C order, packed on the device straight from the mask and the data."""
    m = mask.ravel()._ensure_contiguous()
    src = a.ravel()._ensure_contiguous()
    n = m.size
    if n == 0:
        return ndarray._empty_device((0,), a._dtype)
    be = HipBackend()
    tiles = -(-n // _MASK_TILE)
    incl = ndarray._empty_device((tiles,), np.dtype(np.uint64))
    be.mask_tile_counts(n, m._ptr, incl._ptr)
    count = int(incl[tiles - 1])
    out = ndarray._empty_device((count,), a._dtype)
    if count:
        be.mask_compact(a._dtype.itemsize, n, m._ptr, incl._ptr, src._ptr, out._ptr)
    return out


def _unravel(flat: ndarray, shape):
    """Coordinate arrays (int64) of C-order positions ``flat`` in ``shape``."""
    coords = []
    rest = _prod(shape)
    for s in shape:
        rest //= s
        c = flat // rest if rest > 1 else flat
        coords.append(c % s if s > 1 else c * 0)
    return coords


# ------------------------------------------------------- index arrays
def _norm_index(idx: ndarray, n: int, axis: int, mode: str = "raise") -> ndarray:
    """int64 indices into an axis of length ``n``, negatives wrapped once,
    out-of-range indices raising IndexError (mode 'raise') or wrapped /
    clipped (modes 'wrap' / 'clip', as np.take)."""
    from . import reductions
    if idx._dtype.kind not in "iu":
        if idx._dtype.kind == "b":
            raise IndexError("boolean index arrays are handled by their nonzero positions")
        raise IndexError("arrays used as indices must be of integer (or boolean) type")
    idx = idx.astype(_I64) if idx._dtype != _I64 else idx
    if idx.size == 0:
        return idx
    if mode == "wrap":
        return idx % n if n else idx
    if mode == "clip":
        if n == 0:
            raise IndexError("cannot do a non-empty take from an empty axes.")
        return ew.where(idx < 0, 0, ew.where(idx >= n, n - 1, idx))
    lo, hi = int(reductions.min(idx)), int(reductions.max(idx))
    if lo < -n or hi >= n:
        bad = lo if lo < -n else hi
        raise IndexError(f"index {bad} is out of bounds for axis {axis} with size {n}")
    if lo < 0:
        idx = ew.where(idx < 0, idx + n, idx)
    return idx


def _expand_key(a: ndarray, key):
    """Entries ('s', dim, slice) / ('a', dim, int64 ndarray or int) /
    ('n',) covering every dimension of ``a`` (NumPy's rules for Ellipsis,
    None and boolean arrays)."""
    if not isinstance(key, tuple):
        key = (key,)
    items = []
    for k in key:
        if isinstance(k, (bool, np.bool_)):
            raise NotImplementedError("scalar boolean indices are not supported on the device")
        if isinstance(k, ndarray) or _is_index_array(k):
            k = _asarray(k)
        items.append(k)
    consumed = 0
    for k in items:
        if isinstance(k, ndarray):
            consumed += k.ndim if k._dtype == np.bool_ else 1
        elif k is not None and k is not Ellipsis:
            consumed += 1
    if sum(1 for k in items if k is Ellipsis) > 1:
        raise IndexError("an index can only have a single ellipsis ('...')")
    if consumed > a.ndim:
        raise IndexError(f"too many indices for array: array is {a.ndim}-dimensional, "
                         f"but {consumed} were indexed")
    entries, dim = [], 0
    for k in items:
        if k is Ellipsis:
            for _ in range(a.ndim - consumed):
                entries.append(("s", dim, slice(None)))
                dim += 1
        elif k is None:
            entries.append(("n",))
        elif isinstance(k, slice):
            entries.append(("s", dim, k))
            dim += 1
        elif isinstance(k, ndarray) and k._dtype == np.bool_:
            shp = a.shape[dim:dim + k.ndim]
            if k.ndim == 0:
                raise NotImplementedError("0-d boolean indices are not supported on the device")
            if tuple(k.shape) != tuple(shp):
                for j, (ms, s) in enumerate(zip(k.shape, shp)):
                    if ms != s:
                        raise IndexError(f"boolean index did not match indexed array along "
                                         f"axis {dim + j}; size of axis is {s} but size of "
                                         f"corresponding boolean axis is {ms}")
            pos = _flat_nonzero(k)
            for j, c in enumerate(_unravel(pos, shp)):
                entries.append(("a", dim + j, c))
            dim += k.ndim
        elif isinstance(k, ndarray):
            entries.append(("a", dim, k))
            dim += 1
        elif _int_scalar(k):
            entries.append(("a", dim, int(k)))
            dim += 1
        else:
            raise IndexError("only integers, slices (`:`), ellipsis (`...`), numpy.newaxis "
                             "(`None`) and integer or boolean arrays are valid indices")
    while dim < a.ndim:
        entries.append(("s", dim, slice(None)))
        dim += 1
    return entries


class _Plan:
    """Offsets (int64, C-order over the indexed result dims) of the first
    element of each row, the result shape and the row layout."""

    def __init__(self, a: ndarray, key, mode="raise"):
        entries = _expand_key(a, key)
        shape, strides = a.shape, a._strides
        # normalise the advanced indices
        adv = []
        for pos, e in enumerate(entries):
            if e[0] != "a":
                continue
            _, d, v = e
            if isinstance(v, int):
                n = shape[d]
                if mode == "raise" and not -n <= v < n:
                    raise IndexError(f"index {v} is out of bounds for axis {d} with size {n}")
                v = v % n if n else v
            else:
                v = _norm_index(v, shape[d], d, mode)
            adv.append((pos, d, v))
        if not adv:
            raise IndexError("advanced indexing needs an integer or boolean array index")
        from ._broadcasting import broadcast_shapes
        bshape = broadcast_shapes(*[() if isinstance(v, int) else v.shape for _, _, v in adv])
        positions = [p for p, _, _ in adv]
        adjacent = positions == list(range(positions[0], positions[0] + len(positions)))
        # fold trailing whole contiguous dims into rows
        row_elems, tail = 1, len(entries)
        while tail > 0:
            e = entries[tail - 1]
            if e[0] != "s":
                break
            d = e[1]
            start, stop, step = e[2].indices(shape[d])
            if not (start == 0 and step == 1 and stop == shape[d] and strides[d] == row_elems
                    or shape[d] == 1 and start == 0 and stop == 1):
                break
            row_elems *= shape[d]
            tail -= 1
        # result dims of the non-folded entries
        dims, placed = [], False          # (kind, entry) per result dim group
        if not adjacent:
            dims.append(("B", None))
            placed = True
        for e in entries[:tail]:
            if e[0] == "a":
                if not placed:
                    dims.append(("B", None))
                    placed = True
            else:
                dims.append((e[0], e))
        rshape = []
        bpos = 0
        for kind, e in dims:
            if kind == "B":
                bpos = len(rshape)
                rshape.extend(bshape)
            elif kind == "n":
                rshape.append(1)
            else:
                rshape.append(len(range(*e[2].indices(shape[e[1]]))))
        self.rshape = tuple(rshape)
        self.row_shape = tuple(shape[e[1]] for e in entries[tail:])
        self.row_elems = row_elems
        # word size: every offset is a multiple of g elements
        g = a._offset
        for e in entries[:tail]:
            if e[0] == "s":
                start, _, step = e[2].indices(shape[e[1]])
                g = math.gcd(math.gcd(g, strides[e[1]] * step), strides[e[1]] * start)
            elif e[0] == "a":
                g = math.gcd(g, strides[e[1]])
        g = math.gcd(g, row_elems) if g else row_elems
        isz = a._dtype.itemsize
        word = 16
        while word > 1 and ((g * isz) % word or (row_elems * isz) % word):
            word //= 2
        step_el = max(1, word // isz)     # offsets are counted in steps of step_el elements
        self.word, self.unit = word, max(1, isz // word)
        self.row_words = row_elems * isz // word
        # offsets: base + sum of broadcast contributions
        nd = len(rshape)
        terms = []
        rdim = 0
        for kind, e in dims:
            if kind == "B":
                for _, d, v in adv:
                    st = strides[d] // step_el
                    if isinstance(v, int):
                        terms.append(v * st)
                        continue
                    vs = (1,) * (len(bshape) - v.ndim) + tuple(v.shape)
                    shp = (1,) * bpos + vs + (1,) * (nd - bpos - len(bshape))
                    terms.append(v.reshape(shp) * st if st != 1 else v.reshape(shp))
                rdim += len(bshape)
            elif kind == "n":
                rdim += 1
            else:
                d = e[1]
                start, stop, step = e[2].indices(shape[d])
                length = rshape[rdim]
                if length > 1:
                    from .creation import arange
                    shp = (1,) * rdim + (length,) + (1,) * (nd - rdim - 1)
                    st = strides[d] * step // step_el
                    terms.append(arange(0, length, dtype=np.int64).reshape(shp) * st)
                terms.append(start * strides[d] // step_el)
                rdim += 1
        base = a._offset // step_el
        off = None
        scal = base
        for t in terms:
            if isinstance(t, int):
                scal += t
            else:
                off = t if off is None else off + t
        if off is None:
            off = _asarray(np.full(rshape, scal, dtype=np.int64))
        elif scal:
            off = off + scal
        if tuple(off.shape) != self.rshape:
            off = off._broadcast_copy(self.rshape, _I64)
        self.offsets = off._ensure_contiguous() if off._dtype == _I64 else off.astype(_I64)._ensure_contiguous()
        self.n = _prod(self.rshape)


def _row_index(a: ndarray, key):
    """The index array when ``key`` is one integer array on axis 0 followed
    only by whole slices and ``a`` has contiguous rows, else None."""
    items = key if isinstance(key, tuple) else (key,)
    if not items or a.ndim == 0 or a._strides[0] < 0:
        return None
    k0 = items[0]
    if not isinstance(k0, (ndarray, np.ndarray, list)):
        return None
    if any(not (isinstance(k, slice) and k == slice(None)) for k in items[1:]):
        return None
    if len(items) > a.ndim:
        return None
    from ._fusion import _c_contig_strides
    if tuple(a._strides[1:]) != _c_contig_strides(a.shape[1:]):
        return None
    idx = _asarray(k0)
    return idx if idx._dtype.kind in "iu" else None


def _gather_rows(a: ndarray, idx: ndarray) -> ndarray:
    """a[idx] along axis 0 with the raw indices: the kernel wraps negative
    indices and flags out-of-range ones, so no offset array and no bounds
    reductions are needed (the message is worked out only on error)."""
    be = HipBackend()
    isz = a._dtype.itemsize
    rows = a.shape[1:]
    rowbytes = _prod(rows) * isz
    off_b, st_b = a._offset * isz, a._strides[0] * isz
    word = 16
    while word > 1 and (rowbytes % word or st_b % word or off_b % word):
        word //= 2
    ix = idx.astype(_I64) if idx._dtype != _I64 else idx
    ix = ix._ensure_contiguous()
    out = ndarray._empty_device(tuple(idx.shape) + tuple(rows), a._dtype)
    if out.size == 0:
        if ix.size and a.shape[0] == 0:
            raise IndexError(f"index {int(ix.ravel()[0])} is out of bounds for axis 0 with size 0")
        return out
    flag = ndarray._empty_device((1,), np.uint32)
    be.fill(dtype_code(flag._dtype), 1, np.zeros(1, np.uint32), flag._ptr)
    be.gather(word, a._buffer.ptr + off_b, a._buffer.nbytes - off_b, ix._ptr, st_b // word,
              ix.size, rowbytes // word, out._ptr, wrap=a.shape[0], flag=flag._ptr)
    if int(flag.get()[0]):
        _norm_index(ix, a.shape[0], 0)  # raises NumPy's IndexError
    return out


def getitem(a: ndarray, key, mode: str = "raise") -> ndarray:
    """``a[key]`` for keys with integer or boolean arrays (a new array);
    ``mode`` treats out-of-range indices as np.take does."""
    a._materialize_if_lazy()
    a._ensure_gpu()
    if (mode == "raise" and isinstance(key, ndarray) and key._dtype == np.bool_ and key.ndim
            and tuple(key.shape) == tuple(a.shape) and a._dtype.itemsize in (1, 2, 4, 8)):
        return _mask_compact(a, key)
    if mode == "raise":
        idx = _row_index(a, key)
        if idx is not None:
            return _gather_rows(a, idx)
    plan = _Plan(a, key, mode)
    out = ndarray._empty_device(plan.rshape + plan.row_shape, a._dtype)
    if out.size:
        HipBackend().gather(plan.word, a._buffer.ptr, a._buffer.nbytes, plan.offsets._ptr,
                            plan.unit, plan.n, plan.row_words, out._ptr)
    return out


def setitem(a: ndarray, key, value) -> None:
    """``a[key] = value`` for keys with integer or boolean arrays."""
    a._materialize_if_lazy()
    a._ensure_gpu()
    plan = _Plan(a, key)
    target = plan.rshape + plan.row_shape
    if _prod(target) == 0:
        return
    v = _asarray(value)
    vshape = tuple(v.shape)
    while len(vshape) > len(target) and vshape[0] == 1:   # NumPy drops leading 1s
        vshape = vshape[1:]
    from ._broadcasting import broadcast_shapes
    try:
        if len(vshape) > len(target):
            raise ValueError
        broadcast_shapes(vshape, target)
    except ValueError:
        raise ValueError(f"shape mismatch: value array of shape {tuple(v.shape)} could not be "
                         f"broadcast to indexing result of shape {target}") from None
    vshape = (1,) * (len(target) - len(vshape)) + vshape
    v = v.reshape(vshape)
    nlead = len(plan.rshape)
    if all(x == 1 for x in vshape[:nlead]):
        # one value row for every target row
        src = v.reshape(vshape[nlead:])._broadcast_copy(plan.row_shape, a._dtype)
        src_rows = 1
    else:
        src = v._broadcast_copy(target, a._dtype)
        src_rows = plan.n
    ew.flush_lazy(a._buffer)
    HipBackend().scatter(plan.word, a._buffer.ptr, a._buffer.nbytes, plan.offsets._ptr,
                         plan.unit, plan.n, plan.row_words, src._ptr, src_rows)


# ------------------------------------------------------------- routines
def nonzero(a):
    """Tuple of int64 coordinate arrays of the nonzero elements (reference
    indexing.py:370-374)."""
    a = _asarray(a)
    if a.ndim == 0:
        raise ValueError("Calling nonzero on 0d arrays is not allowed. Use np.atleast_1d(scalar).nonzero() instead.")
    pos = _flat_nonzero(a)
    return tuple(c._ensure_contiguous() if isinstance(c, ndarray) else c
                 for c in _unravel(pos, a.shape))


def flatnonzero(a):
    """int64 positions of the nonzero elements of ``a.ravel()`` (reference
    indexing.py:377-381)."""
    return _flat_nonzero(_asarray(a))


def argwhere(a):
    """(count, ndim) int64 coordinates of the nonzero elements (reference
    indexing.py:384-388)."""
    a = _asarray(a)
    if a.ndim == 0:
        pos = _flat_nonzero(a.reshape((1,)))
        return ndarray._empty_device((pos.size, 0), _I64)
    coords = nonzero(a)
    out = ndarray._empty_device((coords[0].size, a.ndim), _I64)
    for d, c in enumerate(coords):
        out[:, d] = c
    return out


def take(a, indices, axis=None, out=None, mode="raise"):
    """Elements of ``a`` (flattened when ``axis`` is None) at ``indices``
    along ``axis``; modes 'raise', 'wrap', 'clip' as np.take (reference
    indexing.py:24-100)."""
    if mode not in ("raise", "wrap", "clip"):
        raise ValueError(f"clipmode not understood: {mode!r}")
    a = _asarray(a)
    if axis is None:
        a = a.ravel()
        axis = 0
    axis = _normalize_axis(axis, a.ndim)
    idx = _asarray(np.asarray(indices, dtype=np.int64)) if _int_scalar(indices) else _asarray(indices)
    if idx._dtype.kind not in "iu":
        raise TypeError("Cannot cast array data from dtype('{}') to dtype('int64') according to "
                        "the rule 'safe'".format(idx._dtype))
    r = getitem(a, (slice(None),) * axis + (idx,), mode)
    if out is not None:
        out[...] = r
        return out
    return r


def put(a, ind, v, mode="raise"):
    """``a.flat[ind] = v``, ``v`` repeated as needed (reference
    indexing.py:103-163).  Modifies ``a`` in place."""
    if mode not in ("raise", "wrap", "clip"):
        raise ValueError(f"clipmode not understood: {mode!r}")
    if not isinstance(a, ndarray):
        raise TypeError("put: first argument must be a device ndarray")
    idx = _asarray(np.asarray(ind, dtype=np.int64) if not isinstance(ind, ndarray) else ind).ravel()
    n = a.size
    if idx.size == 0:
        return None
    idx = _norm_index(idx, n, 0, mode)
    vals = _asarray(v).ravel()
    if vals.size == 0:
        return None
    if vals.size != idx.size:
        from .creation import arange
        vals = take(vals, arange(idx.size, dtype=np.int64) % vals.size)
    setitem(a, tuple(_unravel(idx, a.shape)), vals)
    return None


def _along_axis_key(arr: ndarray, indices: ndarray, axis: int):
    from .creation import arange
    key = []
    for d in range(arr.ndim):
        if d == axis:
            key.append(indices)
        else:
            shp = [1] * arr.ndim
            shp[d] = arr.shape[d]
            key.append(arange(arr.shape[d], dtype=np.int64).reshape(tuple(shp)))
    return tuple(key)


def take_along_axis(arr, indices, axis):
    """np.take_along_axis on the device (reference indexing.py:93-100)."""
    arr = _asarray(arr)
    indices = _asarray(indices)
    if axis is None:
        arr, axis = arr.ravel(), 0
    axis = _normalize_axis(axis, arr.ndim)
    if indices.ndim != arr.ndim:
        raise ValueError("`indices` and `arr` must have the same number of dimensions")
    return getitem(arr, _along_axis_key(arr, indices, axis))


def put_along_axis(arr, indices, values, axis):
    """np.put_along_axis on the device (reference indexing.py:166-176)."""
    indices = _asarray(indices)
    axis = _normalize_axis(axis, arr.ndim)
    if indices.ndim != arr.ndim:
        raise ValueError("`indices` and `arr` must have the same number of dimensions")
    setitem(arr, _along_axis_key(arr, indices, axis), values)
    return None


def compress(condition, a, axis=None, out=None):
    """Slices of ``a`` along ``axis`` where ``condition`` is true (reference
    indexing.py:221-231)."""
    a = _asarray(a)
    cond = _asarray(condition)
    if cond.ndim != 1:
        raise ValueError("condition must be a 1-d array")
    if axis is None:
        a, axis = a.ravel(), 0
    axis = _normalize_axis(axis, a.ndim)
    if cond.size > a.shape[axis]:
        raise IndexError(f"index {cond.size - 1} is out of bounds for axis {axis} with size "
                         f"{a.shape[axis]}")
    r = take(a, _flat_nonzero(cond), axis=axis)
    if out is not None:
        out[...] = r
        return out
    return r


def extract(condition, arr):
    """``arr.ravel()[condition.ravel() != 0]`` (reference indexing.py:242-248)."""
    arr = _asarray(arr)
    cond = _asarray(condition).ravel()
    if cond.size != arr.size:
        raise ValueError("extract: condition and arr must have the same size")
    return take(arr.ravel(), _flat_nonzero(cond))


def putmask(a, mask, values):
    """``a.flat[i] = values[i % len(values)]`` where ``mask.flat[i]``
    (reference indexing.py:179-189)."""
    mask = _asarray(mask)
    if tuple(mask.shape) != tuple(a.shape):
        raise ValueError("putmask: mask and data must be the same size")
    pos = _flat_nonzero(mask)
    if pos.size == 0:
        return None
    vals = _asarray(values).ravel()
    if vals.size == 0:
        return None
    sel = take(vals, pos % vals.size)
    setitem(a, tuple(_unravel(pos, a.shape)), sel)
    return None


def place(arr, mask, vals):
    """The first N of ``vals`` (repeated) go where ``mask`` is true, N = the
    number of true elements (reference indexing.py:192-202)."""
    mask = _asarray(mask)
    if mask.size != arr.size:
        raise ValueError("place: mask and data must be the same size")
    pos = _flat_nonzero(mask)
    if pos.size == 0:
        return None
    v = _asarray(vals).ravel()
    if v.size == 0:
        raise ValueError("Cannot insert from an empty array!")
    if v.size != pos.size:
        from .creation import arange
        v = take(v, arange(pos.size, dtype=np.int64) % v.size)
    setitem(arr, tuple(_unravel(pos, arr.shape)), v)
    return None
