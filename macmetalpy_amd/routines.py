"""More NumPy routines composed of device ops: einsum, pad, insert / delete,
multi-dimensional histograms, bit packing, polynomials, window functions,
i0, unwrap, the array-API unique family, index tricks (mgrid, ogrid, r_,
c_), block, apply_along_axis / apply_over_axes and small array helpers.

The reference wraps NumPy on the host for all of these (index_tricks.py,
window.py, poly_ops.py, functional.py, manipulation.py, math_ext.py,
set_ops.py).  Here array data stays on the device; only control data --
index maps of a few entries per axis, polynomial coefficients read once,
bin edges -- is computed on the host, with NumPy's own formulas.
"""
from __future__ import annotations

import builtins
from collections import namedtuple

import numpy as np

from . import _elementwise as ew
from .ndarray import ndarray, _normalize_axis, _prod

__all__ = ["einsum", "einsum_path", "pad", "insert", "delete", "diagflat", "ediff1d",
           "histogramdd", "histogram2d", "packbits", "unpackbits", "poly", "polyval", "polyadd",
           "polysub", "polymul", "polydiv", "polyder", "polyint", "polyfit", "roots", "poly1d",
           "bartlett", "blackman", "hamming", "hanning", "kaiser", "i0", "unwrap",
           "unique_all", "unique_counts", "unique_inverse", "unique_values", "mgrid", "ogrid",
           "r_", "c_", "s_", "index_exp", "block", "apply_along_axis", "apply_over_axes",
           "resize", "trim_zeros", "isposinf", "isneginf", "mask_indices", "asanyarray",
           "asarray_chkfinite", "asfortranarray", "require", "astype", "broadcast_shapes",
           "fastCopyAndTranspose", "row_stack", "trapz", "isnat"]

s_ = np.s_
index_exp = np.index_exp
broadcast_shapes = np.broadcast_shapes


def _asarray(a, dtype=None):
    from .creation import asarray
    return asarray(a, dtype=dtype) if dtype is not None else asarray(a)


def _host(a):
    """Host copy of small control data (index lists, coefficients)."""
    return a.get() if isinstance(a, ndarray) else np.asarray(a)


# ================================================================ einsum
_LETTERS = "ABCDEFGHIJKLMNOPQRSTUVWXYZabcdefghijklmnopqrstuvwxyz"


def _parse_einsum(subscripts, shapes):
    """Subscripts with the ellipsis expanded into fresh letters (the
    rightmost ellipsis dimensions aligned across operands) and the output
    spec (implicit mode: ellipsis first, then the letters seen once, in
    alphabetical order)."""
    sub = subscripts.replace(" ", "")
    if "->" in sub:
        lhs, out = sub.split("->")
        explicit = True
    else:
        lhs, out, explicit = sub, "", False
    specs = lhs.split(",")
    if len(specs) != len(shapes):
        raise ValueError("more operands provided to einstein sum function than specified in the "
                         "subscripts string" if len(shapes) > len(specs) else
                         "fewer operands provided to einstein sum function than specified in the "
                         "subscripts string")
    used = set(c for c in sub if c.isalpha())
    free = [c for c in _LETTERS if c not in used]
    ell = 0
    for sp, shp in zip(specs, shapes):
        if "..." in sp:
            ell = builtins.max(ell, len(shp) - (len(sp) - 3))
    eletters = "".join(free[:ell])
    full = []
    for sp, shp in zip(specs, shapes):
        if "..." in sp:
            k = len(shp) - (len(sp) - 3)
            if k < 0:
                raise ValueError("operand has more dimensions than subscripts given in einstein sum")
            sp = sp.replace("...", eletters[ell - k:] if k else "")
        if len(sp) != len(shp):
            raise ValueError(f"operand has more dimensions than subscripts given in einstein sum, "
                             f"but no '...' ellipsis provided to broadcast the extra dimensions."
                             if len(shp) > len(sp) else
                             "einstein sum subscripts string contains too many subscripts for "
                             "operand")
        full.append(sp)
    if explicit:
        out = out.replace("...", eletters)
    else:
        counts = {}
        for sp in full:
            for c in sp:
                counts[c] = counts.get(c, 0) + 1
        out = eletters + "".join(sorted(c for c, n in counts.items()
                                        if n == 1 and c not in eletters))
    for c in out:
        if not any(c in sp for sp in full):
            raise ValueError(f"einstein sum subscripts string included output subscript '{c}' "
                             "which never appeared in an input")
    return full, out


def _einsum_diag(a, sp):
    """Repeated letters of one operand: keep their diagonal (moved last)."""
    from .manipulation import diagonal
    while True:
        rep = next((c for c in sp if sp.count(c) > 1), None)
        if rep is None:
            return a, sp
        i = sp.index(rep)
        j = sp.index(rep, i + 1)
        a = diagonal(a, 0, i, j)
        sp = "".join(c for k, c in enumerate(sp) if k not in (i, j)) + rep


def _einsum_sum(a, sp, keep, dt):
    from .reductions import sum as _sum
    drop = tuple(k for k, c in enumerate(sp) if c not in keep)
    if not drop:
        return a, sp
    r = _sum(a, axis=drop, dtype=dt)
    return _asarray(r), "".join(c for c in sp if c in keep)


def einsum(subscripts, *operands, out=None, dtype=None, order="K", casting="safe",
           optimize=False):
    """Einstein summation: diagonals as strided views, letters seen by one
    operand only summed away, each pair of operands contracted by one
    batched matmul (batch letters, kept letters, contracted letters),
    and the result transposed to the output order."""
    from .linalg_top import matmul
    from .manipulation import broadcast_to
    if not isinstance(subscripts, str):
        raise NotImplementedError("einsum's interleaved (operand, sublist) form is not supported")
    ops = [_asarray(o) for o in operands]
    rdt = np.result_type(*[o.dtype for o in ops]) if dtype is None else np.dtype(dtype)
    for o in ops:
        if not np.can_cast(o.dtype, rdt, casting=casting):
            raise TypeError(f"Cannot cast array data from {o.dtype!r} to {rdt!r} according to "
                            f"the rule '{casting}'")
    specs, outspec = _parse_einsum(subscripts, [tuple(o.shape) for o in ops])
    sizes = {}
    for o, sp in zip(ops, specs):
        for c, n in zip(sp, o.shape):
            if sizes.get(c, 1) == 1:
                sizes[c] = n
            elif n not in (1, sizes[c]):
                raise ValueError(f"operands could not be broadcast together with remapped shapes "
                                 f"(letter {c!r}: {sizes[c]} vs {n})")
    work = []
    for k, (o, sp) in enumerate(zip(ops, specs)):
        a = o.astype(rdt) if o.dtype != rdt else o
        a, sp = _einsum_diag(a, sp)
        later = set(outspec).union(*[set(s) for j, s in enumerate(specs) if j != k])
        a, sp = _einsum_sum(a, sp, later, rdt)
        work.append((a, sp))

    a, sa = work[0]
    for idx in builtins.range(1, len(work)):
        b, sb = work[idx]
        rest = set(outspec).union(*[set(s) for _, s in work[idx + 1:]])
        batch = [c for c in sa if c in sb and c in rest]
        contract = [c for c in sa if c in sb and c not in rest]
        left = [c for c in sa if c not in sb]
        right = [c for c in sb if c not in sa]
        pa = [sa.index(c) for c in batch + left + contract]
        pb = [sb.index(c) for c in batch + contract + right]
        A = a.transpose(pa) if pa != list(builtins.range(len(pa))) else a
        B = b.transpose(pb) if pb != list(builtins.range(len(pb))) else b
        ta = tuple(sizes[c] for c in batch + left + contract)
        tb = tuple(sizes[c] for c in batch + contract + right)
        if tuple(A.shape) != ta:
            A = broadcast_to(A, ta)
        if tuple(B.shape) != tb:
            B = broadcast_to(B, tb)
        nb = _prod([sizes[c] for c in batch])
        nl = _prod([sizes[c] for c in left])
        nk = _prod([sizes[c] for c in contract])
        nr = _prod([sizes[c] for c in right])
        A3 = A._ensure_contiguous().reshape((nb, nl, nk))
        B3 = B._ensure_contiguous().reshape((nb, nk, nr))
        if nk == 0 or nb * nl * nr == 0:
            from .creation import zeros
            C = zeros((nb, nl, nr), dtype=rdt)
        else:
            C = matmul(A3, B3)
            if C.dtype != rdt:
                C = C.astype(rdt)
        a = C.reshape(tuple(sizes[c] for c in batch + left + right))
        sa = "".join(batch + left + right)
        a, sa = _einsum_sum(a, sa, rest, rdt)

    a, sa = _einsum_sum(a, sa, set(outspec), rdt)
    shp = tuple(sizes[c] for c in sa)
    if tuple(a.shape) != shp:
        a = broadcast_to(a, shp)
    perm = [sa.index(c) for c in outspec]
    r = a.transpose(perm) if perm != list(builtins.range(len(perm))) else a
    r = r.copy() if r.ndim else r.reshape(())
    if r.dtype != rdt:
        r = r.astype(rdt)
    if out is not None:
        out[...] = r
        return out
    return r


def einsum_path(subscripts, *operands, optimize="greedy", einsum_call=False):
    """NumPy's contraction-order search, run on zero-stride stand-ins of
    the operands' shapes (it reads nothing but shapes)."""
    dummies = [np.broadcast_to(np.zeros((), dtype=o.dtype if isinstance(o, ndarray)
                                        else np.asarray(o).dtype), tuple(np.shape(o)
                                        if not isinstance(o, ndarray) else o.shape))
               for o in operands]
    return np.einsum_path(subscripts, *dummies, optimize=optimize, einsum_call=einsum_call)


# =================================================================== pad
def _pad_index(n, before, after, mode):
    """Source index along one axis for every padded position (host, length
    n + before + after): reflect / symmetric / wrap are periodic extensions
    (period 2(n-1), 2n, n), edge repeats the ends."""
    pos = np.arange(-before, n + after, dtype=np.int64)
    if mode == "edge" or (mode == "reflect" and n == 1):
        return np.clip(pos, 0, n - 1)
    if mode == "wrap":
        return pos % n
    if mode == "reflect":
        p = 2 * (n - 1)
        m = pos % p
        return np.where(m < n, m, p - m)
    if mode == "symmetric":
        p = 2 * n
        m = pos % p
        return np.where(m < n, m, p - 1 - m)
    raise AssertionError(mode)


def _pairs(v, ndim, name):
    arr = np.asarray(v.get() if isinstance(v, ndarray) else v)
    try:
        return np.broadcast_to(arr, (ndim, 2))
    except ValueError:
        raise ValueError(f"operands could not be broadcast together with remapped shapes "
                         f"[original->remapped]: {arr.shape} and requested shape ({ndim},2)") from None


def _scalar_pairs(v, ndim):
    """Per-axis (before, after) values typed as NumPy's pad sees them: one
    or two given values stay NumPy scalars, a full table becomes Python
    scalars (which promote weakly)."""
    x = np.array(v.get() if isinstance(v, ndarray) else v)
    if x.ndim < 3:
        if x.size == 1:
            s = x.ravel()[0]
            return [(s, s)] * ndim
        if x.size == 2 and x.shape != (2, 1):
            x = x.ravel()
            return [(x[0], x[1])] * ndim
    return np.broadcast_to(x, (ndim, 2)).tolist()


def pad(array, pad_width, mode="constant", **kwargs):
    """NumPy's pad: axes are padded in order, each over the already padded
    extent of earlier axes (so corners take the later axis' rule).
    constant / maximum / minimum / mean / linear_ramp fill regions; edge,
    reflect, symmetric and wrap are gathers through per-axis index maps."""
    from .indexing import take
    from . import reductions
    a = _asarray(array)
    nd = a.ndim
    pw = _pairs(pad_width, nd, "pad_width").astype(np.int64)
    if (pw < 0).any():
        raise ValueError("index can't contain negative values")
    if callable(mode):
        raise NotImplementedError("pad with a callable mode is not supported on the device")
    if mode in ("edge", "wrap", "reflect", "symmetric"):
        if kwargs.get("reflect_type", "even") != "even":
            raise NotImplementedError("pad(reflect_type='odd') is not supported on the device")
        r = a
        for ax in builtins.range(nd):
            b, e = int(pw[ax, 0]), int(pw[ax, 1])
            if b == 0 and e == 0:
                continue
            n = a.shape[ax]
            if n == 0:
                raise ValueError(f"can't extend empty axis {ax} using modes other than 'constant' "
                                 "or 'empty'")
            idx = _pad_index(n, b, e, mode)
            r = take(r, _asarray(idx), axis=ax)
        return r.copy() if r is a else r
    if mode not in ("constant", "empty", "maximum", "minimum", "mean", "linear_ramp", "median"):
        raise ValueError(f"mode '{mode}' is not supported")
    if mode == "median":
        raise NotImplementedError("pad(mode='median') is not supported on the device")
    new_shape = tuple(int(n + pw[k, 0] + pw[k, 1]) for k, n in enumerate(a.shape))
    out = ndarray._empty_device(new_shape, a.dtype)
    orig = tuple(slice(int(pw[k, 0]), int(pw[k, 0]) + a.shape[k]) for k in builtins.range(nd))
    if a.size:
        out[orig] = a
    if mode == "empty":
        return out
    if mode == "constant":
        cv = _pairs(kwargs.get("constant_values", 0), nd, "constant_values")
    elif mode == "linear_ramp":
        ev = _scalar_pairs(kwargs.get("end_values", 0), nd)
    else:
        sl = kwargs.get("stat_length", None)
        st = None if sl is None else _pairs(sl, nd, "stat_length")
    for ax in builtins.range(nd):
        b, e = int(pw[ax, 0]), int(pw[ax, 1])
        n = a.shape[ax]
        # region: full extent of axes before ax, original extent after it
        pre = (slice(None),) * ax
        post = orig[ax + 1:]
        if mode == "constant":
            if b:
                out[pre + (slice(0, b),) + post] = cv[ax, 0]
            if e:
                out[pre + (slice(b + n, b + n + e),) + post] = cv[ax, 1]
            continue
        if n == 0 and (b or e):
            raise ValueError(f"can't extend empty axis {ax} using modes other than 'constant' "
                             "or 'empty'")
        if mode == "linear_ramp":
            for side, (lo_, hi_) in ((0, (0, b)), (1, (b + n, b + n + e))):
                w = hi_ - lo_
                if w == 0:
                    continue
                edge_i = b if side == 0 else b + n - 1
                edge = out[pre + (slice(edge_i, edge_i + 1),) + post]
                end = ev[ax][side]
                # NumPy's linspace(end, edge, w, endpoint=False) along the
                # axis: k * step + end with step = (edge - end) / w (or
                # k / w * delta when some step is 0), floored for integer
                # dtypes, reversed on the right
                dt = np.result_type(end, a.dtype, 0.0)
                shp = [1] * nd
                shp[ax] = w
                k = np.arange(w, dtype=dt)
                if side == 1:
                    k = k[::-1].copy()
                kk = _asarray(k.reshape(shp))
                delta = edge.astype(dt) - dt.type(end)
                step = delta / dt.type(w)
                from .reductions import any as _any
                if bool(_any(step == 0)):
                    ramp = kk / dt.type(w) * delta
                else:
                    ramp = kk * step
                ramp = ramp + dt.type(end)
                if a.dtype.kind in "iub":
                    ramp = ew.unary("floor_op", ramp)
                out[pre + (slice(lo_, hi_),) + post] = ramp.astype(a.dtype)
            continue
        # maximum / minimum / mean over the first / last stat_length entries
        for side in (0, 1):
            w = b if side == 0 else e
            if w == 0:
                continue
            L = n if st is None or st[ax, side] is None else builtins.min(int(st[ax, side]), n)
            if L <= 0:
                raise ValueError("stat_length of 0 yields no value for padding")
            chunk = slice(b, b + L) if side == 0 else slice(b + n - L, b + n)
            region = out[pre + (chunk,) + post]
            if mode == "maximum":
                v = reductions.max(region, axis=ax, keepdims=True)
            elif mode == "minimum":
                v = reductions.min(region, axis=ax, keepdims=True)
            else:
                v = reductions.mean(region, axis=ax, keepdims=True)
                if a.dtype.kind in "iub":
                    v = ew.unary("rint_op", v)
                v = v.astype(a.dtype)
            tgt = slice(0, b) if side == 0 else slice(b + n, b + n + e)
            out[pre + (tgt,) + post] = v
    return out


# ======================================================== insert / delete
def _axis_setup(arr, axis):
    a = _asarray(arr)
    if axis is None:
        a = a.ravel()
        axis = 0
    return a, _normalize_axis(axis, a.ndim)


def delete(arr, obj, axis=None):
    """Entries along ``axis`` that ``obj`` (int, slice, index list or
    boolean mask) does not name, gathered on the device."""
    from .indexing import take
    a, ax = _axis_setup(arr, axis)
    n = a.shape[ax]
    keep = np.ones(n, dtype=bool)
    if isinstance(obj, slice):
        keep[obj] = False
    else:
        o = _host(obj)
        if o.dtype == np.bool_:
            if o.shape != (n,):
                raise ValueError(f"boolean array argument obj to delete must be one dimensional "
                                 f"and match the axis length of {n}")
            keep = ~o
        else:
            if o.size and o.dtype.kind not in "iu":
                raise IndexError("arrays used as indices must be of integer (or boolean) type")
            o = o.astype(np.int64).ravel()
            if o.size and (o.min() < -n or o.max() >= n):
                bad = o[(o < -n) | (o >= n)][0]
                raise IndexError(f"index {bad} is out of bounds for axis {ax} with size {n}")
            keep[o] = False
    return take(a, _asarray(np.flatnonzero(keep).astype(np.int64)), axis=ax)


def insert(arr, obj, values, axis=None):
    """NumPy's insert: one gather from the array concatenated with the
    (cast, broadcast) values, through the output->source row map."""
    from .indexing import take
    from .manipulation import concatenate, broadcast_to, moveaxis
    a, ax = _axis_setup(arr, axis)
    n = a.shape[ax]
    if isinstance(obj, slice):
        idx = np.arange(*obj.indices(n), dtype=np.int64)
        scalar = False
    else:
        o = _host(obj)
        if o.dtype == np.bool_:
            raise NotImplementedError("insert with a boolean obj is not supported")
        scalar = o.ndim == 0
        idx = o.astype(np.int64).ravel()
    if idx.size and (idx.min() < -n or idx.max() > n):
        bad = idx[(idx < -n) | (idx > n)][0]
        raise IndexError(f"index {bad} is out of bounds for axis {ax} with size {n}")
    idx = np.where(idx < 0, idx + n, idx)
    v = _asarray(values)
    if v.dtype != a.dtype:
        v = v.astype(a.dtype)
    if scalar:
        while v.ndim < a.ndim:
            v = v.reshape((1,) + tuple(v.shape))
        v = moveaxis(v, 0, ax)
        numnew = v.shape[ax]
        shp = list(a.shape)
        shp[ax] = numnew
        v = broadcast_to(v, tuple(shp))
        at = int(idx[0])
        src = np.concatenate([np.arange(at), n + np.arange(numnew), np.arange(at, n)])
    else:
        numnew = idx.size
        shp = list(a.shape)
        shp[ax] = numnew
        while v.ndim < a.ndim:
            v = v.reshape((1,) + tuple(v.shape))
        if v.ndim == a.ndim and v.shape[ax] not in (1, numnew) and numnew == 1:
            raise ValueError("shape mismatch: value array could not be broadcast")
        v = broadcast_to(v, tuple(shp))
        order = np.argsort(idx, kind="mergesort")
        pos = idx.copy()
        pos[order] += np.arange(numnew)
        total = n + numnew
        src = np.empty(total, dtype=np.int64)
        old = np.ones(total, dtype=bool)
        old[pos] = False
        src[old] = np.arange(n)
        src[pos] = n + np.arange(numnew)
    both = concatenate([a, v.copy()], axis=ax)
    return take(both, _asarray(src.astype(np.int64)), axis=ax)


def diagflat(v, k=0):
    from .manipulation import diag
    return diag(_asarray(v).ravel(), k)


def ediff1d(ary, to_end=None, to_begin=None):
    from .manipulation import concatenate
    a = _asarray(ary).ravel()
    parts = []
    for extra, name in ((to_begin, "to_begin"), (None, None), (to_end, "to_end")):
        if name is None:
            parts.append(a[1:] - a[:-1] if a.size else a.copy())
            continue
        if extra is None:
            continue
        e = np.asarray(_host(extra))
        if not np.can_cast(e, a.dtype, casting="same_kind"):
            raise TypeError(f"dtype of `{name}` must be compatible with input `ary` under the "
                            "`same_kind` rule.")
        parts.append(_asarray(e.ravel().astype(a.dtype)))
    return concatenate(parts) if len(parts) > 1 else parts[0]


# ============================================== multi-dimensional histograms
def histogramdd(sample, bins=10, range=None, density=None, weights=None):
    """NumPy's histogramdd: per-dimension bin numbers by binary search of
    the edges (right edge folded into the last bin), one flat bin index,
    one bincount, outliers cut away."""
    from .extras import _outer_edges, bincount
    from .sorting import searchsorted
    from .manipulation import stack
    if isinstance(sample, (list, tuple)):
        cols = [_asarray(s).ravel() for s in sample]
    else:
        s = _asarray(sample)
        if s.ndim == 1:
            cols = [s]
        else:
            cols = [s[:, i] for i in builtins.range(s.shape[1])]
    D = len(cols)
    try:
        M = len(bins)
        if M != D:
            raise ValueError("The dimension of bins must be equal to the dimension of the sample x.")
        blist = list(bins)
    except TypeError:
        blist = D * [bins]
    rng = (None,) * D if range is None else range
    if len(rng) != D:
        raise ValueError("range argument must have one entry per dimension")
    edges, nbin = [], []
    for i in builtins.range(D):
        b = blist[i]
        if np.ndim(b) == 0 and not isinstance(b, ndarray):
            if b < 1:
                raise ValueError(f"`bins[{i}]` must be positive, when an integer")
            lo, hi = _outer_edges(cols[i], rng[i])
            e = np.linspace(lo, hi, int(b) + 1)
        else:
            e = np.asarray(_host(b))
            if e.ndim != 1:
                raise ValueError(f"`bins[{i}]` must be a scalar or 1d array")
            if np.any(e[:-1] > e[1:]):
                raise ValueError(f"`bins[{i}]` must be monotonically increasing, when an array")
        edges.append(e)
        nbin.append(e.size + 1)
    xy = None
    for i in builtins.range(D):
        c = cols[i]
        cnt = searchsorted(_asarray(edges[i]), c, side="right")
        cnt = ew.where(c == edges[i][-1], cnt - 1, cnt)
        xy = cnt if xy is None else xy * nbin[i] + cnt
    total = _prod(nbin)
    w = None if weights is None else _asarray(weights).ravel()
    hist = bincount(xy.astype(np.int64), weights=w, minlength=total)
    hist = hist.astype(np.float64).reshape(tuple(nbin))
    hist = hist[(slice(1, -1),) * D].copy()
    if density:
        from .reductions import sum as _sum
        s = _sum(hist)
        for i in builtins.range(D):
            shp = [1] * D
            shp[i] = nbin[i] - 2
            hist = hist / _asarray(np.diff(edges[i]).reshape(shp))
        hist = hist / s
    return hist, [_asarray(e) for e in edges]


def histogram2d(x, y, bins=10, range=None, density=None, weights=None):
    try:
        N = len(bins)
    except TypeError:
        N = 1
    if N != 1 and N != 2:
        xe = ye = bins
        bins = [xe, ye]
    hist, edges = histogramdd([x, y], bins, range, density, weights)
    return hist, edges[0], edges[1]


# ============================================================ bit packing
def packbits(a, axis=None, bitorder="big"):
    """Eight truth values per byte (first one in the high bit for 'big'),
    the axis zero-padded to a multiple of 8.  As in the reference
    (bitwise_ops.py:100-103) each element counts by its low byte (its
    uint8 cast) and the bytes come back as uint16, the device type that
    holds uint8 data."""
    from .manipulation import moveaxis, concatenate
    from .reductions import sum as _sum
    x = _asarray(a)
    if x.dtype.kind not in "biu":
        raise TypeError("Expected an input array of integer or boolean data type")
    if bitorder not in ("big", "little"):
        raise ValueError("'order' must be either 'little' or 'big'")
    if axis is None:
        x, ax = x.ravel(), 0
    else:
        ax = _normalize_axis(axis, x.ndim)
    x = moveaxis(x, ax, -1)
    n = x.shape[-1]
    bits = (x != 0) if x.dtype == np.bool_ else ((x & 0xFF) != 0)
    bits = bits.astype(np.uint16)
    padn = (-n) % 8
    if padn:
        from .creation import zeros
        bits = concatenate([bits, zeros(tuple(x.shape[:-1]) + (padn,), dtype=np.uint16)], axis=-1)
    m = (n + padn) // 8
    bits = bits.reshape(tuple(x.shape[:-1]) + (m, 8))
    w = np.array([128, 64, 32, 16, 8, 4, 2, 1] if bitorder == "big" else
                 [1, 2, 4, 8, 16, 32, 64, 128], dtype=np.uint16)
    packed = _asarray(_sum(bits * _asarray(w), axis=-1)).astype(np.uint16)
    return moveaxis(packed, -1, ax).copy()


def unpackbits(a, axis=None, count=None, bitorder="big"):
    """Bits of each element's low byte (its uint8 cast, as in the reference,
    bitwise_ops.py:106-109), as uint16 zeros and ones."""
    from .manipulation import moveaxis
    x = _asarray(a)
    if x.dtype.kind not in "biu":
        raise TypeError("Expected an input array of unsigned byte data type")
    x = (x.astype(np.uint16) if x.dtype.kind == "b" else x & 0xFF).astype(np.uint16)
    if bitorder not in ("big", "little"):
        raise ValueError("'order' must be either 'little' or 'big'")
    if axis is None:
        x, ax = x.ravel(), 0
    else:
        ax = _normalize_axis(axis, x.ndim)
    x = moveaxis(x, ax, -1)
    sh = np.array([7, 6, 5, 4, 3, 2, 1, 0] if bitorder == "big" else
                  [0, 1, 2, 3, 4, 5, 6, 7], dtype=np.uint16)
    bits = (x.reshape(tuple(x.shape) + (1,)) >> _asarray(sh)) & np.uint16(1)
    bits = bits.reshape(tuple(x.shape[:-1]) + (x.shape[-1] * 8,))
    total = bits.shape[-1]
    if count is not None:
        c = int(count)
        if c < 0:
            c = builtins.max(total + c, 0)
        if c <= total:
            bits = bits[..., :c]
        else:
            from .creation import zeros
            from .manipulation import concatenate
            bits = concatenate([bits, zeros(tuple(bits.shape[:-1]) + (c - total,),
                                            dtype=np.uint16)], axis=-1)
    return moveaxis(bits, -1, ax).copy()


# ============================================================ polynomials
def _poly_arr(p):
    if isinstance(p, poly1d):
        return p.coeffs
    return _asarray(p)


def polyval(p, x):
    """Horner's rule as NumPy runs it: y = zeros_like(x), then y = y*x + c
    for each coefficient (read once to the host, as NumPy's scalars)."""
    from .creation import zeros
    coeffs = _host(_poly_arr(p))
    if coeffs.ndim != 1:
        coeffs = np.atleast_1d(coeffs)
    if isinstance(x, poly1d):
        raise NotImplementedError("polyval of a poly1d argument is not supported")
    xs = _asarray(x)
    y = zeros(tuple(xs.shape), dtype=xs.dtype)
    for c in coeffs:
        y = y * xs + c
    return y


def _wrap_poly(val, was_poly):
    return poly1d(val) if was_poly else val


def polyadd(a1, a2):
    from .manipulation import concatenate
    from .creation import zeros
    wp = isinstance(a1, poly1d) or isinstance(a2, poly1d)
    x, y = _asarray(_poly_arr(a1)).ravel(), _asarray(_poly_arr(a2)).ravel()
    d = y.size - x.size
    if d > 0:
        x = concatenate([zeros((d,), dtype=x.dtype), x])
    elif d < 0:
        y = concatenate([zeros((-d,), dtype=y.dtype), y])
    return _wrap_poly(x + y, wp)


def polysub(a1, a2):
    from .manipulation import concatenate
    from .creation import zeros
    wp = isinstance(a1, poly1d) or isinstance(a2, poly1d)
    x, y = _asarray(_poly_arr(a1)).ravel(), _asarray(_poly_arr(a2)).ravel()
    d = y.size - x.size
    if d > 0:
        x = concatenate([zeros((d,), dtype=x.dtype), x])
    elif d < 0:
        y = concatenate([zeros((-d,), dtype=y.dtype), y])
    return _wrap_poly(x - y, wp)


def polymul(a1, a2):
    from .extras import convolve
    wp = isinstance(a1, poly1d) or isinstance(a2, poly1d)
    return _wrap_poly(convolve(_poly_arr(a1), _poly_arr(a2)), wp)


def polydiv(u, v):
    """NumPy's long division (scale by 1/v[0], subtract d*v per quotient
    term), then leading remainder terms within 1e-14 of zero dropped."""
    from .creation import zeros
    wp = isinstance(u, poly1d) or isinstance(v, poly1d)
    uu = _asarray(_poly_arr(u)).ravel() + 0.0
    vv = _asarray(_poly_arr(v)).ravel() + 0.0
    vh = _host(vv)
    uh0 = _host(uu[0:1])[0]
    w_dtype = (uh0 + vh[0]).dtype
    m, n = uu.size - 1, vv.size - 1
    scale = 1.0 / vh[0]
    q = zeros((builtins.max(m - n + 1, 1),), dtype=w_dtype)
    r = uu.astype(w_dtype)
    for k in builtins.range(0, m - n + 1):
        d = scale * r[k]
        q[k:k + 1] = d
        r[k:k + n + 1] = r[k:k + n + 1] - d * vv
    rh = None
    while r.size > 1:
        rh = _host(r[0:1])
        if np.allclose(rh[0], 0, rtol=1e-14):
            r = r[1:]
        else:
            break
    if wp:
        return poly1d(q), poly1d(r)
    return q, r.copy()


def polyder(p, m=1):
    from .creation import arange
    m = int(m)
    if m < 0:
        raise ValueError("Order of derivative must be positive (see polyint)")
    wp = isinstance(p, poly1d)
    y = _asarray(_poly_arr(p))
    for _ in builtins.range(m):
        n = y.size - 1
        y = y[:-1] * arange(n, 0, -1, dtype=np.int64)
    return _wrap_poly(y, wp)


def polyint(p, m=1, k=None):
    from .creation import arange
    from .manipulation import concatenate
    m = int(m)
    if m < 0:
        raise ValueError("Order of integral must be positive (see polyder)")
    if k is None:
        k = np.zeros(m, float)
    k = np.atleast_1d(k)
    if len(k) == 1 and m > 1:
        k = k[0] * np.ones(m, float)
    if len(k) < m:
        raise ValueError("k must be a scalar or a rank-1 array of length 1 or >m.")
    wp = isinstance(p, poly1d)
    y = _asarray(_poly_arr(p))
    for i in builtins.range(m):
        y = concatenate([y / arange(y.size, 0, -1, dtype=np.int64),
                         _asarray(np.asarray([k[i]]))])
    return _wrap_poly(y, wp)


def poly(seq_of_zeros):
    """Coefficients of the polynomial with the given roots (repeated
    convolution with [1, -root], in the roots' dtype)."""
    from .extras import convolve
    from .creation import ones
    z = _asarray(seq_of_zeros)
    if z.ndim == 2 and z.shape[0] == z.shape[1] and z.shape[0] != 0:
        raise NotImplementedError("poly of a matrix (its eigenvalues) is not supported")
    if z.ndim != 1:
        z = z.ravel()
    zh = _host(z)
    dt = zh.dtype
    a = ones((1,), dtype=dt)
    for zero in zh:
        a = convolve(a, _asarray(np.array([1, -zero], dtype=dt)), mode="full")
    return a


def polyfit(x, y, deg, rcond=None, full=False, w=None, cov=False):
    """Least-squares fit through the device QR solver on NumPy's column-
    scaled Vandermonde system."""
    from .linalg import lstsq
    from .extras import vander
    from . import reductions
    if full or cov:
        raise NotImplementedError("polyfit(full=True / cov=True) is not supported on the device")
    order = int(deg) + 1
    xx = _asarray(x).astype(np.float64) + 0.0
    yy = _asarray(y).astype(np.float64) + 0.0
    if deg < 0:
        raise ValueError("expected deg >= 0")
    if xx.ndim != 1:
        raise TypeError("expected 1D vector for x")
    if xx.size == 0:
        raise TypeError("expected non-empty vector for x")
    if yy.ndim < 1 or yy.ndim > 2:
        raise TypeError("expected 1D or 2D array for y")
    if xx.shape[0] != yy.shape[0]:
        raise TypeError("expected x and y to have same length")
    lhs = vander(xx, order)
    rhs = yy
    if w is not None:
        ww = _asarray(w).astype(np.float64)
        lhs = lhs * ww.reshape((ww.size, 1))
        rhs = rhs * (ww if rhs.ndim == 1 else ww.reshape((ww.size, 1)))
    scale = ew.unary("sqrt_op", reductions.sum(lhs * lhs, axis=0))
    lhs = lhs / scale
    c = lstsq(lhs, rhs)[0]
    return (c.T / scale).T.copy() if c.ndim == 2 else c / scale


def roots(p):
    raise NotImplementedError("roots needs the eigenvalues of a general matrix, which the device "
                              "library does not provide")


class poly1d:
    """One-variable polynomial with device coefficients (highest power
    first), evaluated with polyval."""

    __hash__ = None

    def __init__(self, c_or_r, r=False, variable=None):
        if isinstance(c_or_r, poly1d):
            self._coeffs = c_or_r._coeffs
            self._variable = c_or_r._variable if variable is None else variable
            return
        if r:
            c = poly(c_or_r)
        else:
            c = _asarray(c_or_r)
            if c.ndim > 1:
                raise ValueError("Polynomial must be 1d only.")
            c = c.ravel()
            nz = np.flatnonzero(_host(c))
            c = c[int(nz[0]):] if nz.size else c[-1:] * 0
        self._coeffs = c.copy()
        self._variable = "x" if variable is None else variable

    @property
    def coeffs(self):
        return self._coeffs

    c = coef = coefficients = coeffs

    @property
    def order(self):
        return self._coeffs.size - 1

    o = order

    @property
    def variable(self):
        return self._variable

    def __call__(self, val):
        if isinstance(val, poly1d):
            raise NotImplementedError("composition of poly1d objects is not supported")
        return polyval(self._coeffs, val)

    def __len__(self):
        return self.order

    def __array__(self, dtype=None, copy=None):
        h = _host(self._coeffs)
        return h.astype(dtype) if dtype is not None else h

    def __repr__(self):
        return f"poly1d({np.array2string(_host(self._coeffs), separator=', ')})"

    def __neg__(self):
        return poly1d(-self._coeffs)

    def __pos__(self):
        return self

    def __add__(self, other):
        return polyadd(self, other if isinstance(other, poly1d) else poly1d(np.atleast_1d(other)))

    __radd__ = __add__

    def __sub__(self, other):
        return polysub(self, other if isinstance(other, poly1d) else poly1d(np.atleast_1d(other)))

    def __rsub__(self, other):
        return polysub(poly1d(np.atleast_1d(other)), self)

    def __mul__(self, other):
        if np.isscalar(other):
            return poly1d(self._coeffs * other)
        return polymul(self, other)

    def __rmul__(self, other):
        return self.__mul__(other)

    def __pow__(self, k):
        if not isinstance(k, (int, np.integer)) or k < 0:
            raise ValueError("Power to non-negative integers only.")
        res = poly1d([1])
        for _ in builtins.range(k):
            res = polymul(res, self)
        return res

    def __eq__(self, other):
        if not isinstance(other, poly1d):
            return NotImplemented
        a, b = _host(self._coeffs), _host(other._coeffs)
        return a.shape == b.shape and bool(np.all(a == b))

    def __ne__(self, other):
        r = self.__eq__(other)
        return r if r is NotImplemented else not r

    def __getitem__(self, power):
        h = _host(self._coeffs)
        ind = self.order - power
        if ind < 0 or ind > self.order:
            return h.dtype.type(0)
        return h[ind]

    def deriv(self, m=1):
        return poly1d(polyder(self._coeffs, m))

    def integ(self, m=1, k=0):
        return poly1d(polyint(self._coeffs, m, k))

    @property
    def roots(self):
        return roots(self._coeffs)

    r = roots


# ======================================================== window functions
def _window_n(M):
    from .creation import arange
    return arange(1 - M, M, 2, dtype=np.float64)


def bartlett(M):
    from .creation import ones, zeros
    M = float(M)
    if M < 1:
        return zeros((0,), dtype=np.float64)
    if M == 1:
        return ones((1,), dtype=np.float64)
    n = _window_n(M)
    return ew.where(n <= 0, 1 + n / (M - 1), 1 - n / (M - 1))


def _cos_window(M, terms):
    from .creation import ones, zeros
    M = float(M)
    if M < 1:
        return zeros((0,), dtype=np.float64)
    if M == 1:
        return ones((1,), dtype=np.float64)
    n = _window_n(M)
    r = None
    for coef, mult in terms:
        t = coef if mult == 0 else coef * ew.unary("cos_op", mult * np.pi * n / (M - 1))
        r = t if r is None else r + t
    return r


def blackman(M):
    return _cos_window(M, ((0.42, 0), (0.5, 1.0), (0.08, 2.0)))


def hamming(M):
    return _cos_window(M, ((0.54, 0), (0.46, 1.0)))


def hanning(M):
    return _cos_window(M, ((0.5, 0), (0.5, 1.0)))


def kaiser(M, beta):
    from .creation import arange, ones
    if M == 1:
        return ones((1,), dtype=np.float64)
    n = arange(0, M, dtype=np.float64)
    alpha = (M - 1) / 2.0
    return i0(beta * ew.unary("sqrt_op", 1 - ((n - alpha) / alpha) ** 2.0)) / \
        _host(i0(_asarray(np.array(float(beta)))))[()]


def _chbevl(x, vals):
    b0 = vals[0]
    b1 = 0.0
    b2 = 0.0
    for i in builtins.range(1, len(vals)):
        b2 = b1
        b1 = b0
        b0 = x * b1 - b2 + vals[i]
    return 0.5 * (b0 - b2)


def i0(x):
    """Modified Bessel function of order 0 with the Chebyshev expansions
    NumPy evaluates (Cephes' coefficients, read from NumPy), both branches
    as fused expressions."""
    from numpy.lib import _function_base_impl as _fb
    a = _asarray(x)
    if a.dtype.kind == "c":
        raise TypeError("i0 not supported for complex values")
    if a.dtype.kind != "f":
        a = a.astype(np.float64)
    a = ew.unary("abs_op", a)
    small = ew.unary("exp_op", a) * _chbevl(a / 2.0 - 2, _fb._i0A)
    safe = ew.where(a <= 8.0, 9.0, a)
    large = ew.unary("exp_op", safe) * _chbevl(32.0 / safe - 2.0, _fb._i0B) / \
        ew.unary("sqrt_op", safe)
    return ew.where(a <= 8.0, small, large)


def unwrap(p, discont=None, axis=-1, *, period=2 * np.pi):
    """NumPy's unwrap: wrapped differences, corrections where |dd| is at
    least discont, accumulated along the axis."""
    from .reductions import cumsum
    a = _asarray(p)
    ax = _normalize_axis(axis, a.ndim)
    nd = a.ndim
    s1 = (slice(None),) * ax + (slice(1, None),)
    s0 = (slice(None),) * ax + (slice(None, -1),)
    dd = a[s1] - a[s0]
    if discont is None:
        discont = period / 2
    dtype = np.result_type(dd.dtype, period)
    if np.issubdtype(dtype, np.integer):
        interval_high, rem = divmod(period, 2)
        boundary_ambiguous = rem == 0
    else:
        interval_high = period / 2
        boundary_ambiguous = True
    interval_low = -interval_high
    ddmod = ew.binary("mod_op", dd - interval_low, period) + interval_low
    if boundary_ambiguous:
        ddmod = ew.where((ddmod == interval_low) & (dd > 0), interval_high, ddmod)
    ph = ddmod - dd
    ph = ew.where(ew.unary("abs_op", dd) < discont, 0, ph)
    up = a.astype(dtype).copy()
    if a.shape[ax] > 1:
        up[s1] = a[s1] + cumsum(ph, axis=ax)
    return up


# ============================================================ unique family
UniqueAllResult = namedtuple("UniqueAllResult", ["values", "indices", "inverse_indices", "counts"])
UniqueCountsResult = namedtuple("UniqueCountsResult", ["values", "counts"])
UniqueInverseResult = namedtuple("UniqueInverseResult", ["values", "inverse_indices"])


def unique_all(x):
    from .manipulation import unique
    v, i, inv, c = unique(x, return_index=True, return_inverse=True, return_counts=True,
                          equal_nan=False)
    return UniqueAllResult(v, i, inv.reshape(tuple(_asarray(x).shape)), c)


def unique_counts(x):
    from .manipulation import unique
    v, c = unique(x, return_counts=True, equal_nan=False)
    return UniqueCountsResult(v, c)


def unique_inverse(x):
    from .manipulation import unique
    v, inv = unique(x, return_inverse=True, equal_nan=False)
    return UniqueInverseResult(v, inv.reshape(tuple(_asarray(x).shape)))


def unique_values(x):
    from .manipulation import unique
    return unique(x, equal_nan=False)


# ============================================================ index tricks
class _Grid:
    """mgrid / ogrid: the 1-D coordinate vectors come from NumPy's slice
    rules (arange for a real step, linspace for an imaginary one); the
    dense grid is broadcast and stacked on the device."""

    def __init__(self, sparse):
        self.sparse = sparse

    def __getitem__(self, key):
        from .manipulation import broadcast_arrays, stack
        if isinstance(key, slice):
            return _asarray(np.mgrid[key])
        vecs = np.ogrid[key]
        devs = [_asarray(np.ascontiguousarray(v)) for v in vecs]
        if self.sparse:
            return tuple(devs)
        return stack([b.copy() for b in broadcast_arrays(*devs)], axis=0)


mgrid = _Grid(False)
ogrid = _Grid(True)


class _Concat:
    """r_ / c_: slices become ranges, scalars and arrays are joined along
    the axis (an 'axis[,ndmin]' string as first item sets them)."""

    def __init__(self, axis, ndmin, column):
        self.axis, self.ndmin, self.column = axis, ndmin, column

    def __getitem__(self, key):
        from .manipulation import concatenate
        items = key if isinstance(key, tuple) else (key,)
        axis, ndmin, column = self.axis, self.ndmin, self.column
        if items and isinstance(items[0], str):
            spec = items[0]
            items = items[1:]
            if spec in ("r", "c"):
                raise NotImplementedError("r_['r'] / r_['c'] matrix output is not supported")
            parts = [int(s) for s in spec.split(",")]
            axis = parts[0]
            ndmin = parts[1] if len(parts) > 1 else 1
            column = len(parts) > 2 and parts[2] == 0
        arrs, weak, strong = [], [], []
        for it in items:
            if isinstance(it, slice):
                a = _asarray(np.r_[it])
            elif isinstance(it, ndarray):
                a = it
            elif type(it) in (int, float, bool, complex):
                # Python scalars join with NumPy's weak promotion
                weak.append(it)
                a = _asarray(np.array(it, ndmin=1))
            else:
                a = _asarray(np.array(it, ndmin=1))
            if type(it) not in (int, float, bool, complex):
                strong.append(a.dtype)
            if a.ndim == 0:
                a = a.reshape((1,))
            while a.ndim < ndmin:
                a = a.reshape((tuple(a.shape) + (1,)) if column and a.ndim == 1 else
                              ((1,) + tuple(a.shape)))
            arrs.append(a)
        if weak:
            dt = np.result_type(*strong, *weak) if strong else np.result_type(*[
                np.array(w).dtype for w in weak])
            arrs = [x if x.dtype == dt else x.astype(dt) for x in arrs]
        return concatenate(arrs, axis=axis)

    def __len__(self):
        return 0


r_ = _Concat(0, 1, False)
c_ = _Concat(-1, 2, True)


def block(arrays):
    """Nested lists joined innermost-last: the deepest lists along the last
    axis, each outer level one axis further left."""
    from .manipulation import concatenate

    def depth(x):
        if isinstance(x, list):
            if not x:
                raise ValueError("List at arrays cannot be empty")
            ds = {depth(e) for e in x}
            if len(ds) != 1:
                raise ValueError("List depths are mismatched.")
            return 1 + ds.pop()
        if isinstance(x, tuple):
            raise TypeError("arrays is a tuple. Only lists can be used to arrange blocks, and "
                            "np.block does not allow implicit conversion from tuple to ndarray.")
        return 0

    def maxnd(x):
        if isinstance(x, list):
            return builtins.max(maxnd(e) for e in x)
        return _asarray(x).ndim

    d = depth(arrays)
    nd = builtins.max(d, maxnd(arrays))

    def build(x, level):
        if not isinstance(x, list):
            a = _asarray(x)
            return a.reshape((1,) * (nd - a.ndim) + tuple(a.shape)) if a.ndim < nd else a
        parts = [build(e, level + 1) for e in x]
        return concatenate(parts, axis=-(d - level)) if len(parts) > 1 else parts[0].copy()

    return build(arrays, 0)


def apply_along_axis(func1d, axis, arr, *args, **kwargs):
    """func1d on every 1-D slice along the axis (NumPy's loop), results
    stacked in place of that axis."""
    from .manipulation import moveaxis, stack
    a = _asarray(arr)
    ax = _normalize_axis(axis, a.ndim)
    m = moveaxis(a, ax, -1)
    outer = tuple(m.shape[:-1])
    if _prod(outer) == 0:
        raise ValueError("Cannot apply_along_axis when any iteration dimensions are 0")
    res = []
    for idx in np.ndindex(*outer):
        r = func1d(m[idx], *args, **kwargs)
        res.append(_asarray(r))
    out = stack(res, axis=0)
    out = out.reshape(outer + tuple(res[0].shape))
    k = res[0].ndim
    if k == 0:
        return out
    # the function's result axes replace the iterated axis
    perm = list(builtins.range(len(outer)))
    perm = perm[:ax] + list(builtins.range(len(outer), len(outer) + k)) + perm[ax:]
    return out.transpose(perm).copy()


def apply_over_axes(func, a, axes):
    from .manipulation import expand_dims
    val = _asarray(a)
    N = val.ndim
    for ax in np.atleast_1d(np.asarray(axes)).ravel():
        ax = int(ax)
        if ax < 0:
            ax = N + ax
        res = _asarray(func(val, ax))
        if res.ndim == val.ndim:
            val = res
        else:
            res = expand_dims(res, ax)
            if res.ndim == val.ndim:
                val = res
            else:
                raise ValueError("function is not returning an array of the correct shape")
    return val


# ============================================================ small helpers
def resize(a, new_shape):
    from .manipulation import concatenate
    from .creation import zeros
    x = _asarray(a).ravel()
    shp = (int(new_shape),) if isinstance(new_shape, (int, np.integer)) else tuple(new_shape)
    if any(s < 0 for s in shp):
        raise ValueError("all elements of `new_shape` must be non-negative")
    n = _prod(shp)
    if x.size == 0 or n == 0:
        return zeros(shp, dtype=x.dtype)
    reps = -(-n // x.size)
    y = concatenate([x] * reps) if reps > 1 else x
    return y[:n].copy().reshape(shp)


def trim_zeros(filt, trim="fb", axis=None):
    from .indexing import argwhere
    from . import reductions
    a = _asarray(filt)
    t = trim.lower()
    if not set(t) <= {"f", "b"}:
        raise ValueError(f"unexpected character(s) in `trim`: {trim!r}")
    nz = argwhere(a)
    axes = builtins.range(a.ndim) if axis is None else (_normalize_axis(axis, a.ndim),)
    if nz.shape[0] == 0:
        sl = [slice(None)] * a.ndim
        for ax in axes:
            sl[ax] = slice(0, 0)
        return a[tuple(sl)]
    lo = _host(reductions.min(nz, axis=0))
    hi = _host(reductions.max(nz, axis=0)) + 1
    sl = [slice(None)] * a.ndim
    for ax in axes:
        start = int(lo[ax]) if "f" in t else 0
        stop = int(hi[ax]) if "b" in t else a.shape[ax]
        sl[ax] = slice(start, stop)
    return a[tuple(sl)]


def isposinf(x, out=None):
    a = _asarray(x)
    r = ew.unary("isinf_op", a) & ew.unary("logical_not_op", ew.unary("signbit_op", a))
    if out is not None:
        out[...] = r
        return out
    return r


def isneginf(x, out=None):
    a = _asarray(x)
    r = ew.unary("isinf_op", a) & ew.unary("signbit_op", a)
    if out is not None:
        out[...] = r
        return out
    return r


def isnat(x):
    raise TypeError("ufunc 'isnat' is only defined for np.datetime64 and np.timedelta64.")


def mask_indices(n, mask_func, k=0):
    from .creation import ones
    from .indexing import nonzero
    m = ones((n, n), dtype=np.int64)
    return nonzero(_asarray(mask_func(m, k)) != 0)


def asanyarray(a, dtype=None, order=None):
    return _asarray(a, dtype=dtype)


def asarray_chkfinite(a, dtype=None, order=None):
    from .reductions import all as _all
    x = _asarray(a, dtype=dtype)
    if x.dtype.kind in "fc" and not bool(_all(ew.unary("isfinite_op", x))):
        raise ValueError("array must not contain infs or NaNs")
    return x


def asfortranarray(a, dtype=None):
    """Device arrays are stored in C order; the values are those of
    NumPy's Fortran-ordered copy."""
    return _asarray(a, dtype=dtype).copy()


def require(a, dtype=None, requirements=None):
    """Device arrays are C-contiguous, aligned and writeable already; an
    'O' (own data) requirement makes a copy."""
    reqs = [requirements] if isinstance(requirements, str) else list(requirements or [])
    reqs = {str(r).upper() for r in reqs}
    if {"F", "F_CONTIGUOUS", "FORTRAN"} & reqs and {"C", "C_CONTIGUOUS", "CONTIGUOUS"} & reqs:
        raise ValueError("Cannot specify both 'C' and 'F' order")
    x = _asarray(a, dtype=dtype)
    return x.copy() if {"O", "OWNDATA", "E", "ENSUREARRAY"} & reqs else x._ensure_contiguous()


def astype(x, dtype, /, *, copy=True, device=None):
    a = _asarray(x)
    if not copy and a.dtype == np.dtype(dtype):
        return a
    return a.astype(dtype)


def fastCopyAndTranspose(a):
    return _asarray(a).T.copy()


def row_stack(tup, *, dtype=None, casting="same_kind"):
    from .manipulation import vstack
    return vstack(tup, dtype=dtype, casting=casting)


def trapz(y, x=None, dx=1.0, axis=-1):
    from .extras import trapezoid
    return trapezoid(y, x=x, dx=dx, axis=axis)
