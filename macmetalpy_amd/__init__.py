"""macmetalpy_amd -- MacMetalPy's array-compute hot path on AMD MI355X.

Drop-in for the reference's ``import macmetalpy as cp`` names on the hot
path (src/macmetalpy/__init__.py:8-236): ndarray, creation, random inputs,
elementwise ufuncs (arithmetic, transcendental, comparison, bitwise,
logical, predicates), where / clip, sum/mean/max/min/prod/argmax/argmin,
any/all/count_nonzero, NaN-aware reductions (nansum, nanmax, nanargmax, ...),
sort/argsort/searchsorted, cumsum/cumprod,
matmul / linalg.matmul / dot, RawKernel, set_config and synchronize.
Unlike the reference (darwin-only, __init__.py:5-6) it imports on any host;
device work needs libmmp_hip.so and a gfx950 GPU and raises otherwise.
"""
from __future__ import annotations

import math as _math

import numpy as _np

from ._config import get_config, set_config
from .ndarray import ndarray
from .raw_kernel import RawKernel
from .creation import (
    array, asarray, empty, zeros, ones, full, arange, linspace, eye,
    zeros_like, ones_like, empty_like, full_like, ascontiguousarray,
)
from .ufunc_ops import (
    negative, positive, absolute, abs, fabs, sign, square, reciprocal, sqrt, cbrt,
    exp, exp2, expm1, log, log2, log10, log1p, sin, cos, tan, arcsin, arccos, arctan,
    sinh, cosh, tanh, arcsinh, arccosh, arctanh, floor, ceil, rint, trunc, degrees,
    radians, rad2deg, deg2rad,
    add, subtract, multiply, divide, true_divide, floor_divide, mod, remainder, power,
    maximum, minimum, fmax, fmin, arctan2, hypot, fmod, copysign, nextafter, logaddexp,
    logaddexp2, heaviside, float_power, divmod,
    less, less_equal, greater, greater_equal, equal, not_equal,
    invert, bitwise_not, bitwise_invert, bitwise_and, bitwise_or, bitwise_xor, left_shift,
    right_shift, bitwise_left_shift, bitwise_right_shift, logical_and, logical_or,
    logical_xor, logical_not, isnan, isinf, isfinite, signbit,
    spacing, bitwise_count, conjugate, conj, ldexp, gcd, lcm, frexp, modf, vecdot, matvec,
    vecmat,
)
from .math_ops import where, clip, count_nonzero
from .manipulation import (
    concatenate, concat, stack, vstack, hstack, dstack, column_stack, split, array_split,
    hsplit, vsplit, dsplit, unstack, tile, repeat, flip, fliplr, flipud, rot90, roll,
    broadcast_to, broadcast_arrays, moveaxis, rollaxis, swapaxes, squeeze, expand_dims,
    atleast_1d, atleast_2d, atleast_3d, diagonal, diag, trace, tril, triu, copy, copyto,
    append, ptp, diff, outer, meshgrid, cross, kron, tensordot, average, unique,
    permute_dims, matrix_transpose,
)
from .statistics import median, quantile, percentile, nanmedian, nanquantile, nanpercentile
from .indexing import (take, put, take_along_axis, put_along_axis, putmask, place, compress,
                       extract, nonzero, flatnonzero, argwhere)
from .reductions import (
    sum, mean, prod, max, min, amax, amin, argmax, argmin, any, all, cumsum, cumprod, var,
    std,
)
from .nan_ops import (
    nansum, nanprod, nanmax, nanmin, nanmean, nanvar, nanstd, nanargmax, nanargmin,
    nancumsum, nancumprod,
)
from .sorting import sort, argsort, searchsorted
from .extras import (
    isclose, allclose, array_equal, array_equiv, isin, in1d, intersect1d, union1d, setdiff1d,
    setxor1d, round, around, fix, nan_to_num, real, imag, angle, isreal, iscomplex,
    real_if_close, sinc, interp, bincount, digitize, histogram, lexsort, partition,
    argpartition, cov, corrcoef, select, piecewise, choose, gradient, trapezoid, convolve,
    correlate, identity, tri, logspace, geomspace, vander, indices, ix_, fill_diagonal,
    diag_indices, diag_indices_from, tril_indices, triu_indices, tril_indices_from,
    triu_indices_from, ravel_multi_index, unravel_index, finfo, iinfo, result_type, can_cast,
    promote_types, isscalar, ndim, shape, size, asnumpy, get_array_module, cumulative_sum,
    cumulative_prod,
)
from .extras import histogram_bin_edges
from .routines import (
    einsum, einsum_path, pad, insert, delete, diagflat, ediff1d, histogramdd, histogram2d,
    packbits, unpackbits, poly, polyval, polyadd, polysub, polymul, polydiv, polyder, polyint,
    polyfit, roots, poly1d, bartlett, blackman, hamming, hanning, kaiser, i0, unwrap,
    unique_all, unique_counts, unique_inverse, unique_values, mgrid, ogrid, r_, c_, s_,
    index_exp, block, apply_along_axis, apply_over_axes, resize, trim_zeros, isposinf,
    isneginf, mask_indices, asanyarray, asarray_chkfinite, asfortranarray, require, astype,
    broadcast_shapes, fastCopyAndTranspose, row_stack, trapz, isnat,
)
from .host_api import (
    False_, True_, ScalarType, byte, ubyte, short, ushort, intc, uintc, uint, longlong,
    ulonglong, int_, intp, uintp, int8, uint8, single, double, half, longdouble, float_,
    longfloat, csingle, cdouble, clongdouble, complex64, complex128, complex_, cfloat,
    singlecomplex, longcomplex, clongfloat, bytes_, str_, object_, void, datetime64,
    timedelta64, generic, number, integer, signedinteger, unsignedinteger, inexact, floating,
    complexfloating, character, flexible, dtype, sctypeDict, typecodes, little_endian,
    euler_gamma, issubdtype, isdtype, mintypecode, typename, iterable, broadcast, flatiter,
    ndindex, common_type, min_scalar_type, iscomplexobj, isrealobj, isfortran,
    may_share_memory, shares_memory, array2string, array_repr, array_str, set_printoptions,
    get_printoptions, printoptions, format_float_positional, format_float_scientific,
    base_repr, binary_repr, info, errstate, seterr, geterr, seterrcall, geterrcall, getbufsize,
    setbufsize, get_include, show_config, show_runtime, save, savez, savez_compressed, load,
    loadtxt, savetxt, genfromtxt, fromfile, fromregex, frombuffer, fromstring, fromiter,
    from_dlpack, fromfunction, memmap, busday_count, busday_offset, busdaycalendar, is_busday,
    datetime_as_string, datetime_data, matrix, asmatrix, bmat, recarray, record, vectorize,
    frompyfunc, nditer, sort_complex, geterrobj, seterrobj, set_numeric_ops,
)
from .linalg_top import matmul, dot, vdot, inner
from ._backend import HipBackend as MetalBackend  # the reference's backend class name
from . import _gate as _gate_mod

_gate_mod.setup()  # the native dispatch gate takes over the hot elementwise path
from . import linalg
from . import random
from . import fft

# NumPy 2 aliases (reference __init__.py:262-272)
acos = arccos
acosh = arccosh
asin = arcsin
asinh = arcsinh
atan = arctan
atan2 = arctan2
atanh = arctanh
pow = power


def synchronize() -> None:
    """Block until all enqueued device work finished (reference
    __init__.py:233-236).  Lazy (unevaluated) arrays stay lazy."""
    from ._backend import HipBackend
    HipBackend().synchronize()


def materialize(*arrays) -> None:
    """Enqueue the kernels of lazy (fused) arrays now, without waiting for
    them; the reference evaluates lazily only on get()/reductions
    (_fusion.materialize, ndarray.py:478-481)."""
    for a in arrays:
        a._materialize_if_lazy()


def reshape(a, shape):
    return asarray(a).reshape(shape)


def transpose(a, axes=None):
    return asarray(a).transpose(axes)


def ravel(a):
    return asarray(a).ravel()


float16 = _np.float16
float32 = _np.float32
float64 = _np.float64
int16 = _np.int16
int32 = _np.int32
int64 = _np.int64
uint16 = _np.uint16
uint32 = _np.uint32
uint64 = _np.uint64
bool_ = _np.bool_
newaxis = None
nan = float("nan")
inf = float("inf")
pi = _math.pi
e = _math.e

__version__ = "0.1.0"
