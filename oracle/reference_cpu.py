"""NumPy restatement of the reference's CPU/NumPy path (test oracle only).

Every hot-path op of the reference dispatches, on its CPU path, to a NumPy
call chosen from fixed tables; the device path must reproduce those NumPy
results.  Citations are to files of grantkl/MacMetalPy v0.1.3.
"""
from __future__ import annotations

import numpy as np

# src/macmetalpy/ndarray.py:74-91 (_NP_UNARY), names as the reference's ops
UNARY = {
    "neg_op": np.negative, "negative_op": np.negative, "positive_op": np.positive,
    "abs_op": np.abs, "sign_op": np.sign, "square_op": np.square,
    "reciprocal_op": np.reciprocal, "sqrt_op": np.sqrt, "cbrt_op": np.cbrt,
    "exp_op": np.exp, "exp2_op": np.exp2, "expm1_op": np.expm1, "log_op": np.log,
    "log2_op": np.log2, "log10_op": np.log10, "log1p_op": np.log1p,
    "sin_op": np.sin, "cos_op": np.cos, "tan_op": np.tan, "asin_op": np.arcsin,
    "acos_op": np.arccos, "atan_op": np.arctan, "sinh_op": np.sinh, "cosh_op": np.cosh,
    "tanh_op": np.tanh, "asinh_op": np.arcsinh, "acosh_op": np.arccosh,
    "atanh_op": np.arctanh, "floor_op": np.floor, "ceil_op": np.ceil,
    "rint_op": np.rint, "trunc_op": np.trunc, "degrees_op": np.degrees,
    "radians_op": np.radians,
}

# src/macmetalpy/ndarray.py:92-102 (_NP_BINARY).  "mod_op" is np.mod, the
# CPU-path meaning of cp.mod (math_ops.py:540-548 documents the NumPy sign
# rule it aims at).
BINARY = {
    "add_op": np.add, "sub_op": np.subtract, "mul_op": np.multiply,
    "div_op": np.true_divide, "pow_op": np.power, "mod_op": np.mod,
    "min_op": np.minimum, "max_op": np.maximum, "atan2_op": np.arctan2,
    "hypot_op": np.hypot, "fmod_op": np.fmod, "copysign_op": np.copysign,
    "logaddexp_op": np.logaddexp, "logaddexp2_op": np.logaddexp2,
    "fmax_op": np.fmax, "fmin_op": np.fmin, "floor_divide_op": np.floor_divide,
    "heaviside_op": np.heaviside, "nextafter_op": np.nextafter,
}


# Bitwise, logical and predicate ops: the reference's CPU branches call these
# NumPy ufuncs (bitwise_ops.py:27-31 _BITWISE_NP and :70-93,
# logic_ops.py:45-63, math_ops.py:558-578, ufunc_ops.py:352).
UNARY.update({
    "invert_op": np.invert, "logical_not_op": np.logical_not, "isnan_op": np.isnan,
    "isinf_op": np.isinf, "isfinite_op": np.isfinite, "signbit_op": np.signbit,
})
BINARY.update({
    "bit_and_op": np.bitwise_and, "bit_or_op": np.bitwise_or, "bit_xor_op": np.bitwise_xor,
    "lshift_op": np.left_shift, "rshift_op": np.right_shift,
    "logical_and_op": np.logical_and, "logical_or_op": np.logical_or,
    "logical_xor_op": np.logical_xor,
})


def where(cond, x, y):
    """math_ops.where CPU branch (math_ops.py:124-130): np.where."""
    return np.where(cond, x, y)


def clip(a, lo, hi):
    """math_ops.clip CPU branch (math_ops.py:180-190): np.clip."""
    with np.errstate(all="ignore"):
        return np.clip(a, lo, hi)


def any_(a, axis=None, keepdims=False):
    """reductions.any CPU branch (reductions.py:255-268): np.any."""
    return np.any(a, axis=axis, keepdims=keepdims)


def all_(a, axis=None, keepdims=False):
    """reductions.all CPU branch (reductions.py:288-301): np.all."""
    return np.all(a, axis=axis, keepdims=keepdims)


def count_nonzero(a, axis=None, keepdims=False):
    """math_ops.count_nonzero (math_ops.py:693): np.count_nonzero."""
    return np.count_nonzero(a, axis=axis, keepdims=keepdims)


# NaN-aware reductions: the reference's CPU branches call NumPy's nan*
# functions (nan_ops.py:132-141, 187-196, 229-237, 258-266, 293-302,
# 346-355, 397-404, 503-510, 571-576, 596-601).
NAN_REDUCTIONS = {
    "nansum": np.nansum, "nanprod": np.nanprod, "nanmax": np.nanmax, "nanmin": np.nanmin,
    "nanmean": np.nanmean, "nanvar": np.nanvar, "nanstd": np.nanstd,
    "nanargmax": np.nanargmax, "nanargmin": np.nanargmin, "nancumsum": np.nancumsum,
    "nancumprod": np.nancumprod,
}


def nan_reduce(name, x, **kw):
    import warnings
    with warnings.catch_warnings(), np.errstate(all="ignore"):
        warnings.simplefilter("ignore", RuntimeWarning)
        return NAN_REDUCTIONS[name](x, **kw)


# Sorting: the reference's CPU branches call np.sort / np.argsort /
# np.searchsorted (sorting.py:30-31, 49-50, 259-262).  argsort is compared
# with the stable kind (the device sort is stable).
def sort(x, axis=-1, kind=None):
    return np.sort(x, axis=axis, kind=kind)


def argsort_stable(x, axis=-1):
    return np.argsort(x, axis=axis, kind="stable")


def searchsorted(a, v, side="left", sorter=None):
    return np.searchsorted(a, v, side=side, sorter=sorter)


def unary(op_name: str, x: np.ndarray) -> np.ndarray:
    with np.errstate(all="ignore"):
        return UNARY[op_name](x)


def binary(op_name: str, a, b) -> np.ndarray:
    with np.errstate(all="ignore"):
        return BINARY[op_name](a, b)


def floor_divide(a, b):
    """reductions/ufunc path: ufunc_ops.floor_divide -> np.floor_divide."""
    with np.errstate(all="ignore"):
        return np.floor_divide(a, b)


def mod(a, b):
    """math_ops.mod: NumPy remainder (result takes the divisor's sign)."""
    with np.errstate(all="ignore"):
        return np.mod(a, b)


# ---------------------------------------------------------- reductions
def sum(x, axis=None):
    """reductions.sum CPU branch (reductions.py:89-103): np.sum."""
    return np.sum(x, axis=axis)


def mean(x, axis=None):
    """reductions.mean CPU branch (reductions.py:130-143): np.mean."""
    return np.mean(x, axis=axis)


def argmax(x, axis=None):
    """reductions.argmax CPU branch (reductions.py:388-398): np.argmax."""
    return np.argmax(x, axis=axis)


def cumsum(x, axis=None):
    """reductions.cumsum CPU branch (reductions.py:669-675): np.cumsum
    (int32 input -> int64 output)."""
    return np.cumsum(x, axis=axis)


def matmul(a, b):
    """linalg_top.matmul CPU branch (linalg_top.py:99-106): np.matmul."""
    return np.matmul(a, b)


# ----------------------------------- float64-accumulated references
def sum_f64(x, axis=None):
    """Exact-ish reference for float sums: accumulate in float64."""
    return np.sum(np.asarray(x, dtype=np.float64), axis=axis)


def mean_f64(x, axis=None):
    return np.mean(np.asarray(x, dtype=np.float64), axis=axis)


def cumsum_f64(x):
    return np.cumsum(np.asarray(x, dtype=np.float64).ravel())


def matmul_f64(a, b):
    return np.matmul(np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64))


# ------------------------------------------------------- fused configs
def fused_elementwise(x):
    """y = sqrt(abs(x)) + exp(-x**2), op by op in the input dtype (what the
    reference's NumPy path evaluates; x**2 is np.square for float arrays)."""
    with np.errstate(all="ignore"):
        return np.sqrt(np.abs(x)) + np.exp(-(x ** 2))


def fusion_chain_terms(x, r):
    """tanh(x*r + 1.0) * exp(-abs(x)) - log1p(x*x), op by op (float32)."""
    with np.errstate(all="ignore"):
        return np.tanh(x * r + np.float32(1.0)) * np.exp(-np.abs(x)) - np.log1p(x * x)


def fusion_chain(x, r):
    """z = sum(terms, axis=1): the reference's CPU path (np.sum in float32)."""
    return np.sum(fusion_chain_terms(x, r), axis=1)


def fusion_chain_f64(x, r):
    """Row sums of the float32 terms accumulated in float64."""
    return np.sum(fusion_chain_terms(x, r).astype(np.float64), axis=1)


# ------------------------------------------------------------- helpers
def ulp_distance(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """ULP distance between float arrays of the same dtype (NaN == NaN,
    +0 == -0)."""
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype == np.float32:
        ia = a.view(np.int32).astype(np.int64)
        ib = b.view(np.int32).astype(np.int64)
        ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
        ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    elif a.dtype == np.float16:
        ia = a.view(np.int16).astype(np.int64)
        ib = b.view(np.int16).astype(np.int64)
        ia = np.where(ia < 0, -(ia & 0x7FFF), ia)
        ib = np.where(ib < 0, -(ib & 0x7FFF), ib)
    else:
        ia = a.view(np.int64)
        ib = b.view(np.int64)
        ia = np.where(ia < 0, -(ia & 0x7FFFFFFFFFFFFFFF), ia)
        ib = np.where(ib < 0, -(ib & 0x7FFFFFFFFFFFFFFF), ib)
    d = np.abs(ia - ib)
    both_nan = np.isnan(a) & np.isnan(b)
    return np.where(both_nan, 0, d)


def correctly_rounded(fn64, x32):
    """float64 evaluation rounded once to float32 (ULP yardstick)."""
    with np.errstate(all="ignore"):
        return fn64(np.asarray(x32, dtype=np.float64)).astype(np.float32)


def normwise_rel_error(c, ref):
    """||c - ref||_F / ||ref||_F in float64."""
    c = np.asarray(c, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.linalg.norm(c - ref) / np.linalg.norm(ref))
