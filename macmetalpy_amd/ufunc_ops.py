"""Elementwise ufunc front-ends.

Reference: src/macmetalpy/math_ops.py:15-67, 335-548 and
src/macmetalpy/ufunc_ops.py:38-348.  Each function converts its operands
and calls the shared dispatcher (``_elementwise.unary`` / ``binary``), as the
reference's wrappers call ``ndarray._unary_op`` / ``_binary_op``.  ``mod`` /
``remainder`` is a single device op with NumPy's sign rule, where the
reference composes ``x1 - floor_divide(x1, x2) * x2`` (math_ops.py:540-548).
"""
from __future__ import annotations

from . import _elementwise as ew

__all__: list[str] = []


def _unary(name, op_name, doc):
    def f(x, /, out=None, **kwargs):
        if kwargs:
            return _with_kwargs(name, (x,), out, kwargs)
        r = ew.unary(op_name, x)
        return _to_out(r, out)
    f.__name__ = f.__qualname__ = name
    f.__doc__ = doc
    globals()[name] = f
    __all__.append(name)
    return f


def _binary(name, op_name, doc):
    def f(x1, x2, /, out=None, **kwargs):
        if kwargs:
            return _with_kwargs(name, (x1, x2), out, kwargs)
        r = ew.binary(op_name, x1, x2)
        return _to_out(r, out)
    f.__name__ = f.__qualname__ = name
    f.__doc__ = doc
    globals()[name] = f
    __all__.append(name)
    return f


def _with_kwargs(name, inputs, out, kwargs):
    """A ufunc call with keyword arguments (``where=``, ``dtype=``,
    ``casting=``, ``order`` / ``subok``), evaluated as NumPy's ufunc call
    does, by the same code as the NumPy ufunc protocol.  Without ``out``,
    the elements outside ``where`` are left as a new array holds them
    (NumPy leaves them undefined)."""
    import numpy as np
    from . import _ufunc_table
    uf = getattr(np, name)
    kw = dict(kwargs)
    if out is not None:
        kw["out"] = out
    res = _ufunc_table.dispatch(uf, "__call__", inputs, kw)
    if res is NotImplemented:
        raise TypeError(f"{name}() got unsupported keyword arguments {sorted(kwargs)}")
    return res


def fabs(x, /, out=None, **kwargs):
    """Element-wise absolute value in NumPy's result dtype for fabs, which
    has float loops only: integers and bool are converted to float16 /
    float32 / float64 first (as np.fabs does), then the absolute value is
    taken."""
    import numpy as np
    from ._dtypes import ufunc_result_dtype
    from .ndarray import ndarray
    if kwargs:
        return _with_kwargs("fabs", (x,), out, kwargs)
    if not isinstance(x, ndarray):
        x = ew._asarray(x)
    rdt = ufunc_result_dtype(np.fabs, x.dtype)
    if rdt != x.dtype:
        x = x.astype(rdt)
    return _to_out(ew.unary("abs_op", x), out)


__all__.append("fabs")


def _to_out(r, out):
    if out is None:
        return r
    if isinstance(out, tuple):
        out = out[0]
    return out._inplace(r)


for _name, _op, _doc in [
    ("negative", "negative_op", "Element-wise negation."),
    ("positive", "positive_op", "Element-wise +x."),
    ("absolute", "abs_op", "Element-wise absolute value."),
    ("abs", "abs_op", "Element-wise absolute value."),
    ("sign", "sign_op", "Element-wise sign."),
    ("square", "square_op", "Element-wise square."),
    ("reciprocal", "reciprocal_op", "Element-wise 1/x."),
    ("sqrt", "sqrt_op", "Element-wise square root."),
    ("cbrt", "cbrt_op", "Element-wise cube root."),
    ("exp", "exp_op", "Element-wise exponential."),
    ("exp2", "exp2_op", "Element-wise 2**x."),
    ("expm1", "expm1_op", "Element-wise exp(x) - 1, accurate near 0."),
    ("log", "log_op", "Element-wise natural logarithm."),
    ("log2", "log2_op", "Element-wise base-2 logarithm."),
    ("log10", "log10_op", "Element-wise base-10 logarithm."),
    ("log1p", "log1p_op", "Element-wise log(1 + x), accurate near 0."),
    ("sin", "sin_op", "Element-wise sine."),
    ("cos", "cos_op", "Element-wise cosine."),
    ("tan", "tan_op", "Element-wise tangent."),
    ("arcsin", "asin_op", "Element-wise inverse sine."),
    ("arccos", "acos_op", "Element-wise inverse cosine."),
    ("arctan", "atan_op", "Element-wise inverse tangent."),
    ("sinh", "sinh_op", "Element-wise hyperbolic sine."),
    ("cosh", "cosh_op", "Element-wise hyperbolic cosine."),
    ("tanh", "tanh_op", "Element-wise hyperbolic tangent."),
    ("arcsinh", "asinh_op", "Element-wise inverse hyperbolic sine."),
    ("arccosh", "acosh_op", "Element-wise inverse hyperbolic cosine."),
    ("arctanh", "atanh_op", "Element-wise inverse hyperbolic tangent."),
    ("floor", "floor_op", "Element-wise floor."),
    ("ceil", "ceil_op", "Element-wise ceiling."),
    ("rint", "rint_op", "Round to nearest integer (ties to even)."),
    ("trunc", "trunc_op", "Element-wise truncation."),
    ("degrees", "degrees_op", "Radians to degrees."),
    ("radians", "radians_op", "Degrees to radians."),
    ("rad2deg", "degrees_op", "Radians to degrees."),
    ("deg2rad", "radians_op", "Degrees to radians."),
]:
    _unary(_name, _op, _doc)

for _name, _op, _doc in [
    ("add", "add_op", "Element-wise addition."),
    ("subtract", "sub_op", "Element-wise subtraction."),
    ("multiply", "mul_op", "Element-wise multiplication."),
    ("divide", "div_op", "Element-wise true division."),
    ("true_divide", "div_op", "Element-wise true division."),
    ("floor_divide", "floor_divide_op", "Element-wise floor division (NumPy semantics)."),
    ("mod", "mod_op", "Element-wise remainder with the sign of the divisor."),
    ("remainder", "mod_op", "Element-wise remainder with the sign of the divisor."),
    ("power", "pow_op", "Element-wise power."),
    ("maximum", "max_op", "Element-wise maximum (NaN-propagating)."),
    ("minimum", "min_op", "Element-wise minimum (NaN-propagating)."),
    ("fmax", "fmax_op", "Element-wise maximum ignoring NaN."),
    ("fmin", "fmin_op", "Element-wise minimum ignoring NaN."),
    ("arctan2", "atan2_op", "Element-wise arctan(x1/x2) with quadrant."),
    ("hypot", "hypot_op", "Element-wise sqrt(x1**2 + x2**2)."),
    ("fmod", "fmod_op", "Element-wise C fmod (sign of the dividend)."),
    ("copysign", "copysign_op", "Magnitude of x1 with the sign of x2."),
    ("nextafter", "nextafter_op", "Next representable value after x1 towards x2."),
    ("logaddexp", "logaddexp_op", "log(exp(x1) + exp(x2))."),
    ("logaddexp2", "logaddexp2_op", "log2(2**x1 + 2**x2)."),
    ("heaviside", "heaviside_op", "Heaviside step function."),
    ("less", "lt_op", "Element-wise x1 < x2."),
    ("less_equal", "le_op", "Element-wise x1 <= x2."),
    ("greater", "gt_op", "Element-wise x1 > x2."),
    ("greater_equal", "ge_op", "Element-wise x1 >= x2."),
    ("equal", "eq_op", "Element-wise x1 == x2."),
    ("not_equal", "ne_op", "Element-wise x1 != x2."),
]:
    _binary(_name, _op, _doc)


# Bitwise, logical and predicate ufuncs (reference bitwise_ops.py:58-93,
# logic_ops.py:45-63, math_ops.py:558-578, ufunc_ops.py:352).  The reference
# computes bitwise ops in int32 and returns int32; here they keep NumPy's
# dtypes (int64 stays int64, bool stays bool).
for _name, _op, _doc in [
    ("invert", "invert_op", "Bitwise NOT (logical NOT for bool)."),
    ("bitwise_not", "invert_op", "Bitwise NOT (logical NOT for bool)."),
    ("bitwise_invert", "invert_op", "Bitwise NOT (logical NOT for bool)."),
    ("logical_not", "logical_not_op", "Truth value of NOT x."),
    ("isnan", "isnan_op", "True where x is NaN."),
    ("isinf", "isinf_op", "True where x is +inf or -inf."),
    ("isfinite", "isfinite_op", "True where x is neither infinite nor NaN."),
    ("signbit", "signbit_op", "True where the sign bit is set (-0.0 included)."),
]:
    _unary(_name, _op, _doc)

for _name, _op, _doc in [
    ("bitwise_and", "bit_and_op", "Element-wise bitwise AND."),
    ("bitwise_or", "bit_or_op", "Element-wise bitwise OR."),
    ("bitwise_xor", "bit_xor_op", "Element-wise bitwise XOR."),
    ("left_shift", "lshift_op", "Shift bits left (counts outside [0, bits) give 0)."),
    ("bitwise_left_shift", "lshift_op", "Shift bits left."),
    ("right_shift", "rshift_op", "Arithmetic shift right (sign-filling for signed types)."),
    ("bitwise_right_shift", "rshift_op", "Arithmetic shift right."),
    ("logical_and", "logical_and_op", "Truth value of x1 AND x2."),
    ("logical_or", "logical_or_op", "Truth value of x1 OR x2."),
    ("logical_xor", "logical_xor_op", "Truth value of x1 XOR x2."),
]:
    _binary(_name, _op, _doc)


def float_power(x1, x2, /, out=None, **kwargs):
    """x1 ** x2 computed in float64 (NumPy float_power)."""
    from . import creation
    import numpy as np
    a = creation.asarray(x1).astype(np.float64)
    return _to_out(ew.binary("pow_op", a, x2), out)


def divmod(x1, x2, /):
    return ew.binary("floor_divide_op", x1, x2), ew.binary("mod_op", x1, x2)


__all__ += ["float_power", "divmod"]


for _name, _op, _doc in [
    ("spacing", "spacing_op", "Distance to the next representable magnitude, signed like x."),
    ("bitwise_count", "bitwise_count_op", "Number of 1-bits in |x|."),
    ("conjugate", "positive_op", "Complex conjugate (the identity for real dtypes)."),
    ("conj", "positive_op", "Complex conjugate (the identity for real dtypes)."),
]:
    _unary(_name, _op, _doc)

for _name, _op, _doc in [
    ("ldexp", "ldexp_op", "x1 * 2**x2."),
    ("gcd", "gcd_op", "Greatest common divisor of |x1| and |x2|."),
    ("lcm", "lcm_op", "Lowest common multiple of |x1| and |x2|."),
]:
    _binary(_name, _op, _doc)


def frexp(x, /):
    """(mantissa, int32 exponent) with x = mantissa * 2**exponent."""
    import numpy as np
    return ew.unary("frexp_mant_op", x), ew.unary("frexp_exp_op", x).astype(np.int32)


def modf(x, /):
    """(fractional part, integral part), both with the sign of x."""
    from . import creation
    from ._dtypes import ufunc_result_dtype
    import numpy as np
    xa = creation.asarray(x)
    fdt = ufunc_result_dtype(np.sin, xa.dtype)
    return ew.unary("modf_frac_op", xa), ew.unary("trunc_op", xa.astype(fdt))


def vecdot(x1, x2, /, *, axis=-1):
    """Dot products of vectors along ``axis`` (real dtypes)."""
    from .reductions import sum as _sum
    return _sum(ew.binary("mul_op", x1, x2), axis=axis)


def matvec(x1, x2, /):
    """Matrix-vector products over the last two / last dimension."""
    from .linalg_top import matmul
    from . import creation
    v = creation.asarray(x2)
    return matmul(x1, v.reshape(tuple(v.shape) + (1,))).squeeze(-1)


def vecmat(x1, x2, /):
    """Vector-matrix products over the last dimension / last two."""
    from .linalg_top import matmul
    from . import creation
    v = creation.asarray(x1)
    r = matmul(v.reshape(tuple(v.shape[:-1]) + (1, v.shape[-1])), x2)
    return r.squeeze(-2)


__all__ += ["frexp", "modf", "vecdot", "matvec", "vecmat"]
