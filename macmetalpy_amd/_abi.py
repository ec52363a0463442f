"""Numeric codes of the libmmp_hip.so C ABI (mirror of include/mmp_hip.h).

The op names are the reference's kernel names (``"add_op"``, ``"sin_op"``,
... -- src/macmetalpy/_kernels.py:49-402, ndarray.py:74-111) so that the
dispatch code reads like the reference's; each maps to the C op code, the
NumPy ufunc whose type resolution and semantics the op follows, and the
device function of csrc/mmp_ops.h that the fusion engine emits.
"""
from __future__ import annotations

import numpy as np

# ---- status codes -------------------------------------------------------
MMP_OK = 0
MMP_E_NODEVICE = 1
MMP_E_HIP = 2
MMP_E_OOM = 3
MMP_E_ARG = 4
MMP_E_UNSUPPORTED = 5
MMP_E_RTC = 6
MMP_E_INJECTED = 7
MMP_E_WAIT = 8

# ---- dtype codes ----------------------------------------------------------
DTYPE_CODES: dict[np.dtype, int] = {
    np.dtype(np.bool_): 0,
    np.dtype(np.int16): 1,
    np.dtype(np.uint16): 2,
    np.dtype(np.int32): 3,
    np.dtype(np.uint32): 4,
    np.dtype(np.int64): 5,
    np.dtype(np.uint64): 6,
    np.dtype(np.float16): 7,
    np.dtype(np.float32): 8,
    np.dtype(np.float64): 9,
}
MMP_BF16 = 10

# C++ type names used by generated (hiprtc) kernels.
CTYPE_NAMES: dict[np.dtype, str] = {
    np.dtype(np.bool_): "bool",
    np.dtype(np.int16): "mmp_i16",
    np.dtype(np.uint16): "mmp_u16",
    np.dtype(np.int32): "mmp_i32",
    np.dtype(np.uint32): "mmp_u32",
    np.dtype(np.int64): "mmp_i64",
    np.dtype(np.uint64): "mmp_u64",
    np.dtype(np.float16): "mmp_half",
    np.dtype(np.float32): "float",
    np.dtype(np.float64): "double",
}

# Ops the precompiled unary kernels (mmp_unary) also define for integer
# dtypes; they define every op for float dtypes and none for bool (the
# generated kernels cover the rest).  Mirrors UnaryOk in elementwise.hip.
INT_UNARY_OPS = frozenset({"negative_op", "positive_op", "abs_op", "sign_op", "square_op",
                           "reciprocal_op", "floor_op", "ceil_op", "rint_op", "trunc_op"})


def precompiled_unary_ok(op_name: str, dtype) -> bool:
    """True if mmp_unary defines ``op_name`` for ``dtype``."""
    kind = np.dtype(dtype).kind
    return op_name in UNARY_OPS and (kind == "f" or (kind in "iu" and op_name in INT_UNARY_OPS))


# op_name -> (code, numpy ufunc, mmp_ops.h function)
UNARY_OPS: dict[str, tuple[int, np.ufunc, str]] = {
    "neg_op": (0, np.negative, "op_neg"),
    "negative_op": (0, np.negative, "op_neg"),
    "positive_op": (1, np.positive, "op_positive"),
    "abs_op": (2, np.absolute, "op_abs"),
    "sign_op": (3, np.sign, "op_sign"),
    "square_op": (4, np.square, "op_square"),
    "reciprocal_op": (5, np.reciprocal, "op_reciprocal"),
    "sqrt_op": (6, np.sqrt, "op_sqrt"),
    "cbrt_op": (7, np.cbrt, "op_cbrt"),
    "exp_op": (8, np.exp, "op_exp"),
    "exp2_op": (9, np.exp2, "op_exp2"),
    "expm1_op": (10, np.expm1, "op_expm1"),
    "log_op": (11, np.log, "op_log"),
    "log2_op": (12, np.log2, "op_log2"),
    "log10_op": (13, np.log10, "op_log10"),
    "log1p_op": (14, np.log1p, "op_log1p"),
    "sin_op": (15, np.sin, "op_sin"),
    "cos_op": (16, np.cos, "op_cos"),
    "tan_op": (17, np.tan, "op_tan"),
    "asin_op": (18, np.arcsin, "op_arcsin"),
    "acos_op": (19, np.arccos, "op_arccos"),
    "atan_op": (20, np.arctan, "op_arctan"),
    "sinh_op": (21, np.sinh, "op_sinh"),
    "cosh_op": (22, np.cosh, "op_cosh"),
    "tanh_op": (23, np.tanh, "op_tanh"),
    "asinh_op": (24, np.arcsinh, "op_arcsinh"),
    "acosh_op": (25, np.arccosh, "op_arccosh"),
    "atanh_op": (26, np.arctanh, "op_arctanh"),
    "floor_op": (27, np.floor, "op_floor"),
    "ceil_op": (28, np.ceil, "op_ceil"),
    "rint_op": (29, np.rint, "op_rint"),
    "trunc_op": (30, np.trunc, "op_trunc"),
    "degrees_op": (31, np.degrees, "op_degrees"),
    "radians_op": (32, np.radians, "op_radians"),
}

BINARY_OPS: dict[str, tuple[int, np.ufunc, str]] = {
    "add_op": (0, np.add, "op_add"),
    "sub_op": (1, np.subtract, "op_subtract"),
    "mul_op": (2, np.multiply, "op_multiply"),
    "div_op": (3, np.true_divide, "op_true_divide"),
    "floor_divide_op": (4, np.floor_divide, "op_floor_divide"),
    "mod_op": (5, np.remainder, "op_remainder"),
    "pow_op": (6, np.power, "op_power"),
    "max_op": (7, np.maximum, "op_maximum"),
    "min_op": (8, np.minimum, "op_minimum"),
    "fmax_op": (9, np.fmax, "op_fmax"),
    "fmin_op": (10, np.fmin, "op_fmin"),
    "atan2_op": (11, np.arctan2, "op_arctan2"),
    "hypot_op": (12, np.hypot, "op_hypot"),
    "fmod_op": (13, np.fmod, "op_fmod"),
    "copysign_op": (14, np.copysign, "op_copysign"),
    "nextafter_op": (15, np.nextafter, "op_nextafter"),
    "logaddexp_op": (16, np.logaddexp, "op_logaddexp"),
    "logaddexp2_op": (17, np.logaddexp2, "op_logaddexp2"),
    "heaviside_op": (18, np.heaviside, "op_heaviside"),
}

# Comparisons (reference _kernels.py:764-867, which writes int/uchar): bool
# results, operands compared in their NumPy common dtype.  Generated-kernel
# only (no precompiled entry point).
COMPARE_OPS: dict[str, tuple[np.ufunc, str]] = {
    "lt_op": (np.less, "<"),
    "le_op": (np.less_equal, "<="),
    "gt_op": (np.greater, ">"),
    "ge_op": (np.greater_equal, ">="),
    "eq_op": (np.equal, "=="),
    "ne_op": (np.not_equal, "!="),
}

# Ops the fusion engine generates kernels for, with no precompiled entry
# point (reference: bitwise_ops.py:58-93, logic_ops.py:45-63,
# math_ops.py:558-578, ufunc_ops.py:352): op_name -> (numpy ufunc,
# mmp_ops.h function).
EXPR_UNARY_OPS: dict[str, tuple[np.ufunc, str]] = {
    "invert_op": (np.invert, "op_invert"),
    "logical_not_op": (np.logical_not, "op_logical_not"),
    "isnan_op": (np.isnan, "op_isnan"),
    "isinf_op": (np.isinf, "op_isinf"),
    "isfinite_op": (np.isfinite, "op_isfinite"),
    "signbit_op": (np.signbit, "op_signbit"),
    "spacing_op": (np.spacing, "op_spacing"),
    "bitwise_count_op": (np.bitwise_count, "op_bitwise_count"),
    # frexp / modf have two outputs; each output is its own op, typed like
    # np.sin (integers -> float64, float16 stays float16), as NumPy types them
    "frexp_mant_op": (np.sin, "op_frexp_mant"),
    "frexp_exp_op": (np.sin, "op_frexp_exp"),
    "modf_frac_op": (np.sin, "op_modf_frac"),
}
EXPR_BINARY_OPS: dict[str, tuple[np.ufunc, str]] = {
    "bit_and_op": (np.bitwise_and, "op_bitwise_and"),
    "bit_or_op": (np.bitwise_or, "op_bitwise_or"),
    "bit_xor_op": (np.bitwise_xor, "op_bitwise_xor"),
    "lshift_op": (np.left_shift, "op_left_shift"),
    "rshift_op": (np.right_shift, "op_right_shift"),
    "logical_and_op": (np.logical_and, "op_logical_and"),
    "logical_or_op": (np.logical_or, "op_logical_or"),
    "logical_xor_op": (np.logical_xor, "op_logical_xor"),
    "ldexp_op": (np.ldexp, "op_ldexp"),
    "gcd_op": (np.gcd, "op_gcd"),
    "lcm_op": (np.lcm, "op_lcm"),
}
# Ops with a bool result that read their operands in the operands' own
# (common) dtype, like the comparisons.
BOOL_RESULT_OPS = frozenset({"logical_not_op", "isnan_op", "isinf_op", "isfinite_op",
                             "signbit_op", "logical_and_op", "logical_or_op",
                             "logical_xor_op"})

# Unary ops that read their operand in its own dtype (the result has
# another one).
OWN_INPUT_OPS = frozenset({"bitwise_count_op"})

# Ops with a fast_math form in mmp_ops.h (``<fn>_fast``: hardware
# transcendentals for float32 / float16; other dtypes take the accurate op).
FAST_MATH_OPS = frozenset({
    "exp_op", "exp2_op", "log_op", "log2_op", "log10_op", "sin_op", "cos_op", "tan_op",
    "sqrt_op", "reciprocal_op", "tanh_op", "sinh_op", "cosh_op", "div_op", "pow_op",
})

# op_name -> mmp_ops.h function, for every unary / binary op
UNARY_FN = {k: v[2] for k, v in UNARY_OPS.items()}
UNARY_FN.update({k: v[1] for k, v in EXPR_UNARY_OPS.items()})
BINARY_FN = {k: v[2] for k, v in BINARY_OPS.items()}
BINARY_FN.update({k: v[1] for k, v in EXPR_BINARY_OPS.items()})

REDUCE_SUM, REDUCE_PROD, REDUCE_MAX, REDUCE_MIN, REDUCE_MEAN = 0, 1, 2, 3, 4
REDUCE_ARGMAX, REDUCE_ARGMIN = 5, 6
REDUCE_NANSUM, REDUCE_NANPROD, REDUCE_NANMAX, REDUCE_NANMIN, REDUCE_NANMEAN = 7, 8, 9, 10, 11
REDUCE_NANARGMAX, REDUCE_NANARGMIN = 12, 13
ARG_NONE = 0x7FFFFFFFFFFFFFFF  # index a NaN arg-reduction reports for an all-NaN slice
SCAN_CUMSUM, SCAN_CUMPROD = 0, 1

# Exported C symbols (kept in sync with include/mmp_hip.h by a test).
EXPORTS = (
    "mmp_init", "mmp_device_count", "mmp_device_info", "mmp_last_error",
    "mmp_alloc", "mmp_free", "mmp_empty_cache", "mmp_memory_stats",
    "mmp_h2d", "mmp_d2h", "mmp_d2d", "mmp_host_alloc", "mmp_host_free", "mmp_sync",
    "mmp_stream",
    "mmp_event_create", "mmp_event_record", "mmp_event_elapsed_ms",
    "mmp_event_destroy",
    "mmp_unary", "mmp_binary", "mmp_binary_scalar", "mmp_copy",
    "mmp_copy_strided", "mmp_fill",
    "mmp_reduce", "mmp_reduce_noalloc", "mmp_argreduce", "mmp_scan", "mmp_matmul",
    "mmp_sort", "mmp_searchsorted", "mmp_take", "mmp_gather", "mmp_scatter", "mmp_nonzero",
    "mmp_mask_tile_counts", "mmp_mask_positions", "mmp_mask_compact",
    "mmp_bincount", "mmp_histogram",
    "mmp_lu", "mmp_lu_solve", "mmp_cholesky", "mmp_qr", "mmp_qr_q", "mmp_eigh", "mmp_svd",
    "mmp_rtc_compile", "mmp_rtc_build", "mmp_rtc_launch", "mmp_rtc_launch_threads",
    "mmp_wait_status",
    "mmp_debug_fail_next",
)
