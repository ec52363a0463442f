// mmp_ops.h -- per-element operations with NumPy semantics, for gfx950.
//
// One definition of every elementwise op, included both by the precompiled
// kernels (elementwise.hip, built by hipcc) and by the kernels the fusion
// engine generates at run time (compiled by hiprtc).  Because both paths
// evaluate the same functions with the same compile flags
// (-ffp-contract=off), a fused expression is bit-identical to the same
// expression evaluated op by op.
//
// The semantics follow what the reference computes on its CPU/NumPy path
// (src/macmetalpy/ndarray.py:74-111 maps every op to a numpy ufunc), NOT its
// Metal shaders, which differ from NumPy in several places:
//  - integer floor_divide truncates there (_kernels.py:44); here it floors;
//  - remainder there is a - floor_divide(a, b) * b in three launches
//    (math_ops.py:540-548); here it is one op with NumPy's sign rules;
//  - expm1 / log1p there are exp(x)-1 / log(1+x) (_kernels.py:263, 269);
//    here they are the accurate library functions.
// Float16 values are widened to float, computed, and rounded back once, as
// NumPy's float16 loops do.  Integer arithmetic wraps (two's complement).
#pragma once

#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

typedef _Float16 mmp_half;
typedef short mmp_i16;
typedef unsigned short mmp_u16;
typedef int mmp_i32;
typedef unsigned int mmp_u32;
typedef long long mmp_i64;
typedef unsigned long long mmp_u64;

#define MMP_DI __device__ __forceinline__

// ---------------------------------------------------------------- traits
template <typename T> struct mmp_t;
template <> struct mmp_t<float> {
  enum { is_float = 1, is_signed = 1, is_bool = 0 };
  typedef float C;
  typedef float U;
};
template <> struct mmp_t<double> {
  enum { is_float = 1, is_signed = 1, is_bool = 0 };
  typedef double C;
  typedef double U;
};
template <> struct mmp_t<mmp_half> {
  enum { is_float = 1, is_signed = 1, is_bool = 0 };
  typedef float C;
  typedef float U;
};
template <> struct mmp_t<mmp_i16> {
  enum { is_float = 0, is_signed = 1, is_bool = 0 };
  typedef mmp_i16 C;
  typedef mmp_u16 U;
  static constexpr mmp_i16 lowest = (mmp_i16)(-32767 - 1);
};
template <> struct mmp_t<mmp_u16> {
  enum { is_float = 0, is_signed = 0, is_bool = 0 };
  typedef mmp_u16 C;
  typedef mmp_u16 U;
  static constexpr mmp_u16 lowest = 0;
};
template <> struct mmp_t<mmp_i32> {
  enum { is_float = 0, is_signed = 1, is_bool = 0 };
  typedef mmp_i32 C;
  typedef mmp_u32 U;
  static constexpr mmp_i32 lowest = (-2147483647 - 1);
};
template <> struct mmp_t<mmp_u32> {
  enum { is_float = 0, is_signed = 0, is_bool = 0 };
  typedef mmp_u32 C;
  typedef mmp_u32 U;
  static constexpr mmp_u32 lowest = 0u;
};
template <> struct mmp_t<mmp_i64> {
  enum { is_float = 0, is_signed = 1, is_bool = 0 };
  typedef mmp_i64 C;
  typedef mmp_u64 U;
  static constexpr mmp_i64 lowest = (-9223372036854775807LL - 1);
};
template <> struct mmp_t<mmp_u64> {
  enum { is_float = 0, is_signed = 0, is_bool = 0 };
  typedef mmp_u64 C;
  typedef mmp_u64 U;
  static constexpr mmp_u64 lowest = 0ull;
};
template <> struct mmp_t<bool> {
  enum { is_float = 0, is_signed = 0, is_bool = 1 };
  typedef bool C;
  typedef bool U;
  static constexpr bool lowest = false;
};

// --------------------------------------------- float / double math overloads
#define MMP_MATH1(name, f32, f64)                                             \
  MMP_DI float mm_##name(float x) { return f32(x); }                          \
  MMP_DI double mm_##name(double x) { return f64(x); }
#define MMP_MATH2(name, f32, f64)                                             \
  MMP_DI float mm_##name(float x, float y) { return f32(x, y); }              \
  MMP_DI double mm_##name(double x, double y) { return f64(x, y); }

MMP_MATH1(sqrt, sqrtf, sqrt)
MMP_MATH1(cbrt, cbrtf, cbrt)
MMP_MATH1(exp2, exp2f, exp2)
MMP_MATH1(expm1, expm1f, expm1)
MMP_MATH1(log, logf, log)
MMP_MATH1(log2, log2f, log2)
MMP_MATH1(log10, log10f, log10)
MMP_MATH1(sin, sinf, sin)
MMP_MATH1(cos, cosf, cos)
MMP_MATH1(tan, tanf, tan)
MMP_MATH1(asin, asinf, asin)
MMP_MATH1(acos, acosf, acos)
MMP_MATH1(atan, atanf, atan)
MMP_MATH1(sinh, sinhf, sinh)
MMP_MATH1(cosh, coshf, cosh)
MMP_MATH1(asinh, asinhf, asinh)
MMP_MATH1(acosh, acoshf, acosh)
MMP_MATH1(atanh, atanhf, atanh)
MMP_MATH1(floor, floorf, floor)
MMP_MATH1(ceil, ceilf, ceil)
MMP_MATH1(rint, rintf, rint)
MMP_MATH1(trunc, truncf, trunc)
MMP_MATH1(fabs, fabsf, fabs)
MMP_MATH2(pow, powf, pow)
MMP_MATH2(atan2, atan2f, atan2)
MMP_MATH2(hypot, hypotf, hypot)
MMP_MATH2(fmod, fmodf, fmod)
MMP_MATH2(copysign, copysignf, copysign)
MMP_MATH2(nextafter, nextafterf, nextafter)

// log1p for float32.  The device library's log1pf costs ~125 VALU
// instructions, which made it the bottleneck of fused chains; this one
// costs ~25.  Method: m = 1 + x; k is chosen so that m 2^-k lies in
// [0.75, 1.5); f = x 2^-k + (2^-k - 1) (v_ldexp scalings; for the small k
// where it matters the sum is exact by Sterbenz's lemma), so f carries no
// rounding error of 1 + x; then log1p(x) = k ln2 + f + f^2 Q(f), where Q is
// a degree-9 polynomial fitted (iteratively reweighted least squares on
// Chebyshev nodes) to (log1p(f) - f) / f^2 on [-0.25, 0.5], relative error
// of f + f^2 Q below 7e-10.  ln2 is split into a 12-bit head (k ln2_hi is
// exact for |k| <= 128) and a tail.  k = 0 needs no special case (f = x and
// k ln2 adds zero) except for -0.0, which the final select returns as is.
// Max error over every float32 input: 1.27 ULP of the exact value.
MMP_DI float mm_log1p_core(float x) {
  const float m = 1.0f + x;
  const int k = (int)(__builtin_bit_cast(unsigned, m) - 0x3f400000u) >> 23;
  const float f = ldexpf(x, -k) + (ldexpf(1.0f, -k) - 1.0f);
  float q = 0.03731892257928848f;
  q = __builtin_fmaf(q, f, -0.09126769751310349f);
  q = __builtin_fmaf(q, f, 0.11755406111478806f);
  q = __builtin_fmaf(q, f, -0.12750042974948883f);
  q = __builtin_fmaf(q, f, 0.14272044599056244f);
  q = __builtin_fmaf(q, f, -0.16652290523052216f);
  q = __builtin_fmaf(q, f, 0.1999962329864502f);
  q = __builtin_fmaf(q, f, -0.2500028908252716f);
  q = __builtin_fmaf(q, f, 0.33333343267440796f);
  q = __builtin_fmaf(q, f, -0.4999999701976776f);
  const float p = __builtin_fmaf(f * f, q, f);
  const float kf = (float)k;
  const float ln2_hi = __builtin_bit_cast(float, 0x3f317000u);  // 0.693115234375
  const float ln2_lo = 3.1946183e-05f;                          // ln2 - ln2_hi
  float r = __builtin_fmaf(kf, ln2_hi, __builtin_fmaf(kf, ln2_lo, p));
  const float inf = __builtin_inff();
  return (x == 0.0f || x == inf) ? x : r;  // keeps -0.0; +inf -> +inf
}
MMP_DI float mm_log1p(float x) {
  const float inf = __builtin_inff();
  // x <= -1 (the core value is finite or NaN there): adding -inf or NaN
  // gives log1p's value; elsewhere -0.0 changes nothing.  An add rather than
  // a select keeps the compiler from guarding the evaluation by a branch.
  return mm_log1p_core(x) + (x > -1.0f ? -0.0f : (x == -1.0f ? -inf : __builtin_nanf("")));
}
// The same function for arguments known to be >= 0 or NaN (x*x, |x|, ...):
// bit for bit mm_log1p there (NaN payloads aside), without the x <= -1
// cases.
MMP_DI float mm_log1p_nonneg(float x) { return mm_log1p_core(x); }
MMP_DI double mm_log1p(double x) { return log1p(x); }
MMP_DI double mm_log1p_nonneg(double x) { return log1p(x); }

// exp for float32 (the standard reduction: e^x = 2^n 2^f with
// x log2(e) = n + f + l carried as a head and an fma-recovered tail,
// |f| <= 1/2; v_exp_f32 of f + l, v_ldexp_f32 by n, which also rounds
// denormal results).  Written here rather than taken from the device
// library so that the same arithmetic exists without the overflow case
// (mm_exp_nonpos, for arguments known to be <= 0 or NaN: exp(-|x|),
// exp(-x*x)), bit for bit mm_exp there (NaN payloads aside).  Max error
// over every float32 input: 0.89 ULP of the exact value (the device
// library's expf: 1.0).
MMP_DI float mm_exp_core(float x) {
  const float l2e = __builtin_bit_cast(float, 0x3fb8aa3bu);     // log2(e) rounded
  const float l2e_lo = __builtin_bit_cast(float, 0x32a5705fu);  // log2(e) - l2e
  const float ph = x * l2e;
  const float pl = __builtin_fmaf(x, l2e_lo, __builtin_fmaf(x, l2e, -ph));
  const float n = __builtin_rintf(ph);
  const float r = ldexpf(__builtin_amdgcn_exp2f((ph - n) + pl), (int)n);
  return x < -104.0f ? 0.0f : r;  // below half the least denormal; also -inf
}
MMP_DI float mm_exp(float x) { return x > 89.0f ? __builtin_inff() : mm_exp_core(x); }
MMP_DI float mm_exp_nonpos(float x) { return mm_exp_core(x); }
MMP_DI double mm_exp(double x) { return exp(x); }
MMP_DI double mm_exp_nonpos(double x) { return exp(x); }

// tanh for float32, branch-free (the device library's tanhf branches on
// |x| < 0.625, and in a fused loop over random data both sides run with
// exec-mask juggling in between).  Both forms are evaluated and selected:
//  - |x| < 0.625: |x| + |x|^3 P(x^2), P of degree 4 fitted (iteratively
//    reweighted least squares on Chebyshev nodes, 40-digit tanh) to
//    (tanh(x) - x) / x^3; relative error of the form 4.4e-9;
//  - otherwise 1 - 2 / (e + 1) with e = e^{2|x|} = 2^y, y = 2|x| log2(e)
//    carried as a float head and an fma-recovered tail (v_exp_f32 of the
//    head, times 1 + tail ln2), then v_rcp_f32.  |x| is clamped to 16
//    first (tanh is 1 in float32 from 9.01 on), so e stays finite.
// NaN takes the first form (the compare is false) and propagates.  Max
// error over every float32 input: 1.56 ULP of the exact value (the
// library's tanhf: 1.41).
MMP_DI float mm_tanh(float x) {
  const float ax = __builtin_fabsf(x);
  const float s = x * x;
  float p = -0.0057049887254834175f;
  p = __builtin_fmaf(p, s, 0.02063908986747265f);
  p = __builtin_fmaf(p, s, -0.05373971536755562f);
  p = __builtin_fmaf(p, s, 0.13331441581249237f);
  p = __builtin_fmaf(p, s, -0.3333328068256378f);
  const float small = __builtin_fmaf(ax * s, p, ax);
  const float ac = __builtin_fminf(ax, 16.0f);
  const float k_hi = __builtin_bit_cast(float, 0x4038aa3bu);  // 2 log2(e) rounded
  const float k_lo = __builtin_bit_cast(float, 0x33257060u);  // 2 log2(e) - k_hi
  const float y = ac * k_hi;
  const float y_lo = __builtin_fmaf(ac, k_lo, __builtin_fmaf(ac, k_hi, -y));
  float e = __builtin_amdgcn_exp2f(y);
  e = __builtin_fmaf(e, y_lo * 0.693147180559945309f, e);
  const float big = __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
  return __builtin_copysignf(ax >= 0.625f ? big : small, x);
}
MMP_DI double mm_tanh(double x) { return tanh(x); }

MMP_DI bool mm_isnan(float x) { return x != x; }
MMP_DI bool mm_isnan(double x) { return x != x; }
MMP_DI float mm_nan(float) { return __builtin_nanf(""); }
MMP_DI double mm_nan(double) { return __builtin_nan(""); }

// 180/pi and pi/180 as NumPy's float32 loops use them: the quotient of the
// float32 constants, evaluated in float32 (180.0f / NPY_PIf); in double for
// float64.
MMP_DI float mm_rad2deg(float) { return 180.0f / 3.14159265358979323846f; }
MMP_DI double mm_rad2deg(double) { return 180.0 / 3.14159265358979323846; }
MMP_DI float mm_deg2rad(float) { return 3.14159265358979323846f / 180.0f; }
MMP_DI double mm_deg2rad(double) { return 3.14159265358979323846 / 180.0; }

// float32 functions evaluated through float64 and rounded once.  Used where
// the float32 device library is more than 2 ULP away from NumPy's results
// (exp2, log10, arcsin, arccos, arctan2); the float64 path is within
// 0.5 ULP (+ the float64 error) of the correctly rounded value.
MMP_DI float mm_exp2_acc(float x) { return (float)exp2((double)x); }
MMP_DI double mm_exp2_acc(double x) { return exp2(x); }
MMP_DI float mm_log10_acc(float x) { return (float)log10((double)x); }
MMP_DI double mm_log10_acc(double x) { return log10(x); }
MMP_DI float mm_asin_acc(float x) { return (float)asin((double)x); }
MMP_DI double mm_asin_acc(double x) { return asin(x); }
MMP_DI float mm_acos_acc(float x) { return (float)acos((double)x); }
MMP_DI double mm_acos_acc(double x) { return acos(x); }
MMP_DI float mm_atan2_acc(float y, float x) { return (float)atan2((double)y, (double)x); }
MMP_DI double mm_atan2_acc(double y, double x) { return atan2(y, x); }
MMP_DI float mm_ln2(float) { return 0.693147180559945309417f; }
MMP_DI double mm_ln2(double) { return 0.693147180559945309417; }
MMP_DI float mm_log2e(float) { return 1.442695040888963407360f; }
MMP_DI double mm_log2e(double) { return 1.442695040888963407360; }

// ------------------------------------------------------ integer helpers
template <typename T> MMP_DI T iwrap_add(T a, T b) {
  typedef typename mmp_t<T>::U U;
  return (T)(U)((U)a + (U)b);
}
template <typename T> MMP_DI T iwrap_sub(T a, T b) {
  typedef typename mmp_t<T>::U U;
  return (T)(U)((U)a - (U)b);
}
template <typename T> MMP_DI T iwrap_mul(T a, T b) {
  typedef typename mmp_t<T>::U U;
  // 16-bit operands promote to int in C++; multiply in 32-bit unsigned.
  if constexpr (sizeof(T) < 4) {
    return (T)(U)((unsigned int)(U)a * (unsigned int)(U)b);
  } else {
    return (T)(U)((U)a * (U)b);
  }
}

// =====================================================================
// Unary ops.  C = compute type; results rounded to T once.
// =====================================================================
template <typename T> MMP_DI T op_neg(T x) {
  if constexpr (mmp_t<T>::is_float) {
    return (T)(-(typename mmp_t<T>::C)x);
  } else {
    return iwrap_sub((T)0, x);
  }
}
template <typename T> MMP_DI T op_positive(T x) { return x; }
template <typename T> MMP_DI T op_abs(T x) {
  if constexpr (mmp_t<T>::is_float) {
    return (T)mm_fabs((typename mmp_t<T>::C)x);
  } else if constexpr (mmp_t<T>::is_signed) {
    return x < 0 ? iwrap_sub((T)0, x) : x;  // abs(INT_MIN) == INT_MIN
  } else {
    return x;
  }
}
template <typename T> MMP_DI T op_sign(T x) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    C v = (C)x;
    if (mm_isnan(v)) return (T)v;
    return (T)(v > (C)0 ? (C)1 : (v < (C)0 ? (C)-1 : (C)0));
  } else if constexpr (mmp_t<T>::is_signed) {
    return (T)((x > 0) - (x < 0));
  } else {
    return (T)(x > 0 ? 1 : 0);
  }
}
template <typename T> MMP_DI T op_square(T x) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    return (T)((C)x * (C)x);
  } else {
    return iwrap_mul(x, x);
  }
}
template <typename T> MMP_DI T op_reciprocal(T x) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    return (T)((C)1 / (C)x);
  } else {
    // numpy's integer reciprocal converts 1.0 / x to the type: for x == 0 the
    // conversion of inf gives the lowest value of a 32- or 64-bit signed
    // type, and 0 for narrower signed types and every unsigned type (whose
    // conversions go through a wider signed integer and keep its low bits)
    if (x == 0) return (mmp_t<T>::is_signed && sizeof(T) >= 4) ? mmp_t<T>::lowest : (T)0;
    if constexpr (mmp_t<T>::is_signed) {
      return (T)(x == 1 ? 1 : (x == -1 ? -1 : 0));
    } else {
      return (T)(x == 1 ? 1 : 0);
    }
  }
}

#define MMP_FLOAT_UNARY(NAME, EXPR)                                           \
  template <typename T> MMP_DI T op_##NAME(T x_) {                            \
    typedef typename mmp_t<T>::C C;                                           \
    C x = (C)x_;                                                              \
    return (T)(EXPR);                                                         \
  }

MMP_FLOAT_UNARY(sqrt, mm_sqrt(x))
MMP_FLOAT_UNARY(cbrt, mm_cbrt(x))
MMP_FLOAT_UNARY(exp, mm_exp(x))
MMP_FLOAT_UNARY(exp_nonpos, mm_exp_nonpos(x))
MMP_FLOAT_UNARY(exp2, mm_exp2_acc(x))
MMP_FLOAT_UNARY(expm1, mm_expm1(x))
MMP_FLOAT_UNARY(log, mm_log(x))
MMP_FLOAT_UNARY(log2, mm_log2(x))
MMP_FLOAT_UNARY(log10, mm_log10_acc(x))
MMP_FLOAT_UNARY(log1p, mm_log1p(x))
MMP_FLOAT_UNARY(log1p_nonneg, mm_log1p_nonneg(x))
MMP_FLOAT_UNARY(sin, mm_sin(x))
MMP_FLOAT_UNARY(cos, mm_cos(x))
MMP_FLOAT_UNARY(tan, mm_tan(x))
MMP_FLOAT_UNARY(arcsin, mm_asin_acc(x))
MMP_FLOAT_UNARY(arccos, mm_acos_acc(x))
MMP_FLOAT_UNARY(arctan, mm_atan(x))
MMP_FLOAT_UNARY(sinh, mm_sinh(x))
MMP_FLOAT_UNARY(cosh, mm_cosh(x))
MMP_FLOAT_UNARY(tanh, mm_tanh(x))
MMP_FLOAT_UNARY(arcsinh, mm_asinh(x))
MMP_FLOAT_UNARY(arccosh, mm_acosh(x))
MMP_FLOAT_UNARY(arctanh, mm_atanh(x))
MMP_FLOAT_UNARY(degrees, x * mm_rad2deg(x))
MMP_FLOAT_UNARY(radians, x * mm_deg2rad(x))

// floor/ceil/rint/trunc keep integer inputs unchanged (numpy returns the
// integer dtype for floor/ceil/trunc of integers).
#define MMP_ROUNDING_UNARY(NAME, FN)                                          \
  template <typename T> MMP_DI T op_##NAME(T x) {                             \
    if constexpr (mmp_t<T>::is_float) {                                       \
      return (T)FN((typename mmp_t<T>::C)x);                                  \
    } else {                                                                  \
      return x;                                                               \
    }                                                                         \
  }
MMP_ROUNDING_UNARY(floor, mm_floor)
MMP_ROUNDING_UNARY(ceil, mm_ceil)
MMP_ROUNDING_UNARY(rint, mm_rint)
MMP_ROUNDING_UNARY(trunc, mm_trunc)

// =====================================================================
// Binary ops
// =====================================================================
template <typename T> MMP_DI T op_add(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    return (T)((C)a + (C)b);
  } else if constexpr (mmp_t<T>::is_bool) {
    return a || b;
  } else {
    return iwrap_add(a, b);
  }
}
template <typename T> MMP_DI T op_subtract(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    return (T)((C)a - (C)b);
  } else {
    return iwrap_sub(a, b);
  }
}
template <typename T> MMP_DI T op_multiply(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    return (T)((C)a * (C)b);
  } else if constexpr (mmp_t<T>::is_bool) {
    return a && b;
  } else {
    return iwrap_mul(a, b);
  }
}
template <typename T> MMP_DI T op_true_divide(T a, T b) {
  typedef typename mmp_t<T>::C C;
  return (T)((C)a / (C)b);
}

// NumPy's float divmod (numpy/_core/src/npymath/npy_math_internal.h.src,
// npy_divmod): the quotient is (a - fmod(a, b)) / b, corrected towards
// -inf and snapped to the nearest integer; the remainder takes b's sign.
template <typename C> MMP_DI C mm_divmod(C a, C b, C *modulus) {
  C mod = mm_fmod(a, b);
  if (!(b != (C)0)) {  // b == 0 (b is not NaN here)
    *modulus = mod;
    return a / b;
  }
  C div = (a - mod) / b;
  if (mod != (C)0) {
    if ((b < (C)0) != (mod < (C)0)) {
      mod += b;
      div -= (C)1;
    }
  } else {
    mod = mm_copysign((C)0, b);
  }
  C floordiv;
  if (div != (C)0) {
    floordiv = mm_floor(div);
    if (div - floordiv > (C)0.5) floordiv += (C)1;
  } else {
    floordiv = mm_copysign((C)0, a / b);
  }
  *modulus = mod;
  return floordiv;
}

template <typename T> MMP_DI T op_floor_divide(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    C x = (C)a, y = (C)b;
    if (!(y != (C)0) && !mm_isnan(y)) return (T)(x / y);  // npy_floor_divide
    C m;
    return (T)mm_divmod(x, y, &m);
  } else {
    if (b == 0) return (T)0;  // numpy: 0 (with a divide-by-zero warning)
    if constexpr (mmp_t<T>::is_signed) {
      if (b == (T)-1) return iwrap_sub((T)0, a);  // INT_MIN // -1 wraps
      T q = (T)(a / b);
      T r = (T)(a - q * b);
      if (r != 0 && ((r < 0) != (b < 0))) q = (T)(q - 1);
      return q;
    } else {
      return (T)(a / b);
    }
  }
}

template <typename T> MMP_DI T op_remainder(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    C x = (C)a, y = (C)b;
    if (!(y != (C)0) && !mm_isnan(y)) return (T)mm_fmod(x, y);  // npy_remainder
    C m;
    mm_divmod(x, y, &m);
    return (T)m;
  } else {
    if (b == 0) return (T)0;
    if constexpr (mmp_t<T>::is_signed) {
      if (b == (T)-1) return (T)0;
      T q = (T)(a / b);
      T r = (T)(a - q * b);
      if (r != 0 && ((r < 0) != (b < 0))) r = (T)(r + b);
      return r;
    } else {
      return (T)(a % b);
    }
  }
}

template <typename T> MMP_DI T op_fmod(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    return (T)mm_fmod((C)a, (C)b);
  } else {
    if (b == 0) return (T)0;
    if constexpr (mmp_t<T>::is_signed) {
      if (b == (T)-1) return (T)0;
    }
    return (T)(a % b);  // C semantics: sign of the dividend
  }
}

template <typename T> MMP_DI T op_power(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    return (T)mm_pow((C)a, (C)b);
  } else {
    // exponentiation by squaring with wrap-around; negative exponents are
    // rejected by the host before launch (numpy raises ValueError).
    if constexpr (mmp_t<T>::is_signed) {
      if (b < 0) return (T)0;
    }
    typedef typename mmp_t<T>::U U;
    U base = (U)a, e = (U)b, r = (U)1;
    while (e) {
      if (e & (U)1) r = (U)iwrap_mul((T)r, (T)base);
      e = (U)(e >> 1);
      if (e) base = (U)iwrap_mul((T)base, (T)base);
    }
    return (T)r;
  }
}

// maximum/minimum propagate NaN; fmax/fmin ignore NaN.  On ties (+0 vs -0)
// numpy's float32/float64 loops return the second operand and its float16
// loops (npy_half_ge / npy_half_le) the first; both are reproduced.
template <typename T> MMP_DI T op_maximum(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    C x = (C)a, y = (C)b;
    if (mm_isnan(x)) return a;
    if (mm_isnan(y)) return b;
    if constexpr (sizeof(T) == 2) return x >= y ? a : b;
    return x > y ? a : b;
  } else if constexpr (mmp_t<T>::is_bool) {
    return a || b;
  } else {
    return a > b ? a : b;
  }
}
template <typename T> MMP_DI T op_minimum(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    C x = (C)a, y = (C)b;
    if (mm_isnan(x)) return a;
    if (mm_isnan(y)) return b;
    if constexpr (sizeof(T) == 2) return x <= y ? a : b;
    return x < y ? a : b;
  } else if constexpr (mmp_t<T>::is_bool) {
    return a && b;
  } else {
    return a < b ? a : b;
  }
}
template <typename T> MMP_DI T op_fmax(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    C x = (C)a, y = (C)b;
    if (mm_isnan(y)) return a;
    if (mm_isnan(x)) return b;
    if constexpr (sizeof(T) == 2) return x >= y ? a : b;
    return x > y ? a : b;
  } else {
    return op_maximum(a, b);
  }
}
template <typename T> MMP_DI T op_fmin(T a, T b) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    C x = (C)a, y = (C)b;
    if (mm_isnan(y)) return a;
    if (mm_isnan(x)) return b;
    if constexpr (sizeof(T) == 2) return x <= y ? a : b;
    return x < y ? a : b;
  } else {
    return op_minimum(a, b);
  }
}

#define MMP_FLOAT_BINARY(NAME, EXPR)                                          \
  template <typename T> MMP_DI T op_##NAME(T a_, T b_) {                      \
    typedef typename mmp_t<T>::C C;                                           \
    C a = (C)a_, b = (C)b_;                                                   \
    return (T)(EXPR);                                                         \
  }
MMP_FLOAT_BINARY(arctan2, mm_atan2_acc(a, b))
MMP_FLOAT_BINARY(hypot, mm_hypot(a, b))
MMP_FLOAT_BINARY(copysign, mm_copysign(a, b))

// nextafter steps in the representation of T itself; for float16 that is
// the half-precision bit pattern (numpy npy_half_nextafter), not float's.
template <typename T> MMP_DI T op_nextafter(T a_, T b_) {
  if constexpr (sizeof(T) == 2) {
    const unsigned short x = __builtin_bit_cast(unsigned short, a_);
    const unsigned short y = __builtin_bit_cast(unsigned short, b_);
    const float fx = (float)a_, fy = (float)b_;
    if (fx != fx || fy != fy) return (T)__builtin_nanf("");
    if (fx == fy) return a_;  // npy_half_nextafter keeps x (also for -0 vs +0)
    unsigned short r;
    if ((x & 0x7fffu) == 0) {
      r = (unsigned short)((y & 0x8000u) | 1u);  // smallest subnormal towards y
    } else if ((fx < fy) == !(x & 0x8000u)) {
      r = (unsigned short)(x + 1u);  // away from zero
    } else {
      r = (unsigned short)(x - 1u);
    }
    return __builtin_bit_cast(T, r);
  } else {
    typedef typename mmp_t<T>::C C;
    return (T)mm_nextafter((C)a_, (C)b_);
  }
}

// numpy npy_logaddexp / npy_logaddexp2
template <typename T> MMP_DI T op_logaddexp(T a_, T b_) {
  typedef typename mmp_t<T>::C C;
  C x = (C)a_, y = (C)b_;
  if (x == y) return (T)(x + mm_ln2(x));
  C d = x - y;
  if (d > (C)0) return (T)(x + mm_log1p(mm_exp(-d)));
  if (d <= (C)0) return (T)(y + mm_log1p(mm_exp(d)));
  return (T)d;  // NaN
}
template <typename T> MMP_DI T op_logaddexp2(T a_, T b_) {
  typedef typename mmp_t<T>::C C;
  C x = (C)a_, y = (C)b_;
  if (x == y) return (T)(x + (C)1);
  C d = x - y;
  if (d > (C)0) return (T)(x + mm_log2e(x) * mm_log1p(mm_exp2(-d)));
  if (d <= (C)0) return (T)(y + mm_log2e(x) * mm_log1p(mm_exp2(d)));
  return (T)d;
}
// numpy npy_heaviside
template <typename T> MMP_DI T op_heaviside(T a_, T h) {
  typedef typename mmp_t<T>::C C;
  C x = (C)a_;
  if (mm_isnan(x)) return (T)mm_nan(x);
  if (x == (C)0) return h;
  if (x < (C)0) return (T)0;
  return (T)1;
}

// =====================================================================
// Bitwise, shift, logical and predicate ops (the reference's boolean_shader,
// bool_logic_shader and predicate_shader, _kernels.py:870-1049, which work
// on int32 / uchar buffers; here every NumPy integer dtype, with NumPy's
// result dtypes).  Used by generated kernels only.
// =====================================================================
template <typename T> MMP_DI T op_bitwise_and(T a, T b) {
  if constexpr (mmp_t<T>::is_bool) return a && b;
  else return (T)(a & b);
}
template <typename T> MMP_DI T op_bitwise_or(T a, T b) {
  if constexpr (mmp_t<T>::is_bool) return a || b;
  else return (T)(a | b);
}
template <typename T> MMP_DI T op_bitwise_xor(T a, T b) {
  if constexpr (mmp_t<T>::is_bool) return a != b;
  else return (T)(a ^ b);
}
template <typename T> MMP_DI T op_invert(T a) {
  if constexpr (mmp_t<T>::is_bool) return !a;
  else return (T)~a;
}
// numpy npy_lshift / npy_rshift: a count outside [0, bits) -- negative
// counts included, read as unsigned -- shifts everything out: 0, or -1 for
// a negative value shifted right.
template <typename T> MMP_DI T op_left_shift(T a, T b) {
  typedef typename mmp_t<T>::U U;
  if ((U)b < (U)(8 * sizeof(T))) return (T)((U)a << (U)b);
  return (T)0;
}
template <typename T> MMP_DI T op_right_shift(T a, T b) {
  typedef typename mmp_t<T>::U U;
  if ((U)b < (U)(8 * sizeof(T))) return (T)(a >> b);
  if constexpr (mmp_t<T>::is_signed) return a < (T)0 ? (T)-1 : (T)0;
  return (T)0;
}
// truth value: nonzero (NaN is true), as NumPy's logical loops test it
template <typename T> MMP_DI bool mmp_truth(T v) {
  if constexpr (mmp_t<T>::is_float) return (typename mmp_t<T>::C)v != (typename mmp_t<T>::C)0;
  else return v != (T)0;
}
template <typename T> MMP_DI bool op_logical_and(T a, T b) { return mmp_truth(a) && mmp_truth(b); }
template <typename T> MMP_DI bool op_logical_or(T a, T b) { return mmp_truth(a) || mmp_truth(b); }
template <typename T> MMP_DI bool op_logical_xor(T a, T b) { return mmp_truth(a) != mmp_truth(b); }
template <typename T> MMP_DI bool op_logical_not(T a) { return !mmp_truth(a); }
template <typename T> MMP_DI bool op_isnan(T a) {
  if constexpr (mmp_t<T>::is_float) return __builtin_isnan((typename mmp_t<T>::C)a);
  else return false;
}
template <typename T> MMP_DI bool op_isinf(T a) {
  if constexpr (mmp_t<T>::is_float) return __builtin_isinf((typename mmp_t<T>::C)a);
  else return false;
}
template <typename T> MMP_DI bool op_isfinite(T a) {
  if constexpr (mmp_t<T>::is_float) return __builtin_isfinite((typename mmp_t<T>::C)a);
  else return true;
}
// sign bit of the representation: true for -0.0 and negative NaNs
template <typename T> MMP_DI bool op_signbit(T a) {
  if constexpr (mmp_t<T>::is_float) return __builtin_signbit((typename mmp_t<T>::C)a);
  else if constexpr (mmp_t<T>::is_signed) return a < (T)0;
  else return false;
}

// Unsigned integer with the size of T (bit patterns of floats).
template <int N> struct mmp_bits_of;
template <> struct mmp_bits_of<2> { typedef mmp_u16 type; };
template <> struct mmp_bits_of<4> { typedef mmp_u32 type; };
template <> struct mmp_bits_of<8> { typedef mmp_u64 type; };

// np.spacing, NumPy's two definitions: float32 / float64 take the step to
// the next value away from zero, signed like x (npy_spacing: +-0 -> the
// smallest subnormal, +-largest finite -> +-inf); float16 takes the step to
// the next value toward +inf, always positive (npy_half_spacing: 65504 ->
// inf, -0 -> the smallest subnormal).  inf and NaN give NaN.  Neighbouring
// values differ by an exactly representable step.
template <typename T> MMP_DI T op_spacing(T a) {
  if constexpr (!mmp_t<T>::is_float) {
    return a;
  } else {
    typedef typename mmp_bits_of<sizeof(T)>::type B;
    typedef typename mmp_t<T>::C C;
    const C x = (C)a;
    if (__builtin_isnan(x) || __builtin_isinf(x)) return (T)(C)__builtin_nan("");
    const B sign = (B)((B)1 << (8 * sizeof(T) - 1));
    const B b = __builtin_bit_cast(B, a);
    if ((B)(b & (B)~sign) == 0) return __builtin_bit_cast(T, (B)1);
    if constexpr (sizeof(T) == 2) {
      const B up = (b & sign) ? (B)(b - 1) : (B)(b + 1);  // toward +inf
      return (T)((C)__builtin_bit_cast(T, up) - x);
    } else {
      return (T)((C)__builtin_bit_cast(T, (B)(b + 1)) - x);  // away from zero
    }
  }
}
// np.bitwise_count: set bits of |x|
template <typename T> MMP_DI int op_bitwise_count(T a) {
  if constexpr (mmp_t<T>::is_bool) {
    return a ? 1 : 0;
  } else {
    typedef typename mmp_t<T>::U U;
    const U m = (mmp_t<T>::is_signed && a < (T)0) ? (U)((U)0 - (U)a) : (U)a;
    return __builtin_popcountll((unsigned long long)m);
  }
}
// np.frexp, as two ops: the mantissa in [0.5, 1) and the exponent (as a
// value of T, converted to int32 by the caller); 0, inf and NaN keep their
// value with exponent 0.
template <typename T> MMP_DI T op_frexp_mant(T a) {
  typedef typename mmp_t<T>::C C;
  const C x = (C)a;
  if (!__builtin_isfinite(x) || x == (C)0) return a;
  int e;
  return (T)__builtin_frexp(x, &e);
}
template <> MMP_DI float op_frexp_mant(float a) {
  if (!__builtin_isfinite(a) || a == 0.f) return a;
  int e;
  return __builtin_frexpf(a, &e);
}
template <typename T> MMP_DI T op_frexp_exp(T a) {
  typedef typename mmp_t<T>::C C;
  const C x = (C)a;
  if (!__builtin_isfinite(x) || x == (C)0) return (T)0;
  int e;
  if constexpr (sizeof(C) == 4) (void)__builtin_frexpf((float)x, &e);
  else (void)__builtin_frexp((double)x, &e);
  return (T)(C)e;
}
// np.modf fractional part (the integral part is trunc)
template <typename T> MMP_DI T op_modf_frac(T a) {
  typedef typename mmp_t<T>::C C;
  const C x = (C)a;
  if (__builtin_isinf(x)) return (T)__builtin_copysignf(0.f, (float)x);
  return (T)__builtin_copysignf((float)(x - __builtin_truncf(x)), (float)x);
}
template <> MMP_DI float op_modf_frac(float a) {
  if (__builtin_isinf(a)) return __builtin_copysignf(0.f, a);
  const float t = __builtin_truncf(a);
  return __builtin_copysignf(a - t, a);
}
template <> MMP_DI double op_modf_frac(double a) {
  if (__builtin_isinf(a)) return __builtin_copysign(0.0, a);
  const double t = __builtin_trunc(a);
  return __builtin_copysign(a - t, a);
}
// np.ldexp(x, n); n arrives converted to T and is clamped far outside the
// exponent range (the result saturates anyway)
template <typename T> MMP_DI T op_ldexp(T a, T b) {
  typedef typename mmp_t<T>::C C;
  C n = (C)b;
  n = n > (C)100000 ? (C)100000 : (n < (C)-100000 ? (C)-100000 : n);
  if constexpr (sizeof(C) == 4) return (T)__builtin_ldexpf((float)a, (int)n);
  else return (T)__builtin_ldexp((double)a, (int)n);
}
// np.gcd / np.lcm on magnitudes (Euclid), results wrapped to T
template <typename T> MMP_DI T op_gcd(T a, T b) {
  typedef typename mmp_t<T>::U U;
  U x = (mmp_t<T>::is_signed && a < (T)0) ? (U)((U)0 - (U)a) : (U)a;
  U y = (mmp_t<T>::is_signed && b < (T)0) ? (U)((U)0 - (U)b) : (U)b;
  while (y) {
    const U t = (U)(x % y);
    x = y;
    y = t;
  }
  return (T)x;
}
template <typename T> MMP_DI T op_lcm(T a, T b) {
  typedef typename mmp_t<T>::U U;
  const U x = (mmp_t<T>::is_signed && a < (T)0) ? (U)((U)0 - (U)a) : (U)a;
  const U y = (mmp_t<T>::is_signed && b < (T)0) ? (U)((U)0 - (U)b) : (U)b;
  if (!x || !y) return (T)0;
  const U g = (U)op_gcd<T>((T)x, (T)y);
  return (T)(U)(x / g * y);
}

// =====================================================================
// Conversions (astype).  bool targets test != 0 (NaN -> true).
// =====================================================================
template <typename To, typename From> MMP_DI To mmp_convert(From v) {
  if constexpr (mmp_t<To>::is_bool) {
    if constexpr (mmp_t<From>::is_float) {
      return (typename mmp_t<From>::C)v != (typename mmp_t<From>::C)0;
    } else {
      return v != 0;
    }
  } else if constexpr (mmp_t<From>::is_bool) {
    return (To)(v ? 1 : 0);
  } else if constexpr (mmp_t<From>::is_float && !mmp_t<To>::is_float && !mmp_t<To>::is_signed) {
    // float -> unsigned: truncate to int64 first, then wrap, as NumPy's C
    // cast does on x86-64 (-1.0 -> 0xffff for uint16); values of 2^63 and
    // more only fit uint64 directly
    typedef typename mmp_t<From>::C F;
    const F f = (F)v;
    if constexpr (sizeof(To) == 8) {
      if (f >= (F)9223372036854775808.0) return (To)f;
    }
    return (To)(long long)f;
  } else if constexpr (sizeof(From) == 2 && mmp_t<From>::is_float) {
    return (To)(float)v;  // half -> widen first
  } else {
    return (To)v;
  }
}

// =====================================================================
// fast_math forms (set_config(fast_math=True); the reference switches its
// elementwise shader to Metal's fast:: functions, _kernels.py:26-27).  For
// float32 (and float16, computed in float32) they use the hardware
// transcendental instructions -- v_exp_f32 / v_log_f32 (base 2), v_sin_f32
// / v_cos_f32 (argument in revolutions), v_sqrt_f32, v_rcp_f32 -- instead of
// the correctly rounded or 2-ULP library functions.  Bound (the reference's
// unary-math tolerance, rtol = atol = 1e-5): exp [-80, 80], log / log2 /
// log10 [1e-30, 1e30], sin / cos [-100, 100], tan [-1.4, 1.4], sqrt,
// reciprocal, divide, tanh / sinh / cosh [-10, 10], power with a positive
// base in (0, 100] and exponent in [-4, 4].  Denormal inputs and results
// may flush to zero.  float64 and integer operands take the accurate ops.
// =====================================================================
MMP_DI float mm_fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
MMP_DI float mm_fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
MMP_DI float mm_fast_sin(float x) { return __builtin_amdgcn_sinf(x * 0.159154943091895336f); }
MMP_DI float mm_fast_cos(float x) { return __builtin_amdgcn_cosf(x * 0.159154943091895336f); }
MMP_DI float mm_fast_tanh(float x) {
  // tanh|x| = 1 - 2 / (e^{2|x|} + 1); e = inf gives 1
  const float e = __builtin_amdgcn_exp2f(__builtin_fabsf(x) * 2.88539008177792682f);
  const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
  return __builtin_copysignf(t, x);
}

#define MMP_FAST_UNARY(NAME, FEXPR)                                           \
  template <typename T> MMP_DI T op_##NAME##_fast(T x_) {                     \
    if constexpr (__is_same(typename mmp_t<T>::C, float)) {                   \
      const float x = (float)x_;                                              \
      return (T)(FEXPR);                                                      \
    } else {                                                                  \
      return op_##NAME(x_);                                                   \
    }                                                                         \
  }
MMP_FAST_UNARY(exp, mm_fast_exp(x))
MMP_FAST_UNARY(exp2, __builtin_amdgcn_exp2f(x))
MMP_FAST_UNARY(log, __builtin_amdgcn_logf(x) * 0.693147180559945309f)
MMP_FAST_UNARY(log2, __builtin_amdgcn_logf(x))
MMP_FAST_UNARY(log10, __builtin_amdgcn_logf(x) * 0.301029995663981195f)
MMP_FAST_UNARY(sin, mm_fast_sin(x))
MMP_FAST_UNARY(cos, mm_fast_cos(x))
MMP_FAST_UNARY(tan, mm_fast_sin(x) * mm_fast_rcp(mm_fast_cos(x)))
MMP_FAST_UNARY(sqrt, __builtin_amdgcn_sqrtf(x))
MMP_FAST_UNARY(reciprocal, mm_fast_rcp(x))
MMP_FAST_UNARY(tanh, mm_fast_tanh(x))
MMP_FAST_UNARY(sinh, 0.5f * (mm_fast_exp(x) - mm_fast_rcp(mm_fast_exp(x))))
MMP_FAST_UNARY(cosh, 0.5f * (mm_fast_exp(x) + mm_fast_rcp(mm_fast_exp(x))))

template <typename T> MMP_DI T op_true_divide_fast(T a, T b) {
  if constexpr (__is_same(typename mmp_t<T>::C, float)) {
    return (T)((float)a * mm_fast_rcp((float)b));
  } else {
    return op_true_divide(a, b);
  }
}
template <typename T> MMP_DI T op_power_fast(T a, T b) {
  if constexpr (__is_same(typename mmp_t<T>::C, float)) {
    const float x = (float)a, y = (float)b;
    // positive finite base: 2^(y log2 x); anything else takes the exact pow
    if (x > 0.0f && x < __builtin_inff())
      return (T)__builtin_amdgcn_exp2f(y * __builtin_amdgcn_logf(x));
    return op_power(a, b);
  } else {
    return op_power(a, b);
  }
}
