/*
 * oracle.c -- TEST ORACLE ONLY.  Independent C restatement of the integer
 * semantics the reference's CPU/NumPy path produces for the hot path
 * (grantkl/MacMetalPy: ufunc_ops.floor_divide -> np.floor_divide,
 * math_ops.mod -> np.mod (math_ops.py:540-548), reductions.cumsum ->
 * np.cumsum with int64 output (reductions.py:669-675), reductions.argmax ->
 * np.argmax (reductions.py:388-398)).
 *
 * Written from the definitions, in 64-bit arithmetic, and NOT from the
 * device code: floor(a / b) for b != 0, remainder a - b*floor(a/b) (sign of
 * b), 0 for b == 0 (NumPy's integer result for division by zero), results
 * wrapped to int32.  Used by tests to pin the NumPy restatement.
 */
#include <math.h>
#include <stdint.h>

static int64_t floor_div64(int64_t a, int64_t b) {
  int64_t q = a / b;           /* truncates toward zero (C99)   */
  int64_t r = a - q * b;
  if (r != 0 && ((r < 0) != (b < 0))) q -= 1;
  return q;
}

void oracle_floor_divide_i32(const int32_t *a, const int32_t *b, int32_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    if (b[i] == 0) { out[i] = 0; continue; }
    int64_t q = floor_div64((int64_t)a[i], (int64_t)b[i]);
    out[i] = (int32_t)(uint32_t)(uint64_t)q;    /* wrap: INT_MIN // -1 */
  }
}

void oracle_mod_i32(const int32_t *a, const int32_t *b, int32_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    if (b[i] == 0) { out[i] = 0; continue; }
    int64_t A = a[i], B = b[i];
    out[i] = (int32_t)(A - B * floor_div64(A, B));
  }
}

void oracle_cumsum_i32(const int32_t *x, int64_t *out, int64_t n) {
  int64_t acc = 0;
  for (int64_t i = 0; i < n; ++i) { acc += x[i]; out[i] = acc; }
}

double oracle_sum_f32(const float *x, int64_t n) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) acc += (double)x[i];
  return acc;
}

/* first index of the maximum; a NaN is the maximum (first NaN wins) */
int64_t oracle_argmax_f32(const float *x, int64_t n) {
  int64_t best = 0;
  for (int64_t i = 0; i < n; ++i) {
    if (isnan(x[i])) return i;
    if (x[i] > x[best]) best = i;
  }
  return best;
}
