"""Every float32 bit pattern through this build's own float32 functions.

`mm_tanh`, `mm_log1p` and `mm_exp` (csrc/mmp_ops.h) are written here rather than
taken from the device math library, so their accuracy is checked over all
2^32 inputs: a kernel evaluates each one next to the library's float64
function of the same input and records the error in units in the last
place (ULP) of the float32 result.  The worst input the device reports is
then recomputed on the host (NumPy float64) to check the device-side error
arithmetic.  The reference maps these ops to numpy.tanh / numpy.log1p
(src/macmetalpy/ndarray.py:74-102).
"""
import ctypes

import numpy as np
import pytest

import macmetalpy_amd as cp
from macmetalpy_amd import _fusion
from macmetalpy_amd._backend import HipBackend

pytestmark = pytest.mark.gpu

PER_THREAD = 4096
THREADS = (1 << 32) // PER_THREAD          # 2^20 threads, 4096 workgroups of 256

_KERNEL = r"""
__device__ __forceinline__ double ulp_err(float c, double r) {
  if (r != r) return c != c ? 0.0 : 1e30;
  if (c != c) return 1e30;
  const float rf = (float)r;
  if (__builtin_isinf(r) || __builtin_isinf(rf)) return c == rf ? 0.0 : 1e30;
  if (__builtin_isinf(c)) return 1e30;
  int q;
  frexp(r, &q);                       // |r| in [2^(q-1), 2^q)
  const int e = q - 24 < -149 ? -149 : q - 24;
  return fabs((double)c - r) / ldexp(1.0, e);
}
template <int F> __device__ __forceinline__ void eval(float x, float& c, double& r) {
  if (F == 0) { c = mm_tanh(x); r = tanh((double)x); }
  if (F == 1) { c = mm_log1p(x); r = log1p((double)x); }
  if (F == 2) { c = mm_exp(x); r = exp((double)x); }
}
// The sign-specialised forms equal the general ones bit for bit on the
// inputs they are used for (exp: x <= 0 or NaN; log1p: x >= 0 or NaN; two
// NaNs count as equal whatever their payloads): a mismatch counts as an
// error of 1e30 ULP.
__device__ __forceinline__ double same_bits(float a, float b) {
  if (a != a && b != b) return 0.0;
  return __builtin_bit_cast(unsigned, a) == __builtin_bit_cast(unsigned, b) ? 0.0 : 1e30;
}
template <int F> __device__ void sweep(unsigned* out) {
  const unsigned long long t = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x;
  float worst = -1.0f;
  unsigned wbits = 0, n1 = 0, n2 = 0;
  for (unsigned j = 0; j < PER; ++j) {
    const unsigned bits = (unsigned)(t * PER + j);
    const float x = __builtin_bit_cast(float, bits);
    double e;
    if (F == 3) {
      e = (x <= 0.0f || x != x) ? same_bits(mm_exp_nonpos(x), mm_exp(x)) : 0.0;
      e += (x >= 0.0f || x != x) ? same_bits(mm_log1p_nonneg(x), mm_log1p(x)) : 0.0;
    } else {
      float c; double r;
      eval<F>(x, c, r);
      e = ulp_err(c, r);
    }
    const float ef = e > 1e9 ? 1e9f : (float)e;
    if (ef > worst) { worst = ef; wbits = bits; }
    n1 += e > 1.0;
    n2 += e > 2.0;
  }
  out[4 * t + 0] = __builtin_bit_cast(unsigned, worst);
  out[4 * t + 1] = wbits;
  out[4 * t + 2] = n1;
  out[4 * t + 3] = n2;
}
extern "C" __global__ __launch_bounds__(256) void sweep_tanh(unsigned* out) { sweep<0>(out); }
extern "C" __global__ __launch_bounds__(256) void sweep_log1p(unsigned* out) { sweep<1>(out); }
extern "C" __global__ __launch_bounds__(256) void sweep_exp(unsigned* out) { sweep<2>(out); }
extern "C" __global__ __launch_bounds__(256) void sweep_sign_forms(unsigned* out) { sweep<3>(out); }
"""


def _sweep(name):
    be = HipBackend()
    src = _fusion._ops_header() + f"\n#define PER {PER_THREAD}u\n" + _KERNEL
    k = be.compile(src, name, _fusion.RTC_OPTIONS)
    out = cp.empty(4 * THREADS, dtype=np.uint32)
    out._ensure_gpu()
    assert out.size * 4 == THREADS * 16          # one 16-byte record per thread
    be.launch(k, (THREADS // 256, 1, 1), (256, 1, 1), [ctypes.c_void_p(out._ptr)])
    rec = out.get().reshape(THREADS, 4)
    err = rec[:, 0].view(np.float32)
    i = int(np.argmax(err))
    return float(err[i]), int(rec[i, 1]), int(rec[:, 2].sum()), int(rec[:, 3].sum())


def _host_ulp(got, want):
    """Error of float32 ``got`` against float64 ``want`` in float32 ULPs."""
    _, q = np.frexp(want)
    return abs(float(got) - want) / np.ldexp(1.0, max(int(q) - 24, -149))


@pytest.mark.parametrize("name,op,fn,bound", [
    ("sweep_tanh", cp.tanh, np.tanh, 1.6),
    ("sweep_log1p", cp.log1p, np.log1p, 1.3),
    ("sweep_exp", cp.exp, np.exp, 1.1),
])
def test_every_float32_input(name, op, fn, bound):
    worst, wbits, n_gt1, n_gt2 = _sweep(name)
    print(f"{name}: max {worst:.4f} ULP at bits {wbits:#010x}; >1 ULP: {n_gt1}; >2 ULP: {n_gt2}")
    assert worst <= bound and n_gt2 == 0
    # the worst input, recomputed on the host: same error to 1e-3 ULP
    x = np.array([wbits], np.uint32).view(np.float32)
    got = op(cp.array(x)).get()[0]
    want = float(fn(x.astype(np.float64))[0])
    assert abs(_host_ulp(got, want) - worst) < 1e-3


def test_sign_specialised_forms_match_bit_for_bit():
    """exp without its overflow case and log1p without its x <= -1 cases
    (what the code generator calls for exp(-|x|), log1p(x*x), ...) give the
    general functions' bits on every input they are used for (NaN for NaN,
    payloads aside)."""
    worst, wbits, n_gt1, _ = _sweep("sweep_sign_forms")
    assert worst == 0.0 and n_gt1 == 0, f"first mismatch at bits {wbits:#010x}"


def test_tanh_and_log1p_special_values():
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 16.0, 1e30, -1e30,
                  1e-45, -1e-45, 1e-30], np.float32)
    got = cp.tanh(cp.array(x)).get()
    want = np.tanh(x)
    ok = ~np.isnan(want)
    assert np.array_equal(np.signbit(got[ok]), np.signbit(want[ok]))
    np.testing.assert_array_equal(got, want)
    y = np.array([0.0, -0.0, np.inf, -1.0, -2.0, -np.inf, np.nan, 1e-45, -1e-45, 1e-30],
                 np.float32)
    got = cp.log1p(cp.array(y)).get()
    with np.errstate(invalid="ignore", divide="ignore"):
        want = np.log1p(y)
    ok = ~np.isnan(want)
    assert np.array_equal(np.signbit(got[ok]), np.signbit(want[ok]))
    np.testing.assert_array_equal(got, want)
