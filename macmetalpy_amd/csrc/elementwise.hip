// elementwise.hip -- precompiled unary / binary / cast / fill kernels.
//
// Replaces the reference's per-dtype Metal "elementwise" library
// (src/macmetalpy/_kernels.py:21-404) and the plumbing shaders of
// _kernel_cache.py:44-189.  The reference launches one thread per element
// with no bounds check; here every kernel streams 64 bytes per thread per
// operand with 128-bit loads, one tile of 256 threads x 4 x 16 B per block
// (2^28 float32 elements -> 65,536 blocks, far more than the 256 CUs need),
// and handles the ragged tail with scalar accesses.  HBM-bound: the
// algorithmic traffic per element is sizeof(T) per operand read plus
// sizeof(T) written.
#include "mmp_ops.h"
#include "mmp_internal.h"

namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 4;  // 16-byte vectors per thread per operand

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T> union Pack {
  u32x4 v;
  T e[16 / sizeof(T)];
};

// Streaming loads/stores bypass cache retention: each byte is touched once.
template <typename V> __device__ __forceinline__ V ld_stream(const V *p) {
  return __builtin_nontemporal_load(p);
}
template <typename V> __device__ __forceinline__ void st_stream(V v, V *p) {
  __builtin_nontemporal_store(v, p);
}

inline bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// ------------------------------------------------------------ op tables
template <int OP, typename T> __device__ __forceinline__ T apply_unary(T x) {
  if constexpr (OP == MMP_U_NEG) return op_neg(x);
  else if constexpr (OP == MMP_U_POSITIVE) return op_positive(x);
  else if constexpr (OP == MMP_U_ABS) return op_abs(x);
  else if constexpr (OP == MMP_U_SIGN) return op_sign(x);
  else if constexpr (OP == MMP_U_SQUARE) return op_square(x);
  else if constexpr (OP == MMP_U_RECIPROCAL) return op_reciprocal(x);
  else if constexpr (OP == MMP_U_SQRT) return op_sqrt(x);
  else if constexpr (OP == MMP_U_CBRT) return op_cbrt(x);
  else if constexpr (OP == MMP_U_EXP) return op_exp(x);
  else if constexpr (OP == MMP_U_EXP2) return op_exp2(x);
  else if constexpr (OP == MMP_U_EXPM1) return op_expm1(x);
  else if constexpr (OP == MMP_U_LOG) return op_log(x);
  else if constexpr (OP == MMP_U_LOG2) return op_log2(x);
  else if constexpr (OP == MMP_U_LOG10) return op_log10(x);
  else if constexpr (OP == MMP_U_LOG1P) return op_log1p(x);
  else if constexpr (OP == MMP_U_SIN) return op_sin(x);
  else if constexpr (OP == MMP_U_COS) return op_cos(x);
  else if constexpr (OP == MMP_U_TAN) return op_tan(x);
  else if constexpr (OP == MMP_U_ASIN) return op_arcsin(x);
  else if constexpr (OP == MMP_U_ACOS) return op_arccos(x);
  else if constexpr (OP == MMP_U_ATAN) return op_arctan(x);
  else if constexpr (OP == MMP_U_SINH) return op_sinh(x);
  else if constexpr (OP == MMP_U_COSH) return op_cosh(x);
  else if constexpr (OP == MMP_U_TANH) return op_tanh(x);
  else if constexpr (OP == MMP_U_ASINH) return op_arcsinh(x);
  else if constexpr (OP == MMP_U_ACOSH) return op_arccosh(x);
  else if constexpr (OP == MMP_U_ATANH) return op_arctanh(x);
  else if constexpr (OP == MMP_U_FLOOR) return op_floor(x);
  else if constexpr (OP == MMP_U_CEIL) return op_ceil(x);
  else if constexpr (OP == MMP_U_RINT) return op_rint(x);
  else if constexpr (OP == MMP_U_TRUNC) return op_trunc(x);
  else if constexpr (OP == MMP_U_DEGREES) return op_degrees(x);
  else return op_radians(x);
}

template <int OP, typename T> struct UnaryOk {
  static constexpr bool value =
      mmp_t<T>::is_float ||
      (!mmp_t<T>::is_bool &&
       (OP == MMP_U_NEG || OP == MMP_U_POSITIVE || OP == MMP_U_ABS ||
        OP == MMP_U_SIGN || OP == MMP_U_SQUARE || OP == MMP_U_RECIPROCAL ||
        OP == MMP_U_FLOOR || OP == MMP_U_CEIL || OP == MMP_U_RINT ||
        OP == MMP_U_TRUNC));
};

template <int OP, typename T> __device__ __forceinline__ T apply_binary(T a, T b) {
  if constexpr (OP == MMP_B_ADD) return op_add(a, b);
  else if constexpr (OP == MMP_B_SUB) return op_subtract(a, b);
  else if constexpr (OP == MMP_B_MUL) return op_multiply(a, b);
  else if constexpr (OP == MMP_B_DIV) return op_true_divide(a, b);
  else if constexpr (OP == MMP_B_FLOOR_DIVIDE) return op_floor_divide(a, b);
  else if constexpr (OP == MMP_B_MOD) return op_remainder(a, b);
  else if constexpr (OP == MMP_B_POWER) return op_power(a, b);
  else if constexpr (OP == MMP_B_MAXIMUM) return op_maximum(a, b);
  else if constexpr (OP == MMP_B_MINIMUM) return op_minimum(a, b);
  else if constexpr (OP == MMP_B_FMAX) return op_fmax(a, b);
  else if constexpr (OP == MMP_B_FMIN) return op_fmin(a, b);
  else if constexpr (OP == MMP_B_ATAN2) return op_arctan2(a, b);
  else if constexpr (OP == MMP_B_HYPOT) return op_hypot(a, b);
  else if constexpr (OP == MMP_B_FMOD) return op_fmod(a, b);
  else if constexpr (OP == MMP_B_COPYSIGN) return op_copysign(a, b);
  else if constexpr (OP == MMP_B_NEXTAFTER) return op_nextafter(a, b);
  else if constexpr (OP == MMP_B_LOGADDEXP) return op_logaddexp(a, b);
  else if constexpr (OP == MMP_B_LOGADDEXP2) return op_logaddexp2(a, b);
  else return op_heaviside(a, b);
}

template <int OP, typename T> struct BinaryOk {
  static constexpr bool value =
      mmp_t<T>::is_float ||
      (mmp_t<T>::is_bool &&
       (OP == MMP_B_ADD || OP == MMP_B_MUL || OP == MMP_B_MAXIMUM ||
        OP == MMP_B_MINIMUM || OP == MMP_B_FMAX || OP == MMP_B_FMIN)) ||
      (!mmp_t<T>::is_bool &&
       (OP == MMP_B_ADD || OP == MMP_B_SUB || OP == MMP_B_MUL ||
        OP == MMP_B_FLOOR_DIVIDE || OP == MMP_B_MOD || OP == MMP_B_POWER ||
        OP == MMP_B_MAXIMUM || OP == MMP_B_MINIMUM || OP == MMP_B_FMAX ||
        OP == MMP_B_FMIN || OP == MMP_B_FMOD));
};

// -------------------------------------------------------------- kernels
// One tile per block; full tiles use 128-bit streaming accesses when every
// pointer is 16-byte aligned (vec != 0), the tail and unaligned views use
// scalar accesses.
template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void k_unary(const T *__restrict__ x,
                                                  T *__restrict__ y,
                                                  long long n, int vec) {
  constexpr int V = 16 / sizeof(T);
  constexpr long long TILE = (long long)kBlock * kUnroll * V;
  const long long base = (long long)blockIdx.x * TILE;
  if (vec && base + TILE <= n) {
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(x + base);
    u32x4 *yv = reinterpret_cast<u32x4 *>(y + base);
    Pack<T> p[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) p[u].v = ld_stream(xv + u * kBlock + threadIdx.x);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int j = 0; j < V; ++j) p[u].e[j] = apply_unary<OP, T>(p[u].e[j]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) st_stream(p[u].v, yv + u * kBlock + threadIdx.x);
  } else {
    const long long end = base + TILE < n ? base + TILE : n;
    for (long long i = base + threadIdx.x; i < end; i += kBlock)
      y[i] = apply_unary<OP, T>(x[i]);
  }
}

// SCAL: 0 = both operands are arrays, 1 = a is the scalar s, 2 = b is s.
template <int OP, typename T, int SCAL>
__global__ __launch_bounds__(kBlock) void k_binary(const T *__restrict__ a,
                                                   const T *__restrict__ b,
                                                   T s, T *__restrict__ y,
                                                   long long n, int vec) {
  constexpr int V = 16 / sizeof(T);
  constexpr long long TILE = (long long)kBlock * kUnroll * V;
  const long long base = (long long)blockIdx.x * TILE;
  if (vec && base + TILE <= n) {
    const u32x4 *av = reinterpret_cast<const u32x4 *>(a + base);
    const u32x4 *bv = reinterpret_cast<const u32x4 *>(b + base);
    u32x4 *yv = reinterpret_cast<u32x4 *>(y + base);
    Pack<T> pa[kUnroll], pb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if constexpr (SCAL != 1) pa[u].v = ld_stream(av + u * kBlock + threadIdx.x);
      if constexpr (SCAL != 2) pb[u].v = ld_stream(bv + u * kBlock + threadIdx.x);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int j = 0; j < V; ++j) {
        T va, vb;
        if constexpr (SCAL == 1) va = s; else va = pa[u].e[j];
        if constexpr (SCAL == 2) vb = s; else vb = pb[u].e[j];
        if constexpr (SCAL == 1) pb[u].e[j] = apply_binary<OP, T>(va, vb);
        else pa[u].e[j] = apply_binary<OP, T>(va, vb);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if constexpr (SCAL == 1) st_stream(pb[u].v, yv + u * kBlock + threadIdx.x);
      else st_stream(pa[u].v, yv + u * kBlock + threadIdx.x);
    }
  } else {
    const long long end = base + TILE < n ? base + TILE : n;
    for (long long i = base + threadIdx.x; i < end; i += kBlock) {
      T va, vb;
      if constexpr (SCAL == 1) va = s; else va = a[i];
      if constexpr (SCAL == 2) vb = s; else vb = b[i];
      y[i] = apply_binary<OP, T>(va, vb);
    }
  }
}

// Strided copy with conversion.  mode 0: both contiguous; 1: strided
// source -> contiguous destination; 2: strided source and destination.
struct StrideDesc {
  int ndim;
  long long shape[8];
  long long sstride[8];
  long long dstride[8];
};

template <typename Ti, typename To>
__global__ __launch_bounds__(kBlock) void k_copy(const Ti *__restrict__ x,
                                                 To *__restrict__ y,
                                                 long long n, StrideDesc d,
                                                 int mode) {
  const long long stride = (long long)gridDim.x * kBlock;
  for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += stride) {
    if (mode == 0) {
      y[i] = mmp_convert<To, Ti>(x[i]);
      continue;
    }
    long long rem = i, so = 0, dof = 0;
    for (int k = d.ndim - 1; k >= 0; --k) {
      const long long s = d.shape[k];
      const long long q = rem / s;
      const long long idx = rem - q * s;
      so += idx * d.sstride[k];
      dof += idx * d.dstride[k];
      rem = q;
    }
    if (mode == 1) dof = i;
    y[dof] = mmp_convert<To, Ti>(x[so]);
  }
}

// Strided copy by rows: each workgroup takes one row (all dimensions but
// the last) and a tile of kRowTile (4096) columns, resolves the row's source and
// destination offsets once, then copies along the row -- coalesced when
// the last dimension's strides are 0 or 1 (broadcasts, tiles, slices).
// The generic kernel above pays a 64-bit division per dimension for every
// element.
#ifndef MMP_ROW_ITEMS
#define MMP_ROW_ITEMS 16
#endif
constexpr int kRowItems = MMP_ROW_ITEMS;
constexpr int kRowTile = kBlock * kRowItems;

template <typename Ti, typename To>
__global__ __launch_bounds__(kBlock) void k_copy_rows(const Ti *__restrict__ x,
                                                      To *__restrict__ y, StrideDesc d,
                                                      long long ctiles) {
  const int last = d.ndim - 1;
  const long long len = d.shape[last];
  const long long b = blockIdx.x;
  const long long row = b / ctiles;
  const long long c0 = (b - row * ctiles) * kRowTile;
  long long rem = row, so = 0, dof = 0;
  for (int k = last - 1; k >= 0; --k) {
    const long long s = d.shape[k];
    const long long q = rem / s;
    const long long idx = rem - q * s;
    so += idx * d.sstride[k];
    dof += idx * d.dstride[k];
    rem = q;
  }
  const long long ss = d.sstride[last], ds = d.dstride[last];
  if (ss == 1 && ds == 1) {
    // rows contiguous on both sides (slices, tiles, concatenations): row
    // pointers once, 32-bit offsets within the tile, all loads first
    const Ti *xs = x + so + c0;
    To *yd = y + dof + c0;
    const int n = len - c0 < kRowTile ? (int)(len - c0) : kRowTile;
    if (n == kRowTile) {
      Ti v[kRowItems];
#pragma unroll
      for (int u = 0; u < kRowItems; ++u) v[u] = xs[u * kBlock + threadIdx.x];
#pragma unroll
      for (int u = 0; u < kRowItems; ++u) yd[u * kBlock + threadIdx.x] = mmp_convert<To, Ti>(v[u]);
    } else {
      for (int c = threadIdx.x; c < n; c += kBlock) yd[c] = mmp_convert<To, Ti>(xs[c]);
    }
    return;
  }
  // Other strides: all loads first as well (a column past the row's end
  // reads column c0, which exists); a guarded load-convert-store per
  // element had each load waited for before the next was issued.
  Ti v[kRowItems];
#pragma unroll
  for (int u = 0; u < kRowItems; ++u) {
    const long long c = c0 + u * kBlock + threadIdx.x;
    v[u] = x[so + (c < len ? c : c0) * ss];
  }
#pragma unroll
  for (int u = 0; u < kRowItems; ++u) {
    const long long c = c0 + u * kBlock + threadIdx.x;
    if (c < len) y[dof + c * ds] = mmp_convert<To, Ti>(v[u]);
  }
}

// Contiguous cast / copy with vector accesses: per step a thread converts
// E = 16 / sizeof(To) consecutive elements and writes them with one 16-byte
// store, so the lanes of a store instruction cover one contiguous span;
// the matching input (E * sizeof(Ti) bytes: 2 .. 64) is read with the
// widest loads that fit.  4 steps per thread per tile; the last partial
// tile element by element.
template <int B> struct VecBytes;
template <> struct VecBytes<2> { typedef unsigned short type; };
template <> struct VecBytes<4> { typedef unsigned int type; };
template <> struct VecBytes<8> { typedef unsigned int type __attribute__((ext_vector_type(2))); };
template <> struct VecBytes<16> { typedef unsigned int type __attribute__((ext_vector_type(4))); };

template <typename Ti, typename To>
__global__ __launch_bounds__(kBlock) void k_copy_vec(const Ti *__restrict__ x, To *__restrict__ y,
                                                     long long n) {
  constexpr int E = 16 / (int)sizeof(To);        // elements per thread per step
  constexpr int IB = E * (int)sizeof(Ti);        // input bytes per thread per step
  constexpr int LB = IB < 16 ? IB : 16;          // bytes per load
  constexpr int NL = IB / LB;                    // loads per step
  typedef typename VecBytes<LB>::type LV;
  typedef typename VecBytes<16>::type SV;
  constexpr int U = 4;
  constexpr long long TILE = (long long)kBlock * E * U;
  const long long t0 = (long long)blockIdx.x * TILE;
  if (t0 + TILE <= n) {
    union In {
      LV v[NL];
      Ti e[E];
    } in[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const LV *src = reinterpret_cast<const LV *>(x + t0 + ((long long)u * kBlock + threadIdx.x) * E);
#pragma unroll
      for (int c = 0; c < NL; ++c) in[u].v[c] = __builtin_nontemporal_load(src + c);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      union Out {
        SV v;
        To e[E];
      } o;
#pragma unroll
      for (int k = 0; k < E; ++k) o.e[k] = mmp_convert<To, Ti>(in[u].e[k]);
      __builtin_nontemporal_store(o.v, reinterpret_cast<SV *>(y + t0 + ((long long)u * kBlock + threadIdx.x) * E));
    }
    return;
  }
  for (long long i = t0 + threadIdx.x; i < n && i < t0 + TILE; i += kBlock)
    y[i] = mmp_convert<To, Ti>(x[i]);
}

// Permuted copies (a transpose on two axes p, q, batched over the others):
// the destination is contiguous along q, the source along p.  A 64 x 64
// tile goes through LDS (row pitch 65 words, no bank conflicts): read with
// consecutive threads along p, written with consecutive threads along q, so
// both sides are coalesced.  The generic kernel reads one of the two with
// a 64-element stride.
struct TransDesc {
  long long np, nq;                // extents of p and q
  long long sp, sq, dp, dq;        // source / destination strides of p and q
  int nb;                          // batch dimensions
  long long bshape[8], bs[8], bd[8];
  long long tp, tq;                // tiles along p and q
};

template <typename Ti, typename To>
__global__ __launch_bounds__(kBlock) void k_copy_transpose(const Ti *__restrict__ x,
                                                           To *__restrict__ y, TransDesc t) {
  __shared__ Ti tile[64][65];
  long long b = blockIdx.x;
  const long long jq = b % t.tq;
  b /= t.tq;
  const long long jp = b % t.tp;
  b /= t.tp;
  long long so = 0, dof = 0;
  for (int k = t.nb - 1; k >= 0; --k) {
    const long long q = b / t.bshape[k];
    const long long i = b - q * t.bshape[k];
    so += i * t.bs[k];
    dof += i * t.bd[k];
    b = q;
  }
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const long long p0 = jp * 64, q0 = jq * 64;
  // All 16 loads first (an element outside the array reads the tile's
  // corner (p0, q0), which exists), then the guarded LDS writes: a guarded
  // load per element had each load waited for before the next was issued.
  Ti v[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = ty + 4 * i;  // q within the tile
    const long long pp = p0 + tx, qq = q0 + r;
    const bool in = pp < t.np && qq < t.nq;
    v[i] = x[so + (in ? pp : p0) * t.sp + (in ? qq : q0) * t.sq];
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = ty + 4 * i;
    if (p0 + tx < t.np && q0 + r < t.nq) tile[r][tx] = v[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = ty + 4 * i;  // p within the tile
    const long long pp = p0 + r, qq = q0 + tx;
    if (pp < t.np && qq < t.nq) y[dof + pp * t.dp + qq * t.dq] = mmp_convert<To, Ti>(tile[tx][r]);
  }
}

// The same permuted copy for whole 64 x 64 tiles of 2-, 4- or 8-byte
// elements (no conversion) whose rows start 16-byte aligned on both sides:
// every global access is one 16-byte vector (VEC elements) -- a lane reads
// VEC consecutive p of one q row and writes VEC consecutive q of one p row
// -- and per-thread addresses are formed once, then advanced by constant
// steps.  LDS pitch 65 elements: the transposed reads of a wave hit 64
// distinct banks.
template <typename T>
__global__ __launch_bounds__(kBlock) void k_copy_transpose_vec(const T *__restrict__ x,
                                                              T *__restrict__ y, TransDesc t) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int VPR = 64 / VEC;          // vectors per 64-element tile row
  constexpr int RPP = kBlock / VPR;      // tile rows per pass
  __shared__ T tile[64][65];
  long long b = blockIdx.x;
  const long long jq = b % t.tq;
  b /= t.tq;
  const long long jp = b % t.tp;
  b /= t.tp;
  long long so = 0, dof = 0;
  for (int k = t.nb - 1; k >= 0; --k) {
    const long long q = b / t.bshape[k];
    const long long i = b - q * t.bshape[k];
    so += i * t.bs[k];
    dof += i * t.bd[k];
    b = q;
  }
  const int v = threadIdx.x % VPR, r0 = threadIdx.x / VPR;
  const long long p0 = jp * 64, q0 = jq * 64;
  const T *src = x + so + p0 + v * VEC + (q0 + r0) * t.sq;
#pragma unroll
  for (int i = 0; i < 64 / RPP; ++i) {
    union { u32x4 u; T e[VEC]; } w;
    w.u = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src + (long long)i * RPP * t.sq));
#pragma unroll
    for (int e = 0; e < VEC; ++e) tile[r0 + i * RPP][v * VEC + e] = w.e[e];
  }
  __syncthreads();
  T *dst = y + dof + (p0 + r0) * t.dp + q0 + v * VEC;
#pragma unroll
  for (int i = 0; i < 64 / RPP; ++i) {
    union { u32x4 u; T e[VEC]; } w;
#pragma unroll
    for (int e = 0; e < VEC; ++e) w.e[e] = tile[v * VEC + e][r0 + i * RPP];
    __builtin_nontemporal_store(w.u, reinterpret_cast<u32x4 *>(dst + (long long)i * RPP * t.dp));
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_fill(T *__restrict__ y, long long n, T v) {
  const long long stride = (long long)gridDim.x * kBlock;
  for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
    y[i] = v;
}

// ------------------------------------------------------------ launchers
template <typename T> constexpr long long tile_elems() {
  return (long long)kBlock * kUnroll * (16 / sizeof(T));
}

template <int OP, typename T>
int launch_unary(long long n, const void *x, void *out) {
  if constexpr (!UnaryOk<OP, T>::value) {
    return mmpi::fail(MMP_E_UNSUPPORTED, "unary op %d not defined for this dtype", OP);
  } else {
    const long long grid = mmpi::ceil_div(n, tile_elems<T>());
    const int vec = aligned16(x) && aligned16(out);
    hipLaunchKernelGGL((k_unary<OP, T>), dim3((unsigned)grid), dim3(kBlock), 0,
                       mmpi::stream(), (const T *)x, (T *)out, n, vec);
    return mmpi::check_launch("mmp_unary");
  }
}

template <int OP, typename T>
int launch_binary(long long n, const void *a, const void *b, const void *scalar,
                  int mode, void *out) {
  if constexpr (!BinaryOk<OP, T>::value) {
    return mmpi::fail(MMP_E_UNSUPPORTED, "binary op %d not defined for this dtype", OP);
  } else {
    const long long grid = mmpi::ceil_div(n, tile_elems<T>());
    T s{};
    if (scalar) s = *reinterpret_cast<const T *>(scalar);
    const int vec = aligned16(a) && aligned16(b) && aligned16(out);
    if (mode == 0)
      hipLaunchKernelGGL((k_binary<OP, T, 0>), dim3((unsigned)grid), dim3(kBlock), 0,
                         mmpi::stream(), (const T *)a, (const T *)b, s, (T *)out, n, vec);
    else if (mode == 1)
      hipLaunchKernelGGL((k_binary<OP, T, 1>), dim3((unsigned)grid), dim3(kBlock), 0,
                         mmpi::stream(), (const T *)b, (const T *)b, s, (T *)out, n, vec);
    else
      hipLaunchKernelGGL((k_binary<OP, T, 2>), dim3((unsigned)grid), dim3(kBlock), 0,
                         mmpi::stream(), (const T *)a, (const T *)a, s, (T *)out, n, vec);
    return mmpi::check_launch("mmp_binary");
  }
}

#define MMP_UNARY_CODES(X)                                                    \
  X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13)   \
  X(14) X(15) X(16) X(17) X(18) X(19) X(20) X(21) X(22) X(23) X(24) X(25)     \
  X(26) X(27) X(28) X(29) X(30) X(31) X(32)
#define MMP_BINARY_CODES(X)                                                   \
  X(0) X(1) X(2) X(3) X(4) X(5) X(6) X(7) X(8) X(9) X(10) X(11) X(12) X(13)   \
  X(14) X(15) X(16) X(17) X(18)

template <typename T> int unary_for_type(int op, long long n, const void *x, void *out) {
  switch (op) {
#define MMP_CASE(k) case k: return launch_unary<k, T>(n, x, out);
    MMP_UNARY_CODES(MMP_CASE)
#undef MMP_CASE
    default:
      return mmpi::fail(MMP_E_ARG, "unknown unary op code %d", op);
  }
}

template <typename T>
int binary_for_type(int op, long long n, const void *a, const void *b,
                    const void *s, int mode, void *out) {
  switch (op) {
#define MMP_CASE(k) case k: return launch_binary<k, T>(n, a, b, s, mode, out);
    MMP_BINARY_CODES(MMP_CASE)
#undef MMP_CASE
    default:
      return mmpi::fail(MMP_E_ARG, "unknown binary op code %d", op);
  }
}

// A transpose layout: the destination's innermost dimension q (stride 1)
// is strided in the source and another dimension p is contiguous there;
// both extents at least 16.
bool transpose_desc(const StrideDesc &d, TransDesc *t) {
  if (d.ndim < 2) return false;
  const int q = d.ndim - 1;
  if (d.dstride[q] != 1 || d.sstride[q] == 1 || d.shape[q] < 16) return false;
  int p = -1;
  for (int k = 0; k < q; ++k)
    if (d.sstride[k] == 1) p = k;
  if (p < 0 || d.shape[p] < 16) return false;
  t->np = d.shape[p];
  t->nq = d.shape[q];
  t->sp = d.sstride[p];
  t->sq = d.sstride[q];
  t->dp = d.dstride[p];
  t->dq = d.dstride[q];
  t->nb = 0;
  for (int k = 0; k < q; ++k) {
    if (k == p) continue;
    t->bshape[t->nb] = d.shape[k];
    t->bs[t->nb] = d.sstride[k];
    t->bd[t->nb] = d.dstride[k];
    ++t->nb;
  }
  t->tp = mmpi::ceil_div(t->np, 64);
  t->tq = mmpi::ceil_div(t->nq, 64);
  return true;
}

// Whole tiles and 16-byte aligned rows on both sides for the vector
// transpose: extents multiples of 64, every stride other than the two unit
// ones a multiple of the vector, aligned bases.
bool transpose_vec_ok(const TransDesc &t, const void *x, const void *y, int vec) {
  if (t.np % 64 || t.nq % 64 || t.sq % vec || t.dp % vec) return false;
  for (int k = 0; k < t.nb; ++k)
    if (t.bs[k] % vec || t.bd[k] % vec) return false;
  return aligned16(x) && aligned16(y);
}

template <typename Ti>
int copy_from(int dst_dtype, long long n, const void *x, void *y,
              const StrideDesc &d, int mode) {
  if (mode == 0 && aligned16(x) && aligned16(y)) {
    MMP_DISPATCH_ALL(dst_dtype, {
      constexpr long long tile = (long long)kBlock * (16 / (long long)sizeof(T)) * 4;
      const long long blocks = mmpi::ceil_div(n, tile);
      if (blocks <= 0x7fffffffLL) {
        hipLaunchKernelGGL((k_copy_vec<Ti, T>), dim3((unsigned)blocks), dim3(kBlock), 0,
                           mmpi::stream(), (const Ti *)x, (T *)y, n);
        return mmpi::check_launch("mmp_copy(contiguous)");
      }
      break;  // leave the dtype switch: generic path below
    })
  }
  TransDesc t;
  if (mode != 0 && transpose_desc(d, &t)) {
    long long nbatch = 1;
    for (int k = 0; k < t.nb; ++k) nbatch *= t.bshape[k];
    const long long blocks = nbatch * t.tp * t.tq;
    if (blocks <= 0x7fffffffLL && transpose_vec_ok(t, x, y, 16 / (int)sizeof(Ti))) {
      MMP_DISPATCH_ALL(dst_dtype, {
        if constexpr (__is_same(T, Ti) && sizeof(Ti) >= 2) {  // a plain copy of the bits
          hipLaunchKernelGGL((k_copy_transpose_vec<Ti>), dim3((unsigned)blocks), dim3(kBlock), 0,
                             mmpi::stream(), (const Ti *)x, (Ti *)y, t);
          return mmpi::check_launch("mmp_copy(transpose)");
        }
        break;  // leave the dtype switch: the converting kernel below
      })
    }
    if (blocks <= 0x7fffffffLL) {
      MMP_DISPATCH_ALL(dst_dtype, {
        hipLaunchKernelGGL((k_copy_transpose<Ti, T>), dim3((unsigned)blocks), dim3(kBlock), 0,
                           mmpi::stream(), (const Ti *)x, (T *)y, t);
        return mmpi::check_launch("mmp_copy(transpose)");
      })
    }
  }
  if (mode != 0 && d.ndim >= 2 && d.shape[d.ndim - 1] >= 256) {
    const long long len = d.shape[d.ndim - 1];
    const long long ctiles = mmpi::ceil_div(len, kRowTile);
    const long long blocks = (n / len) * ctiles;
    if (blocks <= 0x7fffffffLL) {
      StrideDesc e = d;
      if (mode == 1) {  // contiguous destination: C strides of the shape
        long long acc = 1;
        for (int k = e.ndim - 1; k >= 0; --k) {
          e.dstride[k] = acc;
          acc *= e.shape[k];
        }
      }
      MMP_DISPATCH_ALL(dst_dtype, {
        hipLaunchKernelGGL((k_copy_rows<Ti, T>), dim3((unsigned)blocks), dim3(kBlock), 0,
                           mmpi::stream(), (const Ti *)x, (T *)y, e, ctiles);
        return mmpi::check_launch("mmp_copy(rows)");
      })
    }
  }
  const long long blocks = mmpi::ceil_div(n, kBlock * 4);
  const unsigned grid = (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
  MMP_DISPATCH_ALL(dst_dtype, {
    hipLaunchKernelGGL((k_copy<Ti, T>), dim3(grid), dim3(kBlock), 0, mmpi::stream(),
                       (const Ti *)x, (T *)y, n, d, mode);
    return mmpi::check_launch("mmp_copy");
  })
}

// Collapse adjacent dimensions that are contiguous in both views and drop
// size-1 dimensions, so common cases reach the linear path.
int build_desc(int ndim, const int64_t *shape, const int64_t *ss,
               const int64_t *ds, StrideDesc *d, long long *n) {
  if (ndim < 0 || ndim > 8) return mmpi::fail(MMP_E_ARG, "ndim %d out of range [0, 8]", ndim);
  long long total = 1;
  int m = 0;
  for (int k = 0; k < ndim; ++k) {
    if (shape[k] < 0) return mmpi::fail(MMP_E_ARG, "negative extent");
    total *= shape[k];
    if (shape[k] == 1) continue;
    const long long sk = ss ? ss[k] : 0, dk = ds ? ds[k] : 0;
    if (m > 0 && d->sstride[m - 1] == sk * shape[k] &&
        d->dstride[m - 1] == dk * shape[k]) {
      d->shape[m - 1] *= shape[k];
      d->sstride[m - 1] = sk;
      d->dstride[m - 1] = dk;
    } else {
      d->shape[m] = shape[k];
      d->sstride[m] = sk;
      d->dstride[m] = dk;
      ++m;
    }
  }
  d->ndim = m;
  *n = total;
  return MMP_OK;
}

}  // namespace

extern "C" int mmp_unary(int op, int dtype, int64_t n, const void *x, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0) return mmpi::fail(MMP_E_ARG, "negative size");
  if (n == 0) return MMP_OK;
  if (!x || !out) return mmpi::fail(MMP_E_ARG, "null pointer");
  MMP_DISPATCH_ALL(dtype, { return unary_for_type<T>(op, n, x, out); })
}

extern "C" int mmp_binary(int op, int dtype, int64_t n, const void *a,
                          const void *b, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0) return mmpi::fail(MMP_E_ARG, "negative size");
  if (n == 0) return MMP_OK;
  if (!a || !b || !out) return mmpi::fail(MMP_E_ARG, "null pointer");
  MMP_DISPATCH_ALL(dtype, { return binary_for_type<T>(op, n, a, b, nullptr, 0, out); })
}

extern "C" int mmp_binary_scalar(int op, int dtype, int64_t n, const void *arr,
                                 const void *scalar, int scalar_side, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0) return mmpi::fail(MMP_E_ARG, "negative size");
  if (n == 0) return MMP_OK;
  if (!arr || !scalar || !out) return mmpi::fail(MMP_E_ARG, "null pointer");
  if (scalar_side != 0 && scalar_side != 1)
    return mmpi::fail(MMP_E_ARG, "scalar_side must be 0 or 1");
  const int mode = scalar_side == 0 ? 1 : 2;
  MMP_DISPATCH_ALL(dtype, { return binary_for_type<T>(op, n, arr, arr, scalar, mode, out); })
}

extern "C" int mmp_copy(int src_dtype, int dst_dtype, int ndim, const int64_t *shape,
                        const void *x, const int64_t *x_strides, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (ndim > 0 && (!shape || !x_strides)) return mmpi::fail(MMP_E_ARG, "null shape/strides");
  StrideDesc d{};
  long long n = 1;
  // destination strides: C-contiguous over the original shape
  int64_t dstr[8];
  if (ndim > 8) return mmpi::fail(MMP_E_ARG, "ndim %d > 8", ndim);
  long long acc = 1;
  for (int k = ndim - 1; k >= 0; --k) { dstr[k] = acc; acc *= shape[k]; }
  if (int st = build_desc(ndim, shape, x_strides, dstr, &d, &n)) return st;
  if (n == 0) return MMP_OK;
  if (!x || !out) return mmpi::fail(MMP_E_ARG, "null pointer");
  int mode = 1;
  if (d.ndim == 0 || (d.ndim == 1 && d.sstride[0] == 1)) mode = 0;
  MMP_DISPATCH_ALL(src_dtype, { return copy_from<T>(dst_dtype, n, x, out, d, mode); })
}

extern "C" int mmp_copy_strided(int src_dtype, int dst_dtype, int ndim,
                                const int64_t *shape, const void *src,
                                const int64_t *src_strides, void *dst,
                                const int64_t *dst_strides) {
  if (int st = mmpi::ensure_init()) return st;
  if (ndim > 0 && (!shape || !src_strides || !dst_strides))
    return mmpi::fail(MMP_E_ARG, "null shape/strides");
  StrideDesc d{};
  long long n = 1;
  if (int st = build_desc(ndim, shape, src_strides, dst_strides, &d, &n)) return st;
  if (n == 0) return MMP_OK;
  if (!src || !dst) return mmpi::fail(MMP_E_ARG, "null pointer");
  int mode = 2;
  if (d.ndim == 0 || (d.ndim == 1 && d.sstride[0] == 1 && d.dstride[0] == 1)) mode = 0;
  MMP_DISPATCH_ALL(src_dtype, { return copy_from<T>(dst_dtype, n, src, dst, d, mode); })
}

extern "C" int mmp_fill(int dtype, int64_t n, const void *value, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0) return mmpi::fail(MMP_E_ARG, "negative size");
  if (n == 0) return MMP_OK;
  if (!value || !out) return mmpi::fail(MMP_E_ARG, "null pointer");
  const long long blocks = mmpi::ceil_div(n, kBlock * 4);
  const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
  MMP_DISPATCH_ALL(dtype, {
    T v = *reinterpret_cast<const T *>(value);
    hipLaunchKernelGGL((k_fill<T>), dim3(grid), dim3(kBlock), 0, mmpi::stream(), (T *)out, n, v);
    return mmpi::check_launch("mmp_fill");
  })
}
