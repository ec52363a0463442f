// reduce.hip -- sum / mean / prod / max / min and argmax / argmin.
//
// Replaces the reference's multi-pass Metal reductions: reduce_sum & co.
// (_kernels.py:422-565; one pass per factor of 8192, re-launched from
// Python, ndarray.py:1927-1946), the one-thread-per-row axis kernels
// (_kernels.py:1062-1146) and the two-pass argmax whose second pass is a
// single thread (_kernels.py:1189-1243).
//
// The input is viewed as C-contiguous (outer, len, inner) and the middle
// axis is reduced.
//  * inner == 1 (contiguous rows, includes axis=None as one row): each row
//    is split over S workgroups so that the launch has >= ~2048 of them;
//    a workgroup streams its slice with 128-bit loads, reduces in
//    registers, across the wave64 with butterfly shuffles and across the 4
//    waves through LDS.  With S > 1 the partials go to scratch and the last
//    workgroup of the row to arrive (atomic ticket) combines them in index
//    order -- one launch, deterministic result.
//  * inner > 1 (strided axis): one thread per output column, coalesced
//    across the column index, the reduced axis optionally split over S
//    workgroups with the same ticket scheme.
// Floating sums/means/products accumulate in float64 and round once
// (accuracy bar: 1e-5 relative to a float64-accumulated reference); integer
// sums widen to 64 bits as NumPy does.  HBM-bound: algorithmic bytes =
// sizeof(T) per input element (+ outputs).
#include <algorithm>

#include "mmp_ops.h"
#include "mmp_internal.h"

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
// Split policy (tuning constants, overridable at build time for sweeps):
// at least kMinPerBlock elements per workgroup, about kTargetBlocks
// workgroups per launch, at most kMaxSplits workgroups per row.
#ifndef MMP_REDUCE_TARGET_BLOCKS
#define MMP_REDUCE_TARGET_BLOCKS 1024
#endif
#ifndef MMP_REDUCE_UNROLL
#define MMP_REDUCE_UNROLL 8
#endif
constexpr long long kMinPerBlock = 16384;
constexpr long long kTargetBlocks = MMP_REDUCE_TARGET_BLOCKS;
constexpr long long kTargetBlocksOneRow = 512;
constexpr long long kMaxSplits = 16384;
constexpr int kUnroll = MMP_REDUCE_UNROLL;   // 16-byte loads in flight per thread
constexpr int kColUnroll = 8;                // strided layouts: rows in flight per thread

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <typename T> union Pack {
  u32x4 v;
  T e[16 / sizeof(T)];
};

// --------------------------------------------------------------- ops
template <typename T> struct AccOf {  // accumulator for sum / prod / mean
  typedef typename mmp_t<T>::C C;
  typedef double type;
};
template <> struct AccOf<mmp_i16> { typedef mmp_i64 type; };
template <> struct AccOf<mmp_i32> { typedef mmp_i64 type; };
template <> struct AccOf<mmp_i64> { typedef mmp_i64 type; };
template <> struct AccOf<bool> { typedef mmp_i64 type; };
template <> struct AccOf<mmp_u16> { typedef mmp_u64 type; };
template <> struct AccOf<mmp_u32> { typedef mmp_u64 type; };
template <> struct AccOf<mmp_u64> { typedef mmp_u64 type; };

// Reduction policies: identity, element map, combine, finalize.
template <int OP, typename T> struct Red;

template <typename T> struct Red<MMP_R_SUM, T> {
  typedef typename AccOf<T>::type A;
  static __device__ __forceinline__ A ident() { return (A)0; }
  static __device__ __forceinline__ A map(T v) {
    if constexpr (mmp_t<T>::is_float) return (A)(typename mmp_t<T>::C)v;
    else return (A)v;
  }
  static __device__ __forceinline__ A comb(A a, A b) {
    if constexpr (mmp_t<T>::is_float) return a + b;
    else return (A)((mmp_u64)a + (mmp_u64)b);
  }
};
template <typename T> struct Red<MMP_R_MEAN, T> : Red<MMP_R_SUM, T> {
  typedef double A;
  static __device__ __forceinline__ A ident() { return 0.0; }
  static __device__ __forceinline__ A map(T v) {
    if constexpr (mmp_t<T>::is_float) return (double)(typename mmp_t<T>::C)v;
    else return (double)v;
  }
  static __device__ __forceinline__ A comb(A a, A b) { return a + b; }
};
template <typename T> struct Red<MMP_R_PROD, T> {
  typedef typename AccOf<T>::type A;
  static __device__ __forceinline__ A ident() { return (A)1; }
  static __device__ __forceinline__ A map(T v) {
    if constexpr (mmp_t<T>::is_float) return (A)(typename mmp_t<T>::C)v;
    else return (A)v;
  }
  static __device__ __forceinline__ A comb(A a, A b) {
    if constexpr (mmp_t<T>::is_float) return a * b;
    else return (A)((mmp_u64)a * (mmp_u64)b);
  }
};
// max / min in the compute type; NaN propagates; ties keep the first
template <typename T> struct Red<MMP_R_MAX, T> {
  typedef typename mmp_t<T>::C A;
  static __device__ __forceinline__ A ident() {
    if constexpr (mmp_t<T>::is_float) return -__builtin_huge_valf();
    else return (A)mmp_t<T>::lowest;
  }
  static __device__ __forceinline__ A map(T v) { return (A)v; }
  static __device__ __forceinline__ A comb(A a, A b) {
    if constexpr (mmp_t<T>::is_float) {
      if (a != a) return a;
      if (b != b) return b;
    }
    return b > a ? b : a;
  }
};
template <typename T> struct Red<MMP_R_MIN, T> {
  typedef typename mmp_t<T>::C A;
  static __device__ __forceinline__ A ident() {
    if constexpr (mmp_t<T>::is_float) return __builtin_huge_valf();
    else if constexpr (mmp_t<T>::is_bool) return (A)1;
    else return (A)~(typename mmp_t<T>::U)mmp_t<T>::lowest;
  }
  static __device__ __forceinline__ A map(T v) { return (A)v; }
  static __device__ __forceinline__ A comb(A a, A b) {
    if constexpr (mmp_t<T>::is_float) {
      if (a != a) return a;
      if (b != b) return b;
    }
    return b < a ? b : a;
  }
};

// NaN-ignoring variants (numpy nansum / nanprod / nanmax / nanmin /
// nanmean): a NaN element maps to the identity.  nanmax / nanmin start from
// NaN and replace it by the first non-NaN value, so an all-NaN slice stays
// NaN; nanmean carries (sum, count) and an empty count gives 0/0 = NaN.
template <typename T> MMP_DI bool is_nan_elem(T v) {
  if constexpr (mmp_t<T>::is_float) return (typename mmp_t<T>::C)v != (typename mmp_t<T>::C)v;
  else return false;
}
template <typename T> struct Red<MMP_R_NANSUM, T> : Red<MMP_R_SUM, T> {
  typedef typename Red<MMP_R_SUM, T>::A A;
  static __device__ __forceinline__ A map(T v) {
    return is_nan_elem(v) ? (A)0 : Red<MMP_R_SUM, T>::map(v);
  }
};
template <typename T> struct Red<MMP_R_NANPROD, T> : Red<MMP_R_PROD, T> {
  typedef typename Red<MMP_R_PROD, T>::A A;
  static __device__ __forceinline__ A map(T v) {
    return is_nan_elem(v) ? (A)1 : Red<MMP_R_PROD, T>::map(v);
  }
};
template <int OP, typename T> struct RedNanExt {  // OP: MMP_R_MAX or MMP_R_MIN
  typedef typename mmp_t<T>::C A;
  static __device__ __forceinline__ A ident() {
    if constexpr (mmp_t<T>::is_float) return (A)__builtin_nanf("");
    else return Red<OP, T>::ident();
  }
  static __device__ __forceinline__ A map(T v) { return (A)v; }
  static __device__ __forceinline__ A comb(A a, A b) {
    if constexpr (mmp_t<T>::is_float) {
      if (a != a) return b;
      if (b != b) return a;
    }
    if constexpr (OP == MMP_R_MAX) return b > a ? b : a;
    else return b < a ? b : a;
  }
};
template <typename T> struct Red<MMP_R_NANMAX, T> : RedNanExt<MMP_R_MAX, T> {};
template <typename T> struct Red<MMP_R_NANMIN, T> : RedNanExt<MMP_R_MIN, T> {};
struct MeanAcc {
  double s, n;
};
template <typename T> struct Red<MMP_R_NANMEAN, T> {
  typedef MeanAcc A;
  static __device__ __forceinline__ A ident() { return A{0.0, 0.0}; }
  static __device__ __forceinline__ A map(T v) {
    if (is_nan_elem(v)) return A{0.0, 0.0};
    if constexpr (mmp_t<T>::is_float) return A{(double)(typename mmp_t<T>::C)v, 1.0};
    else return A{(double)v, 1.0};
  }
  static __device__ __forceinline__ A comb(A a, A b) { return A{a.s + b.s, a.n + b.n}; }
};

// argmax / argmin pair; "better" = NaN first, then extreme value, then
// smaller index.  The NaN-ignoring variants never take a NaN: an all-NaN
// slice keeps the identity's index (INT64_MAX).
template <typename C> struct ArgPair {
  C v;
  long long i;
};
template <int OP, typename T> struct Arg {
  typedef typename mmp_t<T>::C C;
  typedef ArgPair<C> A;
  static constexpr bool kMax = OP == MMP_R_ARGMAX || OP == MMP_R_NANARGMAX;
  static constexpr bool kSkipNaN = OP == MMP_R_NANARGMAX || OP == MMP_R_NANARGMIN;
  static __device__ __forceinline__ A ident() {
    A a;
    if constexpr (mmp_t<T>::is_float) a.v = kMax ? -__builtin_huge_valf() : __builtin_huge_valf();
    else if constexpr (kMax) a.v = (C)mmp_t<T>::lowest;
    else if constexpr (mmp_t<T>::is_bool) a.v = (C)1;
    else a.v = (C)~(typename mmp_t<T>::U)mmp_t<T>::lowest;
    a.i = 0x7fffffffffffffffLL;
    return a;
  }
  static __device__ __forceinline__ bool better(const A &x, const A &y) {  // x before y?
    if constexpr (mmp_t<T>::is_float) {
      const bool xn = x.v != x.v, yn = y.v != y.v;
      if constexpr (kSkipNaN) {
        if (xn) return false;
        if (yn) return true;
      } else {
        if (xn || yn) return xn && (!yn || x.i < y.i);
      }
    }
    if (x.v == y.v) return x.i < y.i;
    return kMax ? x.v > y.v : x.v < y.v;
  }
  static __device__ __forceinline__ A comb(const A &x, const A &y) { return better(y, x) ? y : x; }
  // v (visited later) replaces the running best b of one thread's sequence
  static __device__ __forceinline__ bool seq_better(C v, C b) {
    bool r = kMax ? v > b : v < b;
    if constexpr (mmp_t<T>::is_float && !kSkipNaN) r |= (v != v) & (b == b);
    return r;
  }
  // whether an element may become the running best at all
  static __device__ __forceinline__ bool eligible(C v) {
    if constexpr (mmp_t<T>::is_float && kSkipNaN) return v == v;
    else return true;
  }
};

// --------------------------------------------------- wave / block reduce
template <typename A> __device__ __forceinline__ A shfl_xor(A v, int m) {
  if constexpr (sizeof(A) == 16) {
    u32x4 w = __builtin_bit_cast(u32x4, v);
#pragma unroll
    for (int k = 0; k < 4; ++k) w[k] = __shfl_xor(w[k], m, 64);
    return __builtin_bit_cast(A, w);
  } else if constexpr (sizeof(A) == 8) {
    unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    unsigned lo = (unsigned)u, hi = (unsigned)(u >> 32);
    lo = __shfl_xor(lo, m, 64);
    hi = __shfl_xor(hi, m, 64);
    return __builtin_bit_cast(A, ((unsigned long long)hi << 32) | lo);
  } else if constexpr (sizeof(A) == 4) {
    return __builtin_bit_cast(A, __shfl_xor(__builtin_bit_cast(unsigned, v), m, 64));
  } else {
    return (A)__shfl_xor((int)v, m, 64);
  }
}

template <typename R, typename A> __device__ __forceinline__ A wave_reduce(A v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = R::comb(v, shfl_xor(v, m));
  return v;
}
template <typename R, typename C> __device__ __forceinline__ ArgPair<C> wave_reduce_arg(ArgPair<C> v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    ArgPair<C> o;
    o.v = shfl_xor(v.v, m);
    o.i = shfl_xor(v.i, m);
    v = R::comb(v, o);
  }
  return v;
}

template <typename A> struct IsArgPair { static constexpr bool value = false; };
template <typename C> struct IsArgPair<ArgPair<C>> { static constexpr bool value = true; };

// Block-wide reduce; the result is valid in thread 0.
template <typename R, typename A> __device__ A block_reduce(A v, A *lds) {
  if constexpr (IsArgPair<A>::value) {
    v = wave_reduce_arg<R>(v);
  } else {
    v = wave_reduce<R>(v);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) lds[w] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int k = 1; k < kWaves; ++k) v = R::comb(v, lds[k]);
  }
  return v;
}

// Slice reduction over contiguous [p, p + n), element index base `i0`
// (used by argmax).  Called by all threads of the block.
template <typename R, typename T>
__device__ __forceinline__ typename R::A slice_reduce(const T *__restrict__ p, long long n,
                                                      long long i0) {
  typedef typename R::A A;
  constexpr int V = 16 / sizeof(T);
  A acc0 = R::ident(), acc1 = R::ident();
  const unsigned tid = threadIdx.x;
  // head until 16-byte alignment
  long long head = (long long)(((16 - ((uintptr_t)p & 15u)) & 15u) / sizeof(T));
  if (((uintptr_t)p % sizeof(T)) != 0) head = n;  // cannot vectorise
  if (head > n) head = n;
  for (long long i = tid; i < head; i += kBlock) acc0 = R::comb(acc0, R::map(p[i]));
  const long long nvec = (n - head) / V;
  const u32x4 *pv = reinterpret_cast<const u32x4 *>(p + head);
  long long j = tid;
  for (; j + (kUnroll - 1) * kBlock < nvec; j += kUnroll * kBlock) {
    Pack<T> q[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) q[u].v = __builtin_nontemporal_load(pv + j + u * kBlock);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        if (e & 1) acc1 = R::comb(acc1, R::map(q[u].e[e]));
        else acc0 = R::comb(acc0, R::map(q[u].e[e]));
      }
    }
  }
  for (; j < nvec; j += kBlock) {
    Pack<T> q;
    q.v = __builtin_nontemporal_load(pv + j);
#pragma unroll
    for (int e = 0; e < V; ++e) acc0 = R::comb(acc0, R::map(q.e[e]));
  }
  for (long long i = head + nvec * V + tid; i < n; i += kBlock) acc0 = R::comb(acc0, R::map(p[i]));
  (void)i0;
  return R::comb(acc0, acc1);
}

// argmax slice: same traversal, carrying indices.  Each thread visits its
// elements in increasing index order, so within a thread a strict
// comparison keeps the first occurrence of the extreme and no index
// comparison is needed; indices are 32-bit offsets into the slice.  A NaN
// replaces a non-NaN best (the first NaN wins, as NumPy), and the first
// visited element always replaces the "nothing yet" state (so a row whose
// extreme equals the identity, e.g. all -inf, still reports index 0).
// Ties across threads are resolved by R::comb (smaller index).
template <typename R, typename T>
__device__ __forceinline__ typename R::A slice_argreduce(const T *__restrict__ p, long long n,
                                                         long long i0) {
  typedef typename R::A A;
  typedef typename mmp_t<T>::C C;
  constexpr int V = 16 / sizeof(T);
  constexpr unsigned kNone = 0xffffffffu;
  if (n >= (long long)kNone) {  // offsets would not fit in 32 bits: generic path
    A best = R::ident();
    for (long long i = threadIdx.x; i < n; i += kBlock) best = R::comb(best, A{(C)p[i], i0 + i});
    return best;
  }
  C bv = R::ident().v;
  unsigned bi = kNone;
  auto visit = [&](C v, unsigned off) {
    bool upd = (R::seq_better(v, bv) | (bi == kNone)) & R::eligible(v);
    bv = upd ? v : bv;
    bi = upd ? off : bi;
  };
  const unsigned tid = threadIdx.x;
  const unsigned un = (unsigned)n;
  unsigned head = (unsigned)(((16 - ((uintptr_t)p & 15u)) & 15u) / sizeof(T));
  if (((uintptr_t)p % sizeof(T)) != 0) head = un;
  if (head > un) head = un;
  for (unsigned i = tid; i < head; i += kBlock) visit((C)p[i], i);
  const unsigned nvec = (un - head) / V;
  const u32x4 *pv = reinterpret_cast<const u32x4 *>(p + head);
  unsigned j = tid;
  for (; j + (kUnroll - 1) * kBlock < nvec; j += kUnroll * kBlock) {
    Pack<T> q[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) q[u].v = __builtin_nontemporal_load(pv + j + u * kBlock);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const unsigned ib = head + (j + u * kBlock) * V;
#pragma unroll
      for (int e = 0; e < V; ++e) visit((C)q[u].e[e], ib + e);
    }
  }
  for (; j < nvec; j += kBlock) {
    Pack<T> q;
    q.v = __builtin_nontemporal_load(pv + j);
    const unsigned ib = head + j * V;
#pragma unroll
    for (int e = 0; e < V; ++e) visit((C)q.e[e], ib + e);
  }
  for (unsigned i = head + nvec * V + tid; i < un; i += kBlock) visit((C)p[i], i);
  if (bi == kNone) return R::ident();
  return A{bv, i0 + (long long)bi};
}

// ------------------------------------------------------ finalizers
template <int OP, typename T, typename To, typename A>
__device__ __forceinline__ To finalize(A a, long long len) {
  if constexpr (OP == MMP_R_MEAN) {
    return mmp_convert<To, double>(a / (double)len);
  } else if constexpr (OP == MMP_R_NANMEAN) {
    return mmp_convert<To, double>(a.s / a.n);
  } else if constexpr (OP == MMP_R_MAX || OP == MMP_R_MIN || OP == MMP_R_NANMAX ||
                       OP == MMP_R_NANMIN) {
    if constexpr (sizeof(T) == 2 && mmp_t<T>::is_float) return mmp_convert<To, T>((T)a);
    else return mmp_convert<To, A>(a);
  } else {
    return mmp_convert<To, A>(a);
  }
}

// ------------------------------------------------ cross-workgroup words
// Workgroups of one row exchange their partials through scratch words that
// validate themselves: every 64-bit word holds a 32-bit call tag in its high
// half and 32 payload bits in its low half, and is written / read with
// RELAXED agent-scope atomics.  The reader spins until the tag matches the
// current call.  No release/acquire fence is needed -- on multi-XCD CDNA an
// agent-scope fence writes back / invalidates the whole L2 of the XCD, which
// costs far more than the partial itself.
template <typename A> constexpr int words_of() { return (int)((sizeof(A) + 3) / 4); }

template <typename A>
__device__ __forceinline__ void put_tagged(unsigned long long *slot, const A &v, unsigned tag) {
  constexpr int W = words_of<A>();
  unsigned buf[W] = {};
  __builtin_memcpy(buf, &v, sizeof(A));
#pragma unroll
  for (int k = 0; k < W; ++k)
    __hip_atomic_store(slot + k, ((unsigned long long)tag << 32) | buf[k], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Spins (bounded) until every word of the slot carries `tag`.
template <typename A>
__device__ __forceinline__ A get_tagged(const unsigned long long *slot, unsigned tag,
                                        unsigned *timeout, long long spin_limit) {
  constexpr int W = words_of<A>();
  unsigned buf[W];
#pragma unroll
  for (int k = 0; k < W; ++k) {
    unsigned long long w;
    long long spins = 0;
    while (((w = __hip_atomic_load(slot + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) >> 32) !=
           tag) {
      if (++spins > spin_limit) {
        __hip_atomic_store(timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    buf[k] = (unsigned)w;
  }
  A v;
  __builtin_memcpy(&v, buf, sizeof(A));
  return v;
}

struct ReduceScratch {
  unsigned long long *words;  // tagged partial words
  unsigned *tickets;          // arrival counters (left at 0)
  unsigned *timeout;          // pinned host word, set to 1 if a wait ran out
  unsigned tag;               // this call's generation (written)
  unsigned read_tag;          // tag the combine waits for (== tag unless forced)
  long long spin_limit;       // bound of every wait
};

// Combines S tagged partials, slot j at base + j * stride words, in index
// order (deterministic).  The loads of kBatch partials go out before any of
// them is checked, so one thread pays the atomic-load latency once per
// batch rather than once per partial; a partial whose tag is not there yet
// is waited for as get_tagged does.
template <typename R>
__device__ __forceinline__ typename R::A combine_tagged(const unsigned long long *base,
                                                        long long stride, int S,
                                                        const ReduceScratch &sc) {
  typedef typename R::A A;
  constexpr int W = words_of<A>();
  constexpr int kBatch = 8;
  A acc = R::ident();
  for (int j0 = 0; j0 < S; j0 += kBatch) {
    unsigned long long w[kBatch][W];
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
#pragma unroll
      for (int k = 0; k < W; ++k)
        w[b][k] = j0 + b < S ? __hip_atomic_load(base + (long long)(j0 + b) * stride + k,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : 0ull;
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (j0 + b >= S) break;
      bool ok = true;
#pragma unroll
      for (int k = 0; k < W; ++k) ok = ok && (unsigned)(w[b][k] >> 32) == sc.read_tag;
      A part;
      if (ok) {
        unsigned buf[W];
#pragma unroll
        for (int k = 0; k < W; ++k) buf[k] = (unsigned)w[b][k];
        __builtin_memcpy(&part, buf, sizeof(A));
      } else {
        part = get_tagged<A>(base + (long long)(j0 + b) * stride, sc.read_tag, sc.timeout,
                             sc.spin_limit);
      }
      acc = R::comb(acc, part);
    }
  }
  return acc;
}

// Last-arrival combine of the S partials of one row.  Returns true in the
// workgroup that finishes the row; its thread 0 then holds the result in
// *out.  Partials are combined in index order (deterministic).
template <typename R>
__device__ bool last_block_combine(typename R::A v, unsigned long long *words, unsigned *ticket,
                                   int S, int s, const ReduceScratch &sc, typename R::A *out,
                                   typename R::A *lds) {
  typedef typename R::A A;
  constexpr int W = words_of<A>();
  __shared__ int is_last;
  if (threadIdx.x == 0) {
    put_tagged(words + (long long)s * W, v, sc.tag);
    const unsigned t = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (t == (unsigned)(S - 1));
  }
  __syncthreads();
  if (!is_last) return false;
  // Issue the loads of kBatch partials before validating any of them, so
  // the last workgroup pays the atomic-load latency once per batch.
  constexpr int kBatch = 8;
  A acc = R::ident();
  for (int k0 = threadIdx.x; k0 < S; k0 += kBlock * kBatch) {
    unsigned long long w[kBatch][W];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int k = k0 + b * kBlock;
#pragma unroll
      for (int j = 0; j < W; ++j)
        w[b][j] = k < S ? __hip_atomic_load(words + (long long)k * W + j, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT)
                        : 0ull;
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int k = k0 + b * kBlock;
      if (k >= S) break;
      bool ok = true;
#pragma unroll
      for (int j = 0; j < W; ++j) ok = ok && (unsigned)(w[b][j] >> 32) == sc.read_tag;
      A part;
      if (ok) {
        unsigned buf[W];
#pragma unroll
        for (int j = 0; j < W; ++j) buf[j] = (unsigned)w[b][j];
        __builtin_memcpy(&part, buf, sizeof(A));
      } else {
        part = get_tagged<A>(words + (long long)k * W, sc.read_tag, sc.timeout, sc.spin_limit);
      }
      acc = R::comb(acc, part);
    }
  }
  __syncthreads();
  acc = block_reduce<R>(acc, lds);
  if (threadIdx.x == 0) {
    *out = acc;
    __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return true;
}

// ---------------------------------------------------------- kernels
// Rows: grid = rows * S; workgroup (row, s) reduces slice s of its row.
template <int OP, typename T, typename To>
__global__ __launch_bounds__(kBlock) void k_reduce_rows(const T *__restrict__ x, To *__restrict__ out,
                                                       long long len, int S, ReduceScratch sc) {
  typedef Red<OP, T> R;
  typedef typename R::A A;
  __shared__ A lds[kWaves];
  const long long row = blockIdx.x / S;
  const int s = (int)(blockIdx.x - row * S);
  const long long per = (len + S - 1) / S;
  const long long b0 = s * per;
  const long long b1 = b0 + per < len ? b0 + per : len;
  A v = R::ident();
  if (b0 < b1) v = slice_reduce<R, T>(x + row * len + b0, b1 - b0, b0);
  v = block_reduce<R>(v, lds);
  if (S == 1) {
    if (threadIdx.x == 0) out[row] = finalize<OP, T, To>(v, len);
    return;
  }
  A total;
  __syncthreads();
  if (last_block_combine<R>(v, sc.words + row * S * words_of<A>(), sc.tickets + row, S, s, sc,
                            &total, lds) &&
      threadIdx.x == 0)
    out[row] = finalize<OP, T, To>(total, len);
}

template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void k_argreduce_rows(const T *__restrict__ x,
                                                          long long *__restrict__ out,
                                                          long long len, int S, ReduceScratch sc) {
  typedef Arg<OP, T> R;
  typedef typename R::A A;
  __shared__ A lds[kWaves];
  const long long row = blockIdx.x / S;
  const int s = (int)(blockIdx.x - row * S);
  const long long per = (len + S - 1) / S;
  const long long b0 = s * per;
  const long long b1 = b0 + per < len ? b0 + per : len;
  A v = R::ident();
  if (b0 < b1) v = slice_argreduce<R, T>(x + row * len + b0, b1 - b0, b0);
  v = block_reduce<R>(v, lds);
  if (S == 1) {
    if (threadIdx.x == 0) out[row] = v.i;
    return;
  }
  A total;
  __syncthreads();
  if (last_block_combine<R>(v, sc.words + row * S * words_of<A>(), sc.tickets + row, S, s, sc,
                            &total, lds) &&
      threadIdx.x == 0)
    out[row] = total.i;
}

// Strided axis: grid (ceil(inner / 256), outer, S); thread = column.
template <int OP, typename T, typename To>
__global__ __launch_bounds__(kBlock) void k_reduce_cols(const T *__restrict__ x, To *__restrict__ out,
                                                       long long len, long long inner, int S,
                                                       ReduceScratch sc) {
  typedef Red<OP, T> R;
  typedef typename R::A A;
  constexpr int W = words_of<A>();
  const long long o = blockIdx.y;
  const int s = blockIdx.z;
  const long long c = (long long)blockIdx.x * kBlock + threadIdx.x;
  const long long per = (len + S - 1) / S;
  const long long b0 = s * per;
  const long long b1 = b0 + per < len ? b0 + per : len;
  A v = R::ident();
  if (c < inner) {
    const T *p = x + o * len * inner + c;
    long long l = b0;
    for (; l + kColUnroll <= b1; l += kColUnroll) {  // loads first: kColUnroll in flight
      T q[kColUnroll];
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u) q[u] = p[(l + u) * inner];
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u) v = R::comb(v, R::map(q[u]));
    }
    for (; l < b1; ++l) v = R::comb(v, R::map(p[l * inner]));
  }
  if (S == 1) {
    if (c < inner) out[o * inner + c] = finalize<OP, T, To>(v, len);
    return;
  }
  // one tagged partial per (o, column block, s, thread); ticket per (o, cb)
  const long long cb = blockIdx.x, ncb = gridDim.x;
  unsigned long long *grp = sc.words + (o * ncb + cb) * (long long)S * kBlock * W;
  put_tagged(grp + ((long long)s * kBlock + threadIdx.x) * W, v, sc.tag);
  __shared__ int is_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned t = __hip_atomic_fetch_add(sc.tickets + o * ncb + cb, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    is_last = (t == (unsigned)(S - 1));
  }
  __syncthreads();
  if (!is_last) return;
  const A acc = combine_tagged<R>(grp + (long long)threadIdx.x * W, (long long)kBlock * W, S, sc);
  if (c < inner) out[o * inner + c] = finalize<OP, T, To>(acc, len);
  if (threadIdx.x == 0)
    __hip_atomic_store(sc.tickets + o * ncb + cb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Strided arg-reduction: grid (ceil(inner / 256), outer, S); thread =
// column, the reduced axis split over S workgroups combined in index order
// by the last to arrive (as k_reduce_cols).
template <int OP, typename T>
__global__ __launch_bounds__(kBlock) void k_argreduce_cols(const T *__restrict__ x,
                                                          long long *__restrict__ out,
                                                          long long len, long long inner, int S,
                                                          ReduceScratch sc) {
  typedef Arg<OP, T> R;
  typedef typename R::A A;
  typedef typename mmp_t<T>::C C;
  constexpr int W = words_of<A>();
  const long long o = blockIdx.y;
  const int s = blockIdx.z;
  const long long c = (long long)blockIdx.x * kBlock + threadIdx.x;
  const long long per = (len + S - 1) / S;
  const long long b0 = s * per;
  const long long b1 = b0 + per < len ? b0 + per : len;
  A v = R::ident();
  if (c < inner) {
    const T *p = x + o * len * inner + c;
    long long l = b0;
    if (b1 - b0 < 0xffffffffLL) {
      // rows are visited in order: the sequential update rule with 32-bit
      // offsets from b0 (as slice_argreduce) instead of the index-comparing
      // combine per element
      constexpr unsigned kNone = 0xffffffffu;
      C bv = R::ident().v;
      unsigned bi = kNone;
      auto visit = [&](C e, unsigned off) {
        const bool upd = (R::seq_better(e, bv) | (bi == kNone)) & R::eligible(e);
        bv = upd ? e : bv;
        bi = upd ? off : bi;
      };
      for (; l + kColUnroll <= b1; l += kColUnroll) {
        T q[kColUnroll];
#pragma unroll
        for (int u = 0; u < kColUnroll; ++u) q[u] = p[(l + u) * inner];
#pragma unroll
        for (int u = 0; u < kColUnroll; ++u) visit((C)q[u], (unsigned)(l + u - b0));
      }
      for (; l < b1; ++l) visit((C)p[l * inner], (unsigned)(l - b0));
      if (bi != kNone) v = A{bv, b0 + (long long)bi};
    } else {
      for (; l + kColUnroll <= b1; l += kColUnroll) {
        T q[kColUnroll];
#pragma unroll
        for (int u = 0; u < kColUnroll; ++u) q[u] = p[(l + u) * inner];
#pragma unroll
        for (int u = 0; u < kColUnroll; ++u) v = R::comb(v, A{(C)q[u], l + u});
      }
      for (; l < b1; ++l) v = R::comb(v, A{(C)p[l * inner], l});
    }
  }
  if (S == 1) {
    if (c < inner) out[o * inner + c] = v.i;
    return;
  }
  const long long cb = blockIdx.x, ncb = gridDim.x;
  unsigned long long *grp = sc.words + (o * ncb + cb) * (long long)S * kBlock * W;
  put_tagged(grp + ((long long)s * kBlock + threadIdx.x) * W, v, sc.tag);
  __shared__ int is_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned t = __hip_atomic_fetch_add(sc.tickets + o * ncb + cb, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    is_last = (t == (unsigned)(S - 1));
  }
  __syncthreads();
  if (!is_last) return;
  const A acc = combine_tagged<R>(grp + (long long)threadIdx.x * W, (long long)kBlock * W, S, sc);
  if (c < inner) out[o * inner + c] = acc.i;
  if (threadIdx.x == 0)
    __hip_atomic_store(sc.tickets + o * ncb + cb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Strided axis with 16-byte column vectors (element size 2, 4 or 8 bytes,
// inner extent a multiple of the vector, 16-byte aligned base): grid
// (ceil(inner / CW), outer, S) with CW = 64 x VI columns per workgroup.
// A lane owns VI adjacent columns and each wave takes every fourth row of
// the split (one 1 KiB row segment per wave load, kColUnroll loads in
// flight); the four waves' partials meet in LDS in wave order, then one
// partial per (split, column) is combined in split order by the last
// workgroup to arrive, as in k_reduce_cols.  Sums accumulate in the same
// types; only the order of additions inside a split differs.
template <typename T> constexpr int col_vec() { return 16 / (int)sizeof(T); }
template <typename T> constexpr int col_width() { return 64 * col_vec<T>(); }

template <typename R, typename T, typename MapF, typename StoreF>
__device__ __forceinline__ void cols_vec_body(const T *__restrict__ x, long long len,
                                              long long inner, int S, const ReduceScratch &sc,
                                              MapF map, StoreF store) {
  typedef typename R::A A;
  constexpr int W = words_of<A>();
  constexpr int VI = col_vec<T>();
  constexpr int CW = col_width<T>();
  constexpr int KC = (CW + kBlock - 1) / kBlock;  // columns per thread in the combine
  __shared__ A part[kWaves][CW];
  __shared__ int is_last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long long o = blockIdx.y;
  const int s = blockIdx.z;
  const long long c0 = (long long)blockIdx.x * CW;
  const long long c = c0 + (long long)lane * VI;
  const long long per = (len + S - 1) / S;
  const long long b0 = s * per;
  const long long b1 = b0 + per < len ? b0 + per : len;
  A v[VI];
#pragma unroll
  for (int e = 0; e < VI; ++e) v[e] = R::ident();
  if (c < inner) {
    const T *p = x + o * len * inner + c;
    long long l = b0 + wave;
    for (; l + (long long)kWaves * (kColUnroll - 1) < b1; l += (long long)kWaves * kColUnroll) {
      u32x4 q[kColUnroll];
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u)
        q[u] = *reinterpret_cast<const u32x4 *>(p + (l + (long long)kWaves * u) * inner);
#pragma unroll
      for (int u = 0; u < kColUnroll; ++u) {
        Pack<T> pk;
        pk.v = q[u];
#pragma unroll
        for (int e = 0; e < VI; ++e) v[e] = R::comb(v[e], map(pk.e[e], l + (long long)kWaves * u));
      }
    }
    for (; l < b1; l += kWaves) {
      Pack<T> pk;
      pk.v = *reinterpret_cast<const u32x4 *>(p + l * inner);
#pragma unroll
      for (int e = 0; e < VI; ++e) v[e] = R::comb(v[e], map(pk.e[e], l));
    }
  }
#pragma unroll
  for (int e = 0; e < VI; ++e) part[wave][lane * VI + e] = v[e];
  __syncthreads();
  A acc[KC];
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int cc = threadIdx.x + k * kBlock;
    acc[k] = R::ident();
    if (cc < CW) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) acc[k] = R::comb(acc[k], part[w][cc]);
    }
  }
  if (S == 1) {
#pragma unroll
    for (int k = 0; k < KC; ++k) {
      const int cc = threadIdx.x + k * kBlock;
      if (cc < CW && c0 + cc < inner) store(o * inner + c0 + cc, acc[k]);
    }
    return;
  }
  // one tagged partial per (o, column block, s, column); ticket per (o, cb)
  const long long cb = blockIdx.x, ncb = gridDim.x;
  unsigned long long *grp = sc.words + (o * ncb + cb) * (long long)S * CW * W;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int cc = threadIdx.x + k * kBlock;
    if (cc < CW) put_tagged(grp + ((long long)s * CW + cc) * W, acc[k], sc.tag);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned t = __hip_atomic_fetch_add(sc.tickets + o * ncb + cb, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    is_last = (t == (unsigned)(S - 1));
  }
  __syncthreads();
  if (!is_last) return;
#pragma unroll
  for (int k = 0; k < KC; ++k) {
    const int cc = threadIdx.x + k * kBlock;
    if (cc >= CW) continue;
    const A tot = combine_tagged<R>(grp + (long long)cc * W, (long long)CW * W, S, sc);
    if (c0 + cc < inner) store(o * inner + c0 + cc, tot);
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(sc.tickets + o * ncb + cb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int OP, typename T, typename To>
__global__ __launch_bounds__(kBlock) void k_reduce_cols_vec(const T *__restrict__ x,
                                                           To *__restrict__ out, long long len,
                                                           long long inner, int S,
                                                           ReduceScratch sc) {
  typedef Red<OP, T> R;
  cols_vec_body<R, T>(
      x, len, inner, S, sc, [](T q, long long) { return R::map(q); },
      [&](long long i, const typename R::A &a) { out[i] = finalize<OP, T, To>(a, len); });
}

// Whether a strided reduction can take the column-vector kernel.
template <typename T> bool cols_vec_ok(long long inner, const void *x) {
  if (sizeof(T) < 2) return false;  // one-byte types keep the column-per-thread kernels
  return inner % col_vec<T>() == 0 && ((uintptr_t)x & 15) == 0;
}

// ------------------------------------------------------------ launch
// Strided layouts: split the reduced axis so that the launch has about
// `target` workgroups, each reading at least 64 rows.  Measured on 16384^2
// float32 over axis 0 (the splits' partials combined in batched loads):
// the column-vector sum runs best with one workgroup per CU (256: 6.2 TB/s;
// 128: 5.3, 512: 5.8, 1024: 5.4, 2048: 5.3), the column-per-thread
// kernels with 1024 (argmax 4.76 TB/s; 512: 3.2, 2048: 4.45).
#ifndef MMP_COL_TARGET_BLOCKS
#define MMP_COL_TARGET_BLOCKS 1024
#endif
constexpr long long kColVecTargetBlocks = 256;
constexpr long long kColTargetBlocks = MMP_COL_TARGET_BLOCKS;
int col_splits(long long col_blocks, long long len, long long target) {
  long long want = (target + col_blocks - 1) / col_blocks;
  long long maxs = len / 64 > 0 ? len / 64 : 1;
  long long s = want < maxs ? want : maxs;
  if (s < 1) s = 1;
  if (s > 1024) s = 1024;
  return (int)s;
}

int choose_splits(long long rows, long long len) {
  long long want = (kTargetBlocks + rows - 1) / rows;
  // A single row (axis=None) splits into kTargetBlocksOneRow workgroups:
  // two per CU.  Its last-arrival combine runs alone at the end of the
  // kernel, so fewer partials shorten that tail; measured on 16384^2
  // float32, sum / argmax over everything: 1024 splits 6.53 / 6.23 TB/s,
  // 768: 6.12 / 5.74, 640: 5.93 / 5.49, 512: 7.03 / 6.78, 384: 5.89 / 6.05,
  // 256: 7.04 / 4.79 (the same data by rows, axis=1: 6.9 TB/s).
  if (rows == 1) want = kTargetBlocksOneRow;
  long long maxs = (len + kMinPerBlock - 1) / kMinPerBlock;
  long long s = want < maxs ? want : maxs;
  if (s < 1) s = 1;
  if (s > kMaxSplits) s = kMaxSplits;
  return (int)s;
}

// Scratch for `count` tagged partials of type A plus `nticket` tickets.
template <typename A>
int reduce_scratch(long long count, long long nticket, ReduceScratch *sc) {
  int st = MMP_OK;
  sc->words = (unsigned long long *)mmpi::scratch(mmpi::SCRATCH_REDUCE_PARTIALS,
                                                  8ull * words_of<A>() * count, &st);
  if (st) return st;
  sc->tickets = (unsigned *)mmpi::scratch(mmpi::SCRATCH_REDUCE_TICKETS, 4ull * nticket, &st);
  if (st) return st;
  sc->timeout = mmpi::wait_flags() + 1;
  sc->tag = mmpi::next_generation();
  const mmpi::WaitParams wp = mmpi::wait_params();
  sc->read_tag = (sc->tag + wp.tag_offset) & 0x3fffffffu;
  sc->spin_limit = wp.spin_limit;
  return MMP_OK;
}

// Scratch of the allocation-free entry point (mmp_reduce_noalloc): the
// static array `scratch` below, tickets first, then tagged partial words.
constexpr size_t kNoAllocBytes = 4u << 20;
constexpr size_t kNoAllocTicketBytes = 16u << 10;

// Splits of a strided reduction for mmp_reduce_noalloc: the library's
// choice, lowered until the partials fit the static scratch (S = 1 needs
// none).
template <typename A> int noalloc_col_splits(int S, long long groups, int cols_per_group) {
  const long long per_split = groups * (long long)cols_per_group * words_of<A>() * 8;
  const long long fit = (long long)(kNoAllocBytes - kNoAllocTicketBytes) / per_split;
  if (S > fit) S = fit > 1 ? (int)fit : 1;
  return S;
}

template <typename A>
int noalloc_scratch(long long count, long long nticket, ReduceScratch *sc);

template <int OP, typename T, typename To>
int launch_reduce(long long outer, long long len, long long inner, const void *x, void *out,
                  bool noalloc) {
  typedef typename Red<OP, T>::A A;
  ReduceScratch sc{};
  if (inner == 1) {
    const int S = choose_splits(outer, len);
    if (S > 1) {
      if (int st = noalloc ? noalloc_scratch<A>(outer * S, outer, &sc)
                           : reduce_scratch<A>(outer * S, outer, &sc))
        return st;
    }
    const long long grid = outer * S;
    if (grid > 0x7fffffffLL) return mmpi::fail(MMP_E_ARG, "reduction grid too large");
    hipLaunchKernelGGL((k_reduce_rows<OP, T, To>), dim3((unsigned)grid), dim3(kBlock), 0,
                       mmpi::stream(), (const T *)x, (To *)out, len, S, sc);
    return mmpi::check_launch("mmp_reduce(rows)");
  }
  if (outer > 65535) return mmpi::fail(MMP_E_ARG, "strided reduction: outer extent %lld > 65535", outer);
  const bool vec = cols_vec_ok<T>(inner, x);
  const int cw = vec ? col_width<T>() : kBlock;  // columns per workgroup
  const long long ncb = mmpi::ceil_div(inner, cw);
  int S = col_splits(outer * ncb, len, vec ? kColVecTargetBlocks : kColTargetBlocks);
  if (noalloc) S = noalloc_col_splits<A>(S, outer * ncb, cw);
  if (S > 1) {
    if (int st = noalloc ? noalloc_scratch<A>(outer * ncb * S * cw, outer * ncb, &sc)
                         : reduce_scratch<A>(outer * ncb * S * cw, outer * ncb, &sc))
      return st;
  }
  const dim3 grid((unsigned)ncb, (unsigned)outer, (unsigned)S);
  if constexpr (sizeof(T) >= 2) {
    if (vec) {
      hipLaunchKernelGGL((k_reduce_cols_vec<OP, T, To>), grid, dim3(kBlock), 0, mmpi::stream(),
                         (const T *)x, (To *)out, len, inner, S, sc);
      return mmpi::check_launch("mmp_reduce(cols)");
    }
  }
  hipLaunchKernelGGL((k_reduce_cols<OP, T, To>), grid, dim3(kBlock), 0, mmpi::stream(),
                     (const T *)x, (To *)out, len, inner, S, sc);
  return mmpi::check_launch("mmp_reduce(cols)");
}

template <int OP, typename T>
int launch_argreduce(long long outer, long long len, long long inner, const void *x, long long *out) {
  typedef typename Arg<OP, T>::A A;
  ReduceScratch sc{};
  if (inner == 1) {
    const int S = choose_splits(outer, len);
    if (S > 1) {
      if (int st = reduce_scratch<A>(outer * S, outer, &sc)) return st;
    }
    const long long grid = outer * S;
    if (grid > 0x7fffffffLL) return mmpi::fail(MMP_E_ARG, "reduction grid too large");
    hipLaunchKernelGGL((k_argreduce_rows<OP, T>), dim3((unsigned)grid), dim3(kBlock), 0,
                       mmpi::stream(), (const T *)x, out, len, S, sc);
    return mmpi::check_launch("mmp_argreduce(rows)");
  }
  if (outer > 65535) return mmpi::fail(MMP_E_ARG, "strided argreduce: outer extent %lld > 65535", outer);
  const long long ncb = mmpi::ceil_div(inner, kBlock);
  const int S = col_splits(outer * ncb, len, kColTargetBlocks);
  if (S > 1) {
    if (int st = reduce_scratch<A>(outer * ncb * S * kBlock, outer * ncb, &sc)) return st;
  }
  hipLaunchKernelGGL((k_argreduce_cols<OP, T>), dim3((unsigned)ncb, (unsigned)outer, (unsigned)S),
                     dim3(kBlock), 0, mmpi::stream(), (const T *)x, out, len, inner, S, sc);
  return mmpi::check_launch("mmp_argreduce(cols)");
}

// Output dtypes NumPy's rules produce: max/min keep the dtype; sums and
// products of floats give a float (float64 partials may round to float32 /
// float16), of signed ints and bool int64, of unsigned ints uint64; means
// give a float.
template <int OP, typename T, typename To> constexpr bool out_ok() {
  constexpr bool to_float = mmp_t<To>::is_float;
  if (OP == MMP_R_MAX || OP == MMP_R_MIN || OP == MMP_R_NANMAX || OP == MMP_R_NANMIN)
    return __is_same(T, To);
  if (OP == MMP_R_MEAN || OP == MMP_R_NANMEAN) return to_float;
  if (mmp_t<T>::is_float) return to_float;
  if (mmp_t<T>::is_signed || mmp_t<T>::is_bool) return __is_same(To, mmp_i64);
  return __is_same(To, mmp_u64);
}

template <int OP, typename T, typename To>
int reduce_to(long long outer, long long len, long long inner, const void *x, void *out,
              bool noalloc) {
  if constexpr (!out_ok<OP, T, To>()) {
    return mmpi::fail(MMP_E_UNSUPPORTED, "reduction op %d: unsupported output dtype", OP);
  } else {
    return launch_reduce<OP, T, To>(outer, len, inner, x, out, noalloc);
  }
}

template <int OP, typename T>
int reduce_out(int out_dtype, long long outer, long long len, long long inner, const void *x,
               void *out, bool noalloc) {
  switch (out_dtype) {
    case MMP_F32: return reduce_to<OP, T, float>(outer, len, inner, x, out, noalloc);
    case MMP_F64: return reduce_to<OP, T, double>(outer, len, inner, x, out, noalloc);
    case MMP_F16: return reduce_to<OP, T, mmp_half>(outer, len, inner, x, out, noalloc);
    case MMP_I64: return reduce_to<OP, T, mmp_i64>(outer, len, inner, x, out, noalloc);
    case MMP_U64: return reduce_to<OP, T, mmp_u64>(outer, len, inner, x, out, noalloc);
    case MMP_I32: return reduce_to<OP, T, mmp_i32>(outer, len, inner, x, out, noalloc);
    case MMP_U32: return reduce_to<OP, T, mmp_u32>(outer, len, inner, x, out, noalloc);
    case MMP_I16: return reduce_to<OP, T, mmp_i16>(outer, len, inner, x, out, noalloc);
    case MMP_U16: return reduce_to<OP, T, mmp_u16>(outer, len, inner, x, out, noalloc);
    case MMP_BOOL: return reduce_to<OP, T, bool>(outer, len, inner, x, out, noalloc);
    default: return mmpi::fail(MMP_E_UNSUPPORTED, "reduction output dtype %d", out_dtype);
  }
}

template <typename T>
int reduce_op(int op, int out_dtype, int64_t outer, int64_t len, int64_t inner, const void *x,
              void *out, bool noalloc) {
  switch (op) {
    case MMP_R_SUM: return reduce_out<MMP_R_SUM, T>(out_dtype, outer, len, inner, x, out, noalloc);
    case MMP_R_PROD: return reduce_out<MMP_R_PROD, T>(out_dtype, outer, len, inner, x, out, noalloc);
    case MMP_R_MAX: return reduce_out<MMP_R_MAX, T>(out_dtype, outer, len, inner, x, out, noalloc);
    case MMP_R_MIN: return reduce_out<MMP_R_MIN, T>(out_dtype, outer, len, inner, x, out, noalloc);
    case MMP_R_MEAN: return reduce_out<MMP_R_MEAN, T>(out_dtype, outer, len, inner, x, out, noalloc);
    case MMP_R_NANSUM:
      return reduce_out<MMP_R_NANSUM, T>(out_dtype, outer, len, inner, x, out, noalloc);
    case MMP_R_NANPROD:
      return reduce_out<MMP_R_NANPROD, T>(out_dtype, outer, len, inner, x, out, noalloc);
    case MMP_R_NANMAX:
      return reduce_out<MMP_R_NANMAX, T>(out_dtype, outer, len, inner, x, out, noalloc);
    case MMP_R_NANMIN:
      return reduce_out<MMP_R_NANMIN, T>(out_dtype, outer, len, inner, x, out, noalloc);
    case MMP_R_NANMEAN:
      return reduce_out<MMP_R_NANMEAN, T>(out_dtype, outer, len, inner, x, out, noalloc);
    default: return mmpi::fail(MMP_E_ARG, "unknown reduction op %d", op);
  }
}

int reduce_dispatch(int op, int dtype, int out_dtype, int64_t outer, int64_t len, int64_t inner,
                    const void *x, void *out, bool noalloc) {
  MMP_DISPATCH_ALL(dtype, { return reduce_op<T>(op, out_dtype, outer, len, inner, x, out, noalloc); })
}

int check_view(long long outer, long long len, long long inner, const void *x, const void *out) {
  if (outer < 0 || len < 0 || inner < 0) return mmpi::fail(MMP_E_ARG, "negative extent");
  if (len == 0) return mmpi::fail(MMP_E_ARG, "reduction over an empty axis");
  if (outer * inner > 0 && (!x || !out)) return mmpi::fail(MMP_E_ARG, "null pointer");
  return MMP_OK;
}

__global__ void k_zero_words(unsigned long long *p, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    p[i] = 0ull;
}

}  // namespace

// The allocation-free entry point's scratch: one copy per device (each GPU
// the library runs on holds it until the process ends).  In host code the
// name is only a stand-in for the symbol; kernels get the device address
// that hipGetSymbolAddress returned for the current device.
static __device__ __align__(256) unsigned long long scratch[kNoAllocBytes / 8];

namespace {
constexpr int kMaxDevices = 64;
void *g_noalloc_ptr[kMaxDevices] = {};

template <typename A>
int noalloc_scratch(long long count, long long nticket, ReduceScratch *sc) {
  const int dev = mmpi::device_id();
  void *base = (dev >= 0 && dev < kMaxDevices) ? g_noalloc_ptr[dev] : nullptr;
  if (!base) return mmpi::fail(MMP_E_ARG, "mmp_reduce_noalloc: scratch not set up on device %d", dev);
  const unsigned long long words_bytes = 8ull * words_of<A>() * (unsigned long long)count;
  if ((unsigned long long)nticket * 4ull > kNoAllocTicketBytes ||
      words_bytes > kNoAllocBytes - kNoAllocTicketBytes)
    return mmpi::fail(MMP_E_ARG,
                      "mmp_reduce_noalloc: this reduction needs %llu bytes of partials and %lld "
                      "tickets; the static scratch holds %zu bytes and %zu tickets",
                      words_bytes, nticket, kNoAllocBytes - kNoAllocTicketBytes,
                      kNoAllocTicketBytes / 4);
  sc->tickets = static_cast<unsigned *>(base);
  sc->words = reinterpret_cast<unsigned long long *>(static_cast<char *>(base) + kNoAllocTicketBytes);
  // Zero the partial words this call uses, on the stream, before its
  // kernels.  A captured call replays with the tag fixed at capture time;
  // without the clear the combining workgroup could accept a word of the
  // previous replay that carries the same tag before this replay's store
  // lands.  After it, only this launch can write a word with its tag (tags
  // are never 0).  A kernel rather than hipMemsetAsync, so that a capture
  // records a kernel node.
  const long long nwords = (long long)(words_bytes / 8);
  if (nwords > 0) {
    const unsigned zblocks = (unsigned)std::min<long long>(256, (nwords + 255) / 256);
    hipLaunchKernelGGL(k_zero_words, dim3(zblocks), dim3(256), 0, mmpi::stream(), sc->words,
                       nwords);
    if (int st = mmpi::check_launch("mmp_reduce_noalloc: partial clear")) return st;
  }
  sc->timeout = mmpi::wait_flags() + 1;
  sc->tag = mmpi::next_generation();
  const mmpi::WaitParams wp = mmpi::wait_params();
  sc->read_tag = (sc->tag + wp.tag_offset) & 0x3fffffffu;
  sc->spin_limit = wp.spin_limit;
  return MMP_OK;
}
}  // namespace

namespace mmpi {
// Called by mmp_init with `device` current and the library stream created:
// resolve this device's copy of `scratch` and clear it (tickets must start
// at zero; every kernel leaves the tickets it used at zero).
int noalloc_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return fail(MMP_E_ARG, "device %d out of range", device);
  void *p = nullptr;
  if (int st = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch)), "hipGetSymbolAddress(scratch)"))
    return st;
  hipLaunchKernelGGL(k_zero_words, dim3(256), dim3(256), 0, stream(),
                     static_cast<unsigned long long *>(p), (long long)(kNoAllocBytes / 8));
  if (int st = check_hip(hipGetLastError(), "noalloc scratch clear")) return st;
  g_noalloc_ptr[device] = p;
  return MMP_OK;
}
}  // namespace mmpi

extern "C" int mmp_reduce(int op, int dtype, int out_dtype, int64_t outer, int64_t len,
                          int64_t inner, const void *x, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (int st = check_view(outer, len, inner, x, out)) return st;
  if (outer * inner == 0) return MMP_OK;
  std::lock_guard<std::mutex> lk(mmpi::launch_mutex());
  return reduce_dispatch(op, dtype, out_dtype, outer, len, inner, x, out, false);
}

extern "C" int mmp_reduce_noalloc(int op, int dtype, int out_dtype, int64_t outer, int64_t len,
                                  int64_t inner, const void *x, void *out) {
  // Never initialises the library itself: initialisation allocates.
  if (!mmpi::initialized())
    return mmpi::fail(MMP_E_ARG, "mmp_reduce_noalloc: call mmp_init first");
  if (int st = check_view(outer, len, inner, x, out)) return st;
  if (outer * inner == 0) return MMP_OK;
  std::lock_guard<std::mutex> lk(mmpi::launch_mutex());
  return reduce_dispatch(op, dtype, out_dtype, outer, len, inner, x, out, true);
}

extern "C" int mmp_argreduce(int op, int dtype, int64_t outer, int64_t len, int64_t inner,
                             const void *x, int64_t *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (int st = check_view(outer, len, inner, x, out)) return st;
  if (outer * inner == 0) return MMP_OK;
  std::lock_guard<std::mutex> lk(mmpi::launch_mutex());
  MMP_DISPATCH_ALL(dtype, {
    if (op == MMP_R_ARGMAX)
      return launch_argreduce<MMP_R_ARGMAX, T>(outer, len, inner, x, (long long *)out);
    if (op == MMP_R_ARGMIN)
      return launch_argreduce<MMP_R_ARGMIN, T>(outer, len, inner, x, (long long *)out);
    if (op == MMP_R_NANARGMAX)
      return launch_argreduce<MMP_R_NANARGMAX, T>(outer, len, inner, x, (long long *)out);
    if (op == MMP_R_NANARGMIN)
      return launch_argreduce<MMP_R_NANARGMIN, T>(outer, len, inner, x, (long long *)out);
    return mmpi::fail(MMP_E_ARG, "unknown arg-reduction op %d", op);
  })
}
