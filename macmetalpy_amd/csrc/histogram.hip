// histogram.hip -- integer counts for bincount and histogram.
//
// Replaces the reference's NumPy host calls behind bincount / histogram
// (math_ext.py, nan_ops.py's histogram family).  Counts are exact integers,
// so the order of the atomic additions does not change any result:
//  * mmp_bincount: counts[v] for integer values v in [0, nbins); other
//    values are not counted (callers check the range first).
//  * mmp_histogram: counts[b] = #{x : edges[b] <= x < edges[b+1]}, the last
//    bin closed on the right, compared in double (x converted, edges given
//    as double); NaN and values outside [edges[0], edges[-1]] are not
//    counted.  The bin is the last edge <= x (binary search), which is
//    NumPy's searchsorted rule for its bins.
// Each workgroup counts its grid-stride share into 32-bit LDS counters
// (at most 2^32 elements per workgroup) and adds them to the 64-bit totals
// with one atomic per non-empty bin; bin counts beyond the LDS budget go
// straight to global atomics.  The totals are zeroed by a fill kernel in
// the same stream first.
#include <type_traits>

#include "mmp_ops.h"
#include "mmp_internal.h"

namespace {

constexpr int kBlock = 256;
constexpr int kMaxGrid = 1024;
constexpr int kLdsBins = 12288;    // 48 KiB of 32-bit counters
constexpr int kLdsEdges = 4097;    // 32 KiB of edges + 16 KiB of counters

typedef unsigned long long u64;

__global__ __launch_bounds__(kBlock) void k_zero_counts(u64 *__restrict__ c, long long n) {
  for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n; i += (long long)gridDim.x * kBlock)
    c[i] = 0;
}

template <typename T>
__device__ __forceinline__ long long as_index(T v) {
  if constexpr (sizeof(T) == 8 && !std::is_signed<T>::value)
    return v > (T)0x7fffffffffffffffull ? -1ll : (long long)v;
  else
    return (long long)v;
}

template <typename T, bool LDS>
__global__ __launch_bounds__(kBlock) void k_bincount(const T *__restrict__ x, long long n, int nbins,
                                                     u64 *__restrict__ counts) {
  __shared__ unsigned h[LDS ? kLdsBins : 1];
  const int tid = threadIdx.x;
  if constexpr (LDS) {
    for (int b = tid; b < nbins; b += kBlock) h[b] = 0u;
    __syncthreads();
  }
  for (long long i = (long long)blockIdx.x * kBlock + tid; i < n; i += (long long)gridDim.x * kBlock) {
    const long long v = as_index(x[i]);
    if (v >= 0 && v < nbins) {
      if constexpr (LDS)
        atomicAdd(&h[v], 1u);
      else
        atomicAdd(&counts[v], (u64)1);
    }
  }
  if constexpr (LDS) {
    __syncthreads();
    for (int b = tid; b < nbins; b += kBlock) {
      const unsigned c = h[b];
      if (c) atomicAdd(&counts[b], (u64)c);
    }
  }
}

template <typename T, bool LDS>
__global__ __launch_bounds__(kBlock) void k_histogram(const T *__restrict__ x, long long n,
                                                      const double *__restrict__ edges, int ne,
                                                      u64 *__restrict__ counts) {
  __shared__ double e_lds[LDS ? kLdsEdges : 1];
  __shared__ unsigned h[LDS ? kLdsEdges - 1 : 1];
  const int tid = threadIdx.x;
  const double *e = edges;
  if constexpr (LDS) {
    for (int b = tid; b < ne; b += kBlock) e_lds[b] = edges[b];
    for (int b = tid; b < ne - 1; b += kBlock) h[b] = 0u;
    __syncthreads();
    e = e_lds;
  }
  const double lo = e[0], hi = e[ne - 1];
  for (long long i = (long long)blockIdx.x * kBlock + tid; i < n; i += (long long)gridDim.x * kBlock) {
    const double v = (double)x[i];
    if (!(v >= lo && v <= hi)) continue;  // NaN and out-of-range values
    int l = 0, r = ne;                     // first edge > v
    while (l < r) {
      const int mid = (l + r) >> 1;
      if (e[mid] > v) r = mid;
      else l = mid + 1;
    }
    int b = l - 1;
    if (b > ne - 2) b = ne - 2;
    if constexpr (LDS)
      atomicAdd(&h[b], 1u);
    else
      atomicAdd(&counts[b], (u64)1);
  }
  if constexpr (LDS) {
    __syncthreads();
    for (int b = tid; b < ne - 1; b += kBlock) {
      const unsigned c = h[b];
      if (c) atomicAdd(&counts[b], (u64)c);
    }
  }
}

unsigned grid_for(long long n) {
  const long long g = mmpi::ceil_div(n, kBlock);
  return (unsigned)(g < 1 ? 1 : (g > kMaxGrid ? kMaxGrid : g));
}

int zero(u64 *c, long long n) {
  hipLaunchKernelGGL(k_zero_counts, dim3(grid_for(n)), dim3(kBlock), 0, mmpi::stream(), c, n);
  return mmpi::check_launch("histogram counts");
}

template <typename T>
int bincount_t(const void *x, long long n, long long nbins, u64 *counts) {
  const unsigned g = grid_for(n);
  if (nbins <= kLdsBins)
    hipLaunchKernelGGL((k_bincount<T, true>), dim3(g), dim3(kBlock), 0, mmpi::stream(), (const T *)x, n,
                       (int)nbins, counts);
  else
    hipLaunchKernelGGL((k_bincount<T, false>), dim3(g), dim3(kBlock), 0, mmpi::stream(), (const T *)x, n,
                       (int)nbins, counts);
  return mmpi::check_launch("mmp_bincount");
}

template <typename T>
int histogram_t(const void *x, long long n, const double *edges, long long ne, u64 *counts) {
  const unsigned g = grid_for(n);
  if (ne <= kLdsEdges)
    hipLaunchKernelGGL((k_histogram<T, true>), dim3(g), dim3(kBlock), 0, mmpi::stream(), (const T *)x, n,
                       edges, (int)ne, counts);
  else
    hipLaunchKernelGGL((k_histogram<T, false>), dim3(g), dim3(kBlock), 0, mmpi::stream(), (const T *)x, n,
                       edges, (int)ne, counts);
  return mmpi::check_launch("mmp_histogram");
}

}  // namespace

extern "C" int mmp_bincount(int dtype, int64_t n, const void *x, int64_t nbins, int64_t *counts) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0 || nbins < 0 || nbins > 0x7fffffffll)
    return mmpi::fail(MMP_E_ARG, "mmp_bincount: n %lld nbins %lld", (long long)n, (long long)nbins);
  if (nbins == 0) return MMP_OK;
  if (!counts || (n && !x)) return mmpi::fail(MMP_E_ARG, "mmp_bincount: null pointer");
  if (int st = zero((u64 *)counts, nbins)) return st;
  if (n == 0) return MMP_OK;
  u64 *c = (u64 *)counts;
  switch (dtype) {
    case MMP_BOOL: return bincount_t<unsigned char>(x, n, nbins, c);
    case MMP_I16: return bincount_t<short>(x, n, nbins, c);
    case MMP_U16: return bincount_t<unsigned short>(x, n, nbins, c);
    case MMP_I32: return bincount_t<int>(x, n, nbins, c);
    case MMP_U32: return bincount_t<unsigned>(x, n, nbins, c);
    case MMP_I64: return bincount_t<long long>(x, n, nbins, c);
    case MMP_U64: return bincount_t<unsigned long long>(x, n, nbins, c);
    default: return mmpi::fail(MMP_E_UNSUPPORTED, "mmp_bincount: dtype %d (integers only)", dtype);
  }
}

extern "C" int mmp_histogram(int dtype, int64_t n, const void *x, int64_t nedges, const double *edges,
                             int64_t *counts) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0 || nedges < 2 || nedges > 0x7fffffffll)
    return mmpi::fail(MMP_E_ARG, "mmp_histogram: n %lld nedges %lld", (long long)n, (long long)nedges);
  if (!counts || !edges || (n && !x)) return mmpi::fail(MMP_E_ARG, "mmp_histogram: null pointer");
  if (int st = zero((u64 *)counts, nedges - 1)) return st;
  if (n == 0) return MMP_OK;
  u64 *c = (u64 *)counts;
  switch (dtype) {
    case MMP_I16: return histogram_t<short>(x, n, edges, nedges, c);
    case MMP_U16: return histogram_t<unsigned short>(x, n, edges, nedges, c);
    case MMP_I32: return histogram_t<int>(x, n, edges, nedges, c);
    case MMP_U32: return histogram_t<unsigned>(x, n, edges, nedges, c);
    case MMP_F16: return histogram_t<mmp_half>(x, n, edges, nedges, c);
    case MMP_F32: return histogram_t<float>(x, n, edges, nedges, c);
    case MMP_F64: return histogram_t<double>(x, n, edges, nedges, c);
    default: return mmpi::fail(MMP_E_UNSUPPORTED, "mmp_histogram: dtype %d", dtype);
  }
}
