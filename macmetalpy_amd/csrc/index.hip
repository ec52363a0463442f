// index.hip -- gathers, scatters and compaction for advanced indexing.
//
// Replaces the reference's host paths for integer-array and boolean-mask
// indexing (ndarray.__getitem__ / __setitem__ fall back to NumPy,
// ndarray.py:874-891, 943-957) and its NumPy-based indexing routines
// (indexing.py:24-110 take / put, 179-249 putmask / place / compress /
// extract, 370-391 nonzero / flatnonzero / argwhere).
//
//  * mmp_gather / mmp_scatter move "rows" of row_words words of W bytes:
//    row i of the gathered array is the row starting at word offset
//    off[i] * unit of the source buffer (unit = words per offset step).
//    The host builds the offsets with NumPy's indexing rules and folds
//    trailing contiguous dimensions into the rows, so a[idx] of a 2-D
//    array moves whole rows.  One thread per word, grid-stride; offsets
//    are checked against the buffer, so no access leaves it.
//  * mmp_nonzero turns the inclusive int64 count of a mask (its cumsum)
//    into the positions of the nonzero elements: element i is selected
//    where incl[i] != incl[i - 1], and lands at incl[i] - 1.
#include "mmp_ops.h"
#include "mmp_internal.h"

namespace {

constexpr int kBlock = 256;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

inline unsigned grid_for(long long work) {
  const long long b = mmpi::ceil_div(work, kBlock);
  return (unsigned)(b < (1ll << 20) ? (b > 0 ? b : 1) : (1ll << 20));
}

// Word w of the output: row i = w / wpr, word c = w % wpr (32-bit division
// when the extents allow it, the common case).
template <bool SMALL>
__device__ __forceinline__ void split(long long w, long long wpr, long long &i, long long &c) {
  if constexpr (SMALL) {
    const unsigned q = (unsigned)w / (unsigned)wpr;
    i = q;
    c = (long long)((unsigned)w - q * (unsigned)wpr);
  } else {
    i = w / wpr;
    c = w - i * wpr;
  }
}

// wrap > 0: the offsets are row indices in [-wrap, wrap) (negatives count
// from the end); any other index reads nothing and sets *flag.
template <typename W, bool SMALL>
__global__ __launch_bounds__(kBlock) void k_gather(const W *__restrict__ src, long long src_words,
                                                   const long long *__restrict__ off, long long unit,
                                                   long long wrap, unsigned *__restrict__ flag,
                                                   long long n, long long wpr, W *__restrict__ out) {
  const long long total = n * wpr;
  for (long long w = (long long)blockIdx.x * kBlock + threadIdx.x; w < total;
       w += (long long)gridDim.x * kBlock) {
    long long i, c;
    split<SMALL>(w, wpr, i, c);
    long long o = off[i];
    if (wrap > 0) {
      if (o < 0) o += wrap;
      if (o < 0 || o >= wrap) {
        if (flag) __hip_atomic_store(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        out[w] = W{};
        continue;
      }
    }
    const long long s = o * unit + c;
    out[w] = (s >= 0 && s < src_words) ? src[s] : W{};
  }
}

template <typename W, bool SMALL>
__global__ __launch_bounds__(kBlock) void k_scatter(W *__restrict__ dst, long long dst_words,
                                                    const long long *__restrict__ off, long long unit,
                                                    long long n, long long wpr,
                                                    const W *__restrict__ src, long long src_rows) {
  const long long total = n * wpr;
  for (long long w = (long long)blockIdx.x * kBlock + threadIdx.x; w < total;
       w += (long long)gridDim.x * kBlock) {
    long long i, c;
    split<SMALL>(w, wpr, i, c);
    const long long d = off[i] * unit + c;
    const long long r = src_rows == 1 ? 0 : i;  // one source row broadcast to every target
    if (d >= 0 && d < dst_words) dst[d] = src[r * wpr + c];
  }
}

__global__ __launch_bounds__(kBlock) void k_nonzero(const long long *__restrict__ incl, long long n,
                                                    long long count, long long *__restrict__ out) {
  for (long long i = (long long)blockIdx.x * kBlock + threadIdx.x; i < n;
       i += (long long)gridDim.x * kBlock) {
    const long long v = incl[i];
    const long long prev = i > 0 ? incl[i - 1] : 0;
    if (v != prev && v >= 1 && v <= count) out[v - 1] = i;
  }
}

template <typename W>
int gather_w(const void *src, long long src_bytes, const long long *off, long long unit,
             long long wrap, unsigned *flag, long long n, long long wpr, void *out) {
  const long long total = n * wpr;
  const bool small = total < (1ll << 31) && wpr < (1ll << 31);
  const unsigned grid = grid_for(total);
  const long long words = src_bytes / (long long)sizeof(W);
  if (small)
    hipLaunchKernelGGL((k_gather<W, true>), dim3(grid), dim3(kBlock), 0, mmpi::stream(),
                       (const W *)src, words, off, unit, wrap, flag, n, wpr, (W *)out);
  else
    hipLaunchKernelGGL((k_gather<W, false>), dim3(grid), dim3(kBlock), 0, mmpi::stream(),
                       (const W *)src, words, off, unit, wrap, flag, n, wpr, (W *)out);
  return mmpi::check_launch("mmp_gather");
}

template <typename W>
int scatter_w(void *dst, long long dst_bytes, const long long *off, long long unit, long long n,
              long long wpr, const void *src, long long src_rows) {
  const long long total = n * wpr;
  const bool small = total < (1ll << 31) && wpr < (1ll << 31);
  const unsigned grid = grid_for(total);
  if (small)
    hipLaunchKernelGGL((k_scatter<W, true>), dim3(grid), dim3(kBlock), 0, mmpi::stream(), (W *)dst,
                       dst_bytes / (long long)sizeof(W), off, unit, n, wpr, (const W *)src, src_rows);
  else
    hipLaunchKernelGGL((k_scatter<W, false>), dim3(grid), dim3(kBlock), 0, mmpi::stream(), (W *)dst,
                       dst_bytes / (long long)sizeof(W), off, unit, n, wpr, (const W *)src, src_rows);
  return mmpi::check_launch("mmp_scatter");
}

bool word_ok(int word, const void *a, const void *b) {
  return word == 1 || word == 2 || word == 4 || word == 8 || word == 16
             ? ((uintptr_t)a % word == 0 && (uintptr_t)b % word == 0)
             : false;
}

}  // namespace

extern "C" int mmp_gather(int word, const void *src, int64_t src_bytes, const int64_t *offsets,
                          int64_t unit, int64_t wrap, uint32_t *flag, int64_t n,
                          int64_t row_words, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (src_bytes < 0 || n < 0 || row_words < 0 || unit < 0 || wrap < 0)
    return mmpi::fail(MMP_E_ARG, "mmp_gather: negative extent");
  if (n == 0 || row_words == 0) return MMP_OK;
  if (!offsets || !out || !src) return mmpi::fail(MMP_E_ARG, "mmp_gather: null pointer");
  if (!word_ok(word, src, out)) return mmpi::fail(MMP_E_ARG, "mmp_gather: word size %d / alignment", word);
  const long long *o = (const long long *)offsets;
  switch (word) {
    case 1: return gather_w<unsigned char>(src, src_bytes, o, unit, wrap, flag, n, row_words, out);
    case 2: return gather_w<unsigned short>(src, src_bytes, o, unit, wrap, flag, n, row_words, out);
    case 4: return gather_w<unsigned>(src, src_bytes, o, unit, wrap, flag, n, row_words, out);
    case 8: return gather_w<unsigned long long>(src, src_bytes, o, unit, wrap, flag, n, row_words, out);
    default: return gather_w<u32x4>(src, src_bytes, o, unit, wrap, flag, n, row_words, out);
  }
}

extern "C" int mmp_scatter(int word, void *dst, int64_t dst_bytes, const int64_t *offsets,
                           int64_t unit, int64_t n, int64_t row_words, const void *src,
                           int64_t src_rows) {
  if (int st = mmpi::ensure_init()) return st;
  if (dst_bytes < 0 || n < 0 || row_words < 0 || unit < 0 || src_rows < 1)
    return mmpi::fail(MMP_E_ARG, "mmp_scatter: negative extent");
  if (src_rows != 1 && src_rows != n) return mmpi::fail(MMP_E_ARG, "mmp_scatter: src_rows %lld", (long long)src_rows);
  if (n == 0 || row_words == 0) return MMP_OK;
  if (!offsets || !dst || !src) return mmpi::fail(MMP_E_ARG, "mmp_scatter: null pointer");
  if (!word_ok(word, dst, src)) return mmpi::fail(MMP_E_ARG, "mmp_scatter: word size %d / alignment", word);
  const long long *o = (const long long *)offsets;
  switch (word) {
    case 1: return scatter_w<unsigned char>(dst, dst_bytes, o, unit, n, row_words, src, src_rows);
    case 2: return scatter_w<unsigned short>(dst, dst_bytes, o, unit, n, row_words, src, src_rows);
    case 4: return scatter_w<unsigned>(dst, dst_bytes, o, unit, n, row_words, src, src_rows);
    case 8: return scatter_w<unsigned long long>(dst, dst_bytes, o, unit, n, row_words, src, src_rows);
    default: return scatter_w<u32x4>(dst, dst_bytes, o, unit, n, row_words, src, src_rows);
  }
}

extern "C" int mmp_nonzero(int64_t n, const int64_t *incl, int64_t count, int64_t *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0 || count < 0) return mmpi::fail(MMP_E_ARG, "mmp_nonzero: negative extent");
  if (n == 0 || count == 0) return MMP_OK;
  if (!incl || !out) return mmpi::fail(MMP_E_ARG, "mmp_nonzero: null pointer");
  hipLaunchKernelGGL(k_nonzero, dim3(grid_for(n)), dim3(kBlock), 0, mmpi::stream(),
                     (const long long *)incl, (long long)n, (long long)count, (long long *)out);
  return mmpi::check_launch("mmp_nonzero");
}
