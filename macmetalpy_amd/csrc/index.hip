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
//  * mmp_mask_tile_counts / mmp_mask_positions do the same from the mask
//    bytes themselves, by tiles of 4096 elements: a tile's selected count,
//    the inclusive count over tiles (the library scan), then each tile
//    writes its positions from its tile's start offset and an in-tile
//    exclusive count.  The mask is read twice (1 byte per element each) and
//    nothing per element is written besides the positions.
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

// Mask compaction by tiles of kMaskTile elements; thread t of a tile owns
// elements 16 t .. 16 t + 15 (one 16-byte load when the tile is whole and
// aligned).  Any nonzero byte selects.
constexpr int kMaskItems = 16;
constexpr int kMaskTile = kBlock * kMaskItems;

// This thread's 16 selection flags as a bit mask.
__device__ __forceinline__ unsigned mask_bits(const unsigned char *__restrict__ m, long long n,
                                              long long t0) {
  const long long i0 = t0 + (long long)threadIdx.x * kMaskItems;
  unsigned bits = 0;
  if (i0 + kMaskItems <= n && (((uintptr_t)(m + i0)) & 15u) == 0) {
    const u32x4 v = *reinterpret_cast<const u32x4 *>(m + i0);
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
      for (int b = 0; b < 4; ++b) bits |= (((v[w] >> (8 * b)) & 0xffu) != 0u ? 1u : 0u) << (4 * w + b);
  } else {
    for (int k = 0; k < kMaskItems; ++k)
      if (i0 + k < n && m[i0 + k] != 0) bits |= 1u << k;
  }
  return bits;
}

// Workgroup exclusive sum of one value per thread (wave shuffles, then the
// wave totals through LDS); *total = the workgroup's sum.
__device__ __forceinline__ unsigned block_excl_sum(unsigned v, unsigned *total) {
  __shared__ unsigned wsum[kBlock / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const unsigned o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  unsigned pre = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kBlock / 64; ++w) {
    if (w < wave) pre += wsum[w];
    tot += wsum[w];
  }
  *total = tot;
  return pre + inc - v;
}

__global__ __launch_bounds__(kBlock) void k_mask_counts(const unsigned char *__restrict__ m,
                                                        long long n, unsigned *__restrict__ counts) {
  const long long t0 = (long long)blockIdx.x * kMaskTile;
  unsigned total;
  block_excl_sum((unsigned)__builtin_popcount(mask_bits(m, n, t0)), &total);
  if (threadIdx.x == 0) counts[blockIdx.x] = total;
}

__global__ __launch_bounds__(kBlock) void k_mask_positions(const unsigned char *__restrict__ m,
                                                           long long n,
                                                           const unsigned long long *__restrict__ incl,
                                                           long long *__restrict__ out) {
  const long long t0 = (long long)blockIdx.x * kMaskTile;
  unsigned bits = mask_bits(m, n, t0);
  unsigned total;
  const unsigned ex = block_excl_sum((unsigned)__builtin_popcount(bits), &total);
  // the tile's first output slot: inclusive count through this tile minus its own
  long long o = (long long)incl[blockIdx.x] - (long long)total + ex;
  const long long i0 = t0 + (long long)threadIdx.x * kMaskItems;
  while (bits) {
    const int k = __builtin_ctz(bits);
    out[o++] = i0 + k;
    bits &= bits - 1;
  }
}

// The selected elements themselves (W bytes each) of a contiguous source
// of the mask's shape, in order: a[mask] without the positions.  The tile's
// source is read coalesced into LDS, each thread takes its 16 elements from
// there, writes the selected ones back packed (LDS slot = in-tile rank), and
// the packed run leaves with coalesced stores.
template <typename W>
__global__ __launch_bounds__(kBlock) void k_mask_compact(const unsigned char *__restrict__ m,
                                                         long long n,
                                                         const unsigned long long *__restrict__ incl,
                                                         const W *__restrict__ src, W *__restrict__ out) {
  __shared__ __attribute__((aligned(16))) W buf[kMaskTile];
  const long long t0 = (long long)blockIdx.x * kMaskTile;
  const int tn = n - t0 < kMaskTile ? (int)(n - t0) : kMaskTile;  // elements in this tile
  const W *s = src + t0;
  constexpr int VW = 16 / (int)sizeof(W);
  if (tn == kMaskTile && (((uintptr_t)s) & 15u) == 0) {
    for (int v = threadIdx.x; v < kMaskTile / VW; v += kBlock)
      *reinterpret_cast<u32x4 *>(&buf[v * VW]) = *reinterpret_cast<const u32x4 *>(s + v * VW);
  } else {
    for (int i = threadIdx.x; i < tn; i += kBlock) buf[i] = s[i];
  }
  unsigned bits = mask_bits(m, n, t0);
  unsigned total;
  const unsigned ex = block_excl_sum((unsigned)__builtin_popcount(bits), &total);  // syncs
  W mine[kMaskItems];
#pragma unroll
  for (int k = 0; k < kMaskItems; ++k) mine[k] = buf[threadIdx.x * kMaskItems + k];
  __syncthreads();
  unsigned r = ex;
#pragma unroll
  for (int k = 0; k < kMaskItems; ++k)
    if ((bits >> k) & 1u) buf[r++] = mine[k];
  __syncthreads();
  const long long o = (long long)incl[blockIdx.x] - (long long)total;
  for (unsigned j = threadIdx.x; j < total; j += kBlock) out[o + j] = buf[j];
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

extern "C" int mmp_mask_tile_counts(int64_t n, const void *mask, uint64_t *tile_incl) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0) return mmpi::fail(MMP_E_ARG, "mmp_mask_tile_counts: negative extent");
  if (n == 0) return MMP_OK;
  if (!mask || !tile_incl) return mmpi::fail(MMP_E_ARG, "mmp_mask_tile_counts: null pointer");
  const long long tiles = mmpi::ceil_div(n, kMaskTile);
  if (tiles > 0x7fffffffLL) return mmpi::fail(MMP_E_ARG, "mmp_mask_tile_counts: mask too large");
  void *counts = nullptr;
  if (int st = mmp_alloc((size_t)tiles * sizeof(unsigned), &counts)) return st;
  hipLaunchKernelGGL(k_mask_counts, dim3((unsigned)tiles), dim3(kBlock), 0, mmpi::stream(),
                     (const unsigned char *)mask, (long long)n, (unsigned *)counts);
  int st = mmpi::check_launch("mmp_mask_tile_counts");
  if (!st) st = mmp_scan(MMP_S_CUMSUM, MMP_U32, MMP_U64, 1, tiles, 1, counts, tile_incl);
  (void)mmp_free(counts);  // stream-ordered: reused only by later work
  return st;
}

extern "C" int mmp_mask_positions(int64_t n, const void *mask, const uint64_t *tile_incl,
                                  int64_t *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0) return mmpi::fail(MMP_E_ARG, "mmp_mask_positions: negative extent");
  if (n == 0) return MMP_OK;
  if (!mask || !tile_incl || !out) return mmpi::fail(MMP_E_ARG, "mmp_mask_positions: null pointer");
  const long long tiles = mmpi::ceil_div(n, kMaskTile);
  if (tiles > 0x7fffffffLL) return mmpi::fail(MMP_E_ARG, "mmp_mask_positions: mask too large");
  hipLaunchKernelGGL(k_mask_positions, dim3((unsigned)tiles), dim3(kBlock), 0, mmpi::stream(),
                     (const unsigned char *)mask, (long long)n, (const unsigned long long *)tile_incl,
                     (long long *)out);
  return mmpi::check_launch("mmp_mask_positions");
}

extern "C" int mmp_mask_compact(int word, int64_t n, const void *mask, const uint64_t *tile_incl,
                                const void *src, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0) return mmpi::fail(MMP_E_ARG, "mmp_mask_compact: negative extent");
  if (n == 0) return MMP_OK;
  if (!mask || !tile_incl || !src || !out) return mmpi::fail(MMP_E_ARG, "mmp_mask_compact: null pointer");
  const long long tiles = mmpi::ceil_div(n, kMaskTile);
  if (tiles > 0x7fffffffLL) return mmpi::fail(MMP_E_ARG, "mmp_mask_compact: mask too large");
  const dim3 grid((unsigned)tiles);
  const auto *m = (const unsigned char *)mask;
  const auto *ti = (const unsigned long long *)tile_incl;
  switch (word) {
    case 1: hipLaunchKernelGGL((k_mask_compact<unsigned char>), grid, dim3(kBlock), 0, mmpi::stream(),
                               m, (long long)n, ti, (const unsigned char *)src, (unsigned char *)out); break;
    case 2: hipLaunchKernelGGL((k_mask_compact<unsigned short>), grid, dim3(kBlock), 0, mmpi::stream(),
                               m, (long long)n, ti, (const unsigned short *)src, (unsigned short *)out); break;
    case 4: hipLaunchKernelGGL((k_mask_compact<unsigned>), grid, dim3(kBlock), 0, mmpi::stream(),
                               m, (long long)n, ti, (const unsigned *)src, (unsigned *)out); break;
    case 8: hipLaunchKernelGGL((k_mask_compact<unsigned long long>), grid, dim3(kBlock), 0, mmpi::stream(),
                               m, (long long)n, ti, (const unsigned long long *)src, (unsigned long long *)out); break;
    default: return mmpi::fail(MMP_E_ARG, "mmp_mask_compact: element size %d not 1, 2, 4 or 8", word);
  }
  return mmpi::check_launch("mmp_mask_compact");
}
