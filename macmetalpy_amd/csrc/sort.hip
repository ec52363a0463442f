// sort.hip -- sort / argsort along the last axis, searchsorted, take.
//
// Replaces the reference's GPU sort, a bitonic network launched from
// Python one compare-exchange pass at a time (sorting.py:59-196: padding
// to a power of two, log2(n)^2 / 2 launches, unstable, int32 indices,
// NaN unordered), and its one-thread binary searchsorted
// (sorting.py:218-263).
//
// Sort: least-significant-digit radix sort with 8-bit digits over
// order-preserving unsigned keys, stable, three launches per digit:
//  * k_radix_hist: one 256-bin histogram per 4096-key tile (LDS atomics
//    into 16 padded sub-histograms), written digit-major:
//    counts[d * tiles + b];
//  * one inclusive scan of the counts (mmp_scan), so that the global
//    offset of digit d in tile b is incl[d * tiles + b] - counts[...];
//  * k_radix_scatter: each wave ranks a contiguous quarter of the tile in
//    rounds of 64 keys: the lanes holding one digit find each other with
//    eight 64-lane ballots and take consecutive ranks after the digit's
//    running count in a wave-private LDS counter (no block barrier per
//    round); the four waves' counts then become per-digit offsets, keys
//    are placed into an LDS staging tile in sorted order and written out
//    from there, so that consecutive threads write consecutive addresses
//    of one digit's run (coalesced).  Waves, rounds and lanes follow input
//    order, which makes every pass stable.
// Rows (the leading axes of an N-D input) are sorted independently: tiles
// never cross a row, and the tile counts are scanned in (row, digit, tile)
// order, so every row's keys land in its own range.  Keys: float bit
// patterns with the sign flipped (positive) or all bits inverted
// (negative); NaN sorts last, as in NumPy.  When an index is carried
// (argsort, stable) keys are canonical -- -0.0 equals +0.0 and all
// NaNs are equal -- and sorted values are gathered from the input by the
// final index, which reproduces np.sort(kind='stable') bit for bit; a
// keys-only 1-D sort keeps every value's bits except the sign of NaNs.
// HBM traffic per digit pass: keys (and 4-byte indices) read twice and
// written once.
#include "mmp_ops.h"
#include "mmp_internal.h"

#include <algorithm>
#include <type_traits>

namespace {

constexpr int kBlock = 256;
constexpr int kIPT = 16;  // 8, 24 and 32 keys per thread measured slower
constexpr int kTile = kBlock * kIPT;
constexpr int kRadix = 256;

template <int B> struct UInt;
template <> struct UInt<2> { typedef unsigned short type; };
template <> struct UInt<4> { typedef unsigned int type; };
template <> struct UInt<8> { typedef unsigned long long type; };

// key type: 16 bits for bool and 16-bit types, else the type's width
template <typename T> struct KeyOf {
  typedef typename UInt<(sizeof(T) < 2 ? 2 : sizeof(T))>::type K;
};

template <typename T, bool CANON>
__device__ __forceinline__ typename KeyOf<T>::K to_key(T v) {
  typedef typename KeyOf<T>::K K;
  if constexpr (mmp_t<T>::is_bool) {
    return (K)(v ? 1 : 0);
  } else if constexpr (mmp_t<T>::is_float) {
    constexpr K sign = (K)1 << (8 * sizeof(K) - 1);
    K u = __builtin_bit_cast(K, v);
    const bool nan = (typename mmp_t<T>::C)v != (typename mmp_t<T>::C)v;
    if (nan) u = CANON ? (K)~(K)0 >> 1 : (K)(u & ~sign);  // positive NaN, above +inf
    if (CANON && u == sign) u = 0;                          // -0.0 -> +0.0
    return (u & sign) ? (K)~u : (K)(u | sign);
  } else if constexpr (mmp_t<T>::is_signed) {
    constexpr K sign = (K)1 << (8 * sizeof(K) - 1);
    return (K)((K)v ^ sign);
  } else {
    return (K)v;
  }
}

template <typename T> __device__ __forceinline__ T from_key(typename KeyOf<T>::K k) {
  typedef typename KeyOf<T>::K K;
  if constexpr (mmp_t<T>::is_bool) {
    return k != 0;
  } else if constexpr (mmp_t<T>::is_float) {
    constexpr K sign = (K)1 << (8 * sizeof(K) - 1);
    return __builtin_bit_cast(T, (K)((k & sign) ? (K)(k ^ sign) : (K)~k));
  } else if constexpr (mmp_t<T>::is_signed) {
    constexpr K sign = (K)1 << (8 * sizeof(K) - 1);
    return (T)(K)(k ^ sign);
  } else {
    return (T)k;
  }
}

template <typename K>
__device__ __forceinline__ unsigned digit_of(K key, int shift) {
  return (unsigned)(key >> shift) & 255u;
}

// Segmented tiling: row r (of `len` elements) owns tiles r * tpr ..
// r * tpr + tpr - 1; tile j of a row covers row positions
// [j * kTile, min((j + 1) * kTile, len)).  Tile counts are stored
// (row, digit, tile)-major, so one inclusive scan over all of them gives
// every (row, digit, tile) its global output offset: rows stay apart
// without extra digit passes.
struct SegTile {
  unsigned start;  // global position of the tile's first element
  unsigned count;  // elements in the tile
  unsigned row, j;
};
// Workgroup ids are dealt round-robin over the eight XCDs; tile numbers are
// remapped so that each XCD takes a contiguous range of tiles.  Neighbouring
// tiles' digit counts share cache lines (count_slot is tile-minor), which
// then fill in one XCD's L2 instead of being written piecewise from eight.
__device__ __forceinline__ unsigned xcd_tile(unsigned b, unsigned tiles) {
  return (tiles & 7u) == 0 ? (b & 7u) * (tiles >> 3) + (b >> 3) : b;
}
__device__ __forceinline__ SegTile seg_tile(unsigned b, unsigned len, unsigned tpr) {
  SegTile t;
  t.row = b / tpr;
  t.j = b - t.row * tpr;
  const unsigned off = t.j * (unsigned)kTile;
  t.start = t.row * len + off;
  t.count = len - off < (unsigned)kTile ? len - off : (unsigned)kTile;
  return t;
}
__device__ __forceinline__ size_t count_slot(const SegTile &t, unsigned d, unsigned tpr) {
  return ((size_t)t.row * kRadix + d) * tpr + t.j;
}

// Tile histogram of one digit.  FIRST: the pass reads the input values and
// converts them to keys on the fly (no separate conversion sweep).  Whole
// 16-byte-aligned tiles are read with 16-byte loads.
template <typename T, bool FIRST, bool CANON>
__global__ __launch_bounds__(kBlock) void k_radix_hist(const void *__restrict__ src, int shift,
                                                       unsigned len, unsigned tpr,
                                                       unsigned *__restrict__ counts) {
  typedef typename KeyOf<T>::K K;
  typedef typename std::conditional<FIRST, T, K>::type E;  // element type read
  // kSub sub-histograms, lane l counting into l % kSub, each padded by one
  // word: lanes with equal digits (the sign and exponent byte of floats
  // takes a handful of values) then hit kSub different banks instead of
  // queueing on one LDS word.
  constexpr int kSub = 16, kStride = kRadix + 1;
  __shared__ unsigned h[kSub * kStride];
  const int t = threadIdx.x;
  unsigned *hs = h + (t & (kSub - 1)) * kStride;
  for (int k = t; k < kSub * kStride; k += kBlock) h[k] = 0;
  __syncthreads();
  const SegTile tl = seg_tile(xcd_tile(blockIdx.x, gridDim.x), len, tpr);
  const E *e = reinterpret_cast<const E *>(src) + tl.start;
  auto key_at = [&](E v) -> K {
    if constexpr (FIRST) return to_key<T, CANON>(v);
    else return v;
  };
  constexpr int V = 16 / sizeof(E);
  if (tl.count == (unsigned)kTile && ((uintptr_t)e & 15u) == 0) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 *pv = reinterpret_cast<const u32x4 *>(e);
#pragma unroll 4
    for (int j = t; j < kTile / V; j += kBlock) {
      union {
        u32x4 v;
        E x[V];
      } q;
      q.v = __builtin_nontemporal_load(pv + j);
#pragma unroll
      for (int i = 0; i < V; ++i) atomicAdd(&hs[digit_of<K>(key_at(q.x[i]), shift)], 1u);
    }
  } else {
    for (unsigned i = t; i < tl.count; i += kBlock)
      atomicAdd(&hs[digit_of<K>(key_at(e[i]), shift)], 1u);
  }
  __syncthreads();
  unsigned c = 0;
#pragma unroll
  for (int k = 0; k < kSub; ++k) c += h[k * kStride + t];
  counts[count_slot(tl, t, tpr)] = c;
}

// exclusive prefix over the 256 threads of a block (value per thread)
__device__ __forceinline__ unsigned block_exclusive_scan(unsigned v, unsigned *lds4) {
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  unsigned incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) lds4[w] = incl;
  __syncthreads();
  unsigned before = 0;
  for (int k = 0; k < w; ++k) before += lds4[k];
  return before + incl - v;
}

// FINAL: 0 = intermediate pass (keys and indices to kout / iout);
// 1 = last pass of a keys-only sort (values to vout);
// 2 = last pass with indices (row-relative int64 indices to oidx and / or
//     values gathered from x to vout).
// FIRST: keys are read from x and converted; indices are the positions.
template <typename T, bool IDX, int FINAL, bool FIRST>
__global__ __launch_bounds__(kBlock) void k_radix_scatter(
    const typename KeyOf<T>::K *__restrict__ kin, const unsigned *__restrict__ iin,
    typename KeyOf<T>::K *__restrict__ kout, unsigned *__restrict__ iout, int shift,
    unsigned len, unsigned tpr, const unsigned *__restrict__ counts,
    const unsigned long long *__restrict__ incl, const T *__restrict__ x, T *__restrict__ vout,
    long long *__restrict__ oidx) {
  typedef typename KeyOf<T>::K K;
  constexpr int kWaves = kBlock / 64;
  constexpr int kPerWave = kTile / kWaves;  // contiguous keys ranked by one wave
  typedef unsigned WC;  // 32-bit: sub-dword LDS stores measured slower
  __shared__ K sk[kTile];
  __shared__ unsigned si[IDX ? kTile : 1];
  __shared__ WC wc[kWaves][kRadix];  // per-wave digit counts, then offsets
  __shared__ unsigned dstart[kRadix];
  __shared__ unsigned long long goff[kRadix];
  __shared__ unsigned lds4[kWaves];

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const SegTile tl = seg_tile(xcd_tile(blockIdx.x, gridDim.x), len, tpr);
  {
    const size_t slot = count_slot(tl, t, tpr);
    const unsigned c = counts[slot];
    dstart[t] = block_exclusive_scan(c, lds4);
    goff[t] = incl[slot] - c;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) wc[k][t] = 0;
  }
  __syncthreads();

  // Wave w ranks tile positions [w * kPerWave, (w + 1) * kPerWave) in rounds
  // of 64 consecutive keys; its counters are private to it, so the rounds
  // need no block barrier.  Within a round the lanes holding one digit find
  // each other with eight ballots; all of them read the digit's running
  // count, then the lowest of them adds the group's size.
  K key[kIPT];
  unsigned id[kIPT];
  unsigned short rank[kIPT];
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  // All loads first, so that they overlap.  The first pass loads its values
  // unguarded (a lane past the tile's end reads the tile's first element)
  // and converts them to keys in a loop of its own: converted inside a
  // guarded load, each value was waited for before the next load was
  // issued (the pass ran at ~3/4 of the others' speed).
  typedef typename std::conditional<mmp_t<T>::is_bool, unsigned char, T>::type L;  // as loaded
  L raw[FIRST ? kIPT : 1];
#pragma unroll
  for (int r = 0; r < kIPT; ++r) {
    const unsigned loc = (unsigned)(w * kPerWave + r * 64 + lane);
    const bool valid = loc < tl.count;
    const unsigned p = tl.start + loc;
    if constexpr (FIRST) {
      // past the tile's end: load its first element (no branch around the load)
      raw[r] = reinterpret_cast<const L *>(x)[valid ? p : tl.start];
      id[r] = p;
    } else {
      key[r] = valid ? kin[p] : (K)0;
      id[r] = (IDX && valid) ? iin[p] : 0u;
    }
  }
  if constexpr (FIRST) {
#pragma unroll
    for (int r = 0; r < kIPT; ++r) {
      const unsigned loc = (unsigned)(w * kPerWave + r * 64 + lane);
      key[r] = loc < tl.count ? to_key<T, IDX>((T)raw[r]) : (K)0;
    }
  }
#pragma unroll
  for (int r = 0; r < kIPT; ++r) {
    const unsigned loc = (unsigned)(w * kPerWave + r * 64 + lane);
    const bool valid = loc < tl.count;
    const unsigned d = valid ? digit_of<K>(key[r], shift) : 0u;
    unsigned long long m = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
      const bool on = (d >> bit) & 1u;
      const unsigned long long bb = __ballot(valid && on);
      m &= on ? bb : ~bb;
    }
    const unsigned long long lower = m & lt_mask;
    const unsigned c = valid ? wc[w][d] : 0u;
    rank[r] = (unsigned short)(c + (unsigned)__popcll(lower));
    if (valid && lower == 0ull) wc[w][d] = (WC)(c + (unsigned)__popcll(m));
  }
  __syncthreads();
  {
    // wave offsets within each digit of the tile
    unsigned acc = 0;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
      const unsigned c = wc[k][t];
      wc[k][t] = (WC)acc;
      acc += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kIPT; ++r) {
    const unsigned loc = (unsigned)(w * kPerWave + r * 64 + lane);
    if (loc < tl.count) {
      const unsigned d = digit_of<K>(key[r], shift);
      const unsigned pos = dstart[d] + wc[w][d] + rank[r];
      sk[pos] = key[r];
      if constexpr (IDX) si[pos] = id[r];
    }
  }
  __syncthreads();

  for (unsigned q = t; q < tl.count; q += kBlock) {
    const K k = sk[q];
    const unsigned i = IDX ? si[q] : 0u;
    const unsigned d = digit_of<K>(k, shift);
    const unsigned long long g = goff[d] + (q - dstart[d]);
    if constexpr (FINAL == 0) {
      kout[g] = k;
      if constexpr (IDX) iout[g] = i;
    } else if constexpr (FINAL == 1) {
      vout[g] = from_key<T>(k);
    } else {
      if (oidx) oidx[g] = (long long)(i % len);
      if (vout) vout[g] = x[i];
    }
  }
}

// Rows of at most one tile: one workgroup sorts a tile in LDS through every
// digit pass and writes it once (the multi-pass path above reads and writes
// each key three times per digit and launches three kernels per digit).  A
// tile holds one row, or for rows of at most 512 keys rpt = min(256,
// 4096 / len) whole consecutive rows; after the key passes one more pass
// then sorts by the row within the tile (its most significant digit), so
// every row's keys end in the row's own positions (rows are contiguous in
// memory: output position p of the tile is row p / len, column p % len).  Each pass ranks keys exactly as
// k_radix_scatter does -- waves, rounds and lanes in position order, eight
// ballots per round, wave-private counters -- with the tile's own digit
// counts as the offsets, so the order (stable) and the keys' canonical
// forms are the multi-pass path's.  A pass whose digit is the same for
// every key of the tile leaves the order as it is and is skipped.  A tile is
// split evenly over the four waves (q positions each, a multiple of 64;
// rounds past q are skipped).  With IDX or packed rows (CARRY) a key
// carries its tile position and row as one word: row << 12 | position.
// Tiles are taken grid-stride.
template <typename T, bool IDX, bool CARRY>
__global__ __launch_bounds__(kBlock) void k_sort_tile(const T *__restrict__ x, unsigned len,
                                                       long long rows, unsigned rpt,
                                                       T *__restrict__ vout,
                                                       long long *__restrict__ oidx) {
  typedef typename KeyOf<T>::K K;
  constexpr int kWaves = kBlock / 64;
  constexpr int kKeyPasses = (int)sizeof(K);
  __shared__ K sk[kTile];
  __shared__ unsigned si[CARRY ? kTile : 1];  // row << 12 | tile position
  __shared__ unsigned wc[kWaves][kRadix];  // per-wave digit counts, then offsets
  __shared__ unsigned dstart[kRadix];
  __shared__ unsigned lds4[kWaves];
  __shared__ int same_digit;

  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const unsigned long long lt_mask = (1ull << lane) - 1ull;
  const long long tiles = (rows + rpt - 1) / rpt;
  const int passes = kKeyPasses + (CARRY && rpt > 1 ? 1 : 0);
  for (long long tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    const long long row0 = tile * rpt;
    const unsigned nrows = (unsigned)(rows - row0 < (long long)rpt ? rows - row0 : rpt);
    const unsigned n = nrows * len;  // <= kTile
    const unsigned q = ((n + kWaves - 1) / kWaves + 63u) & ~63u;  // positions per wave
    const T *xt = x + row0 * (long long)len;
    K key[kIPT];
    unsigned id[kIPT];
#pragma unroll
    for (int r = 0; r < kIPT; ++r) {
      const unsigned loc = w * q + (unsigned)(r * 64 + lane);  // < 4096
      const bool in = r * 64 < (int)q && loc < n;
      key[r] = in ? to_key<T, IDX>(xt[loc]) : (K)0;
      if constexpr (CARRY) id[r] = in ? ((loc / len) << 12) | loc : 0u;
    }
    for (int ps = 0; ps < passes; ++ps) {
      const bool row_pass = ps == kKeyPasses;
      const int shift = 8 * ps;
#pragma unroll
      for (int k = 0; k < kWaves; ++k) wc[k][t] = 0;
      if (t == 0) same_digit = 0;
      __syncthreads();
      unsigned short rank[kIPT];
#pragma unroll
      for (int r = 0; r < kIPT; ++r) {
        if (r * 64 >= (int)q) break;  // wave-uniform
        const unsigned loc = w * q + (unsigned)(r * 64 + lane);
        const bool valid = loc < n;
        const unsigned d = !valid ? 0u : row_pass ? (id[r] >> 12) : digit_of<K>(key[r], shift);
        static_assert(CARRY || !IDX, "indices need the carried positions");
        unsigned long long m = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
          const bool on = (d >> bit) & 1u;
          const unsigned long long bb = __ballot(valid && on);
          m &= on ? bb : ~bb;
        }
        const unsigned long long lower = m & lt_mask;
        const unsigned c = valid ? wc[w][d] : 0u;
        rank[r] = (unsigned short)(c + (unsigned)__popcll(lower));
        if (valid && lower == 0ull) wc[w][d] = c + (unsigned)__popcll(m);
      }
      __syncthreads();
      unsigned total = 0;  // of digit t over the waves; wave offsets within it
#pragma unroll
      for (int k = 0; k < kWaves; ++k) {
        const unsigned c = wc[k][t];
        wc[k][t] = total;
        total += c;
      }
      if (total == n) same_digit = 1;
      dstart[t] = block_exclusive_scan(total, lds4);  // its barrier publishes same_digit
      __syncthreads();
      if (!same_digit) {
#pragma unroll
        for (int r = 0; r < kIPT; ++r) {
          const unsigned loc = w * q + (unsigned)(r * 64 + lane);
          if (r * 64 < (int)q && loc < n) {
            const unsigned d = row_pass ? (id[r] >> 12) : digit_of<K>(key[r], shift);
            const unsigned pos = dstart[d] + wc[w][d] + rank[r];
            sk[pos] = key[r];
            if constexpr (CARRY) si[pos] = id[r];
          }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kIPT; ++r) {
          const unsigned loc = w * q + (unsigned)(r * 64 + lane);
          if (r * 64 < (int)q && loc < n) {
            key[r] = sk[loc];
            if constexpr (CARRY) id[r] = si[loc];
          }
        }
      }
      __syncthreads();  // the next pass rewrites the counters and the staging tile
    }
    T *vt = vout ? vout + row0 * (long long)len : nullptr;
    long long *ot = oidx ? oidx + row0 * (long long)len : nullptr;
#pragma unroll
    for (int r = 0; r < kIPT; ++r) {
      const unsigned loc = w * q + (unsigned)(r * 64 + lane);
      if (r * 64 < (int)q && loc < n) {
        if constexpr (IDX) {
          const unsigned src = id[r] & 4095u, row = id[r] >> 12;
          if (ot) ot[loc] = (long long)(src - row * len);  // position within its row
          if (vt) vt[loc] = xt[src];
        } else {
          vt[loc] = from_key<T>(key[r]);
        }
      }
    }
  }
}

template <typename T, bool IDX, int FINAL, bool FIRST = false>
int launch_scatter(unsigned tiles, const void *kin, const unsigned *iin, void *kout, unsigned *iout,
                   int shift, unsigned len, unsigned tpr, const unsigned *counts,
                   const unsigned long long *incl, const T *x, T *vout, long long *oidx) {
  typedef typename KeyOf<T>::K K;
  hipLaunchKernelGGL((k_radix_scatter<T, IDX, FINAL, FIRST>), dim3(tiles), dim3(kBlock), 0,
                     mmpi::stream(), (const K *)kin, iin, (K *)kout, iout, shift, len, tpr,
                     counts, incl, x, vout, oidx);
  return mmpi::check_launch("mmp_sort(scatter)");
}

// temporaries from the library's stream-ordered pool, released on scope exit
struct Temp {
  void *p = nullptr;
  ~Temp() {
    if (p) (void)mmp_free(p);
  }
  int get(size_t bytes) { return mmp_alloc(bytes ? bytes : 1, &p); }
};

template <typename T>
int sort_impl(long long rows, long long len, const T *x, T *vout, long long *oidx, bool stable) {
  typedef typename KeyOf<T>::K K;
  const long long n64 = rows * len;
  // 32-bit positions; tile counts addressed with 32-bit tile numbers
  if (n64 > 0xffffe000LL) return mmpi::fail(MMP_E_UNSUPPORTED, "mmp_sort: more than 2^32 - 8192 elements");
  const long long tpr64 = mmpi::ceil_div(len, kTile);
  const long long tiles64 = rows * tpr64;
  if (tiles64 > 0x7fffffffLL) return mmpi::fail(MMP_E_UNSUPPORTED, "mmp_sort: too many rows");
  const unsigned n = (unsigned)n64, ulen = (unsigned)len, tpr = (unsigned)tpr64;
  const unsigned tiles = (unsigned)tiles64;
  const bool idx = oidx != nullptr || stable;
  if (len <= kTile) {  // rows of at most one tile: all passes in LDS, whole rows per tile
    // rows of more than 512 keys: one per tile (1024-key rows: 0.94 ms for
    // 65536 rows alone, 1.16 ms packed four to a tile with the row pass);
    // shorter ones packed (256-key rows: 1.85 ms alone, 1.18 packed)
    const unsigned rpt = len > 512 ? 1u : (unsigned)std::min<long long>(256, kTile / len);
    const long long ntiles = (rows + rpt - 1) / rpt;
    // one workgroup per tile (the dispatcher balances them; a fixed share
    // of tiles per workgroup left a long tail: 65536 rows of 1024 keys
    // 1.22 ms on 4096 workgroups against 0.94 on one per tile); only
    // more than 2^20 tiles (rows under 16 keys past 2^28 elements) are
    // taken grid-stride
    const unsigned grid = (unsigned)std::min<long long>(ntiles, 1LL << 20);
    if (idx)
      hipLaunchKernelGGL((k_sort_tile<T, true, true>), dim3(grid), dim3(kBlock), 0,
                         mmpi::stream(), x, ulen, (long long)rows, rpt, vout, oidx);
    else if (rpt > 1)
      hipLaunchKernelGGL((k_sort_tile<T, false, true>), dim3(grid), dim3(kBlock), 0,
                         mmpi::stream(), x, ulen, (long long)rows, rpt, vout, oidx);
    else
      hipLaunchKernelGGL((k_sort_tile<T, false, false>), dim3(grid), dim3(kBlock), 0,
                         mmpi::stream(), x, ulen, (long long)rows, rpt, vout, oidx);
    return mmpi::check_launch("mmp_sort(tile)");
  }
  Temp ka, kb, ia, ib, cnt, inc;
  if (int st = ka.get((size_t)n * sizeof(K))) return st;
  if (int st = kb.get((size_t)n * sizeof(K))) return st;
  if (idx) {
    if (int st = ia.get((size_t)n * 4)) return st;
    if (int st = ib.get((size_t)n * 4)) return st;
  }
  const size_t nslots = (size_t)tiles * kRadix;
  if (int st = cnt.get(nslots * 4)) return st;
  if (int st = inc.get(nslots * 8)) return st;

  const int passes = (int)sizeof(K);
  void *kin = kb.p, *kout = ka.p;  // the first pass reads x, writes ka
  unsigned *iin = (unsigned *)ib.p, *iout = (unsigned *)ia.p;
  for (int ps = 0; ps < passes; ++ps) {
    const int shift = 8 * ps;
    const bool first = ps == 0, last = ps == passes - 1;
    if (first && idx)
      hipLaunchKernelGGL((k_radix_hist<T, true, true>), dim3(tiles), dim3(kBlock), 0,
                         mmpi::stream(), (const void *)x, shift, ulen, tpr, (unsigned *)cnt.p);
    else if (first)
      hipLaunchKernelGGL((k_radix_hist<T, true, false>), dim3(tiles), dim3(kBlock), 0,
                         mmpi::stream(), (const void *)x, shift, ulen, tpr, (unsigned *)cnt.p);
    else
      hipLaunchKernelGGL((k_radix_hist<T, false, false>), dim3(tiles), dim3(kBlock), 0,
                         mmpi::stream(), (const void *)kin, shift, ulen, tpr, (unsigned *)cnt.p);
    if (int st = mmpi::check_launch("mmp_sort(hist)")) return st;
    if (int st = mmp_scan(MMP_S_CUMSUM, MMP_U32, MMP_U64, 1, (int64_t)nslots, 1, cnt.p, inc.p))
      return st;
    const unsigned *c = (const unsigned *)cnt.p;
    const unsigned long long *ic = (const unsigned long long *)inc.p;
    int st;
    if (first) {
      // the first pass is never the last (keys have at least two bytes)
      st = idx ? launch_scatter<T, true, 0, true>(tiles, kin, iin, kout, iout, shift, ulen, tpr,
                                                   c, ic, x, vout, oidx)
               : launch_scatter<T, false, 0, true>(tiles, kin, iin, kout, iout, shift, ulen, tpr,
                                                    c, ic, x, vout, oidx);
    } else if (!idx) {
      st = last ? launch_scatter<T, false, 1>(tiles, kin, iin, kout, iout, shift, ulen, tpr, c, ic,
                                              x, vout, oidx)
                : launch_scatter<T, false, 0>(tiles, kin, iin, kout, iout, shift, ulen, tpr, c, ic,
                                              x, vout, oidx);
    } else {
      st = last ? launch_scatter<T, true, 2>(tiles, kin, iin, kout, iout, shift, ulen, tpr, c, ic,
                                             x, vout, oidx)
                : launch_scatter<T, true, 0>(tiles, kin, iin, kout, iout, shift, ulen, tpr, c, ic,
                                             x, vout, oidx);
    }
    if (st) return st;
    void *tk = kin;
    kin = kout;
    kout = tk;
    unsigned *ti = iin;
    iin = iout;
    iout = ti;
  }
  return MMP_OK;
}

// -------------------------------------------------------- searchsorted
// NumPy's order: NaN after everything, -0.0 == +0.0.
template <typename T> __device__ __forceinline__ bool lt_nan_last(T a_, T b_) {
  if constexpr (mmp_t<T>::is_float) {
    typedef typename mmp_t<T>::C C;
    const C a = (C)a_, b = (C)b_;
    return a < b || (b != b && a == a);
  } else {
    return a_ < b_;
  }
}

template <typename T, bool RIGHT>
__global__ __launch_bounds__(kBlock) void k_searchsorted(const T *__restrict__ a, long long n,
                                                         const T *__restrict__ v, long long m,
                                                         long long *__restrict__ out) {
  const long long i = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (i >= m) return;
  const T q = v[i];
  long long lo = 0, hi = n;
  while (lo < hi) {
    const long long mid = lo + ((hi - lo) >> 1);
    const bool go_right = RIGHT ? !lt_nan_last(q, a[mid]) : lt_nan_last(a[mid], q);
    if (go_right) lo = mid + 1;
    else hi = mid;
  }
  out[i] = lo;
}

// ---------------------------------------------------------------- take
template <typename U>
__global__ __launch_bounds__(kBlock) void k_take(const U *__restrict__ src, long long nsrc,
                                                 const long long *__restrict__ idx, long long n,
                                                 U *__restrict__ out) {
  const long long i = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const long long j = idx[i];
  out[i] = (j >= 0 && j < nsrc) ? src[j] : (U)0;  // out-of-range indices read nothing
}

}  // namespace

extern "C" int mmp_sort(int dtype, int64_t rows, int64_t len, const void *x, void *out_values,
                        int64_t *out_indices, int stable) {
  if (int st = mmpi::ensure_init()) return st;
  if (rows < 0 || len < 0) return mmpi::fail(MMP_E_ARG, "mmp_sort: negative extent");
  if (rows * len == 0) return MMP_OK;
  if (!x || (!out_values && !out_indices)) return mmpi::fail(MMP_E_ARG, "mmp_sort: null pointer");
  MMP_DISPATCH_ALL(dtype, {
    return sort_impl<T>(rows, len, (const T *)x, (T *)out_values, (long long *)out_indices,
                        stable != 0);
  })
}

extern "C" int mmp_searchsorted(int dtype, int64_t n, const void *sorted, int64_t m,
                                const void *values, int side_right, int64_t *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (n < 0 || m < 0) return mmpi::fail(MMP_E_ARG, "mmp_searchsorted: negative extent");
  if (m == 0) return MMP_OK;
  if (!values || !out || (n > 0 && !sorted))
    return mmpi::fail(MMP_E_ARG, "mmp_searchsorted: null pointer");
  const unsigned grid = (unsigned)mmpi::ceil_div(m, kBlock);
  MMP_DISPATCH_ALL(dtype, {
    if (side_right)
      hipLaunchKernelGGL((k_searchsorted<T, true>), dim3(grid), dim3(kBlock), 0, mmpi::stream(),
                         (const T *)sorted, (long long)n, (const T *)values, (long long)m,
                         (long long *)out);
    else
      hipLaunchKernelGGL((k_searchsorted<T, false>), dim3(grid), dim3(kBlock), 0, mmpi::stream(),
                         (const T *)sorted, (long long)n, (const T *)values, (long long)m,
                         (long long *)out);
    return mmpi::check_launch("mmp_searchsorted");
  })
}

extern "C" int mmp_take(int itemsize, int64_t nsrc, const void *src, int64_t n,
                        const int64_t *indices, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (nsrc < 0 || n < 0) return mmpi::fail(MMP_E_ARG, "mmp_take: negative extent");
  if (n == 0) return MMP_OK;
  if (!indices || !out || (nsrc > 0 && !src)) return mmpi::fail(MMP_E_ARG, "mmp_take: null pointer");
  const unsigned grid = (unsigned)mmpi::ceil_div(n, kBlock);
  const long long *ix = (const long long *)indices;
  switch (itemsize) {
    case 1:
      hipLaunchKernelGGL((k_take<unsigned char>), dim3(grid), dim3(kBlock), 0, mmpi::stream(),
                         (const unsigned char *)src, (long long)nsrc, ix, (long long)n,
                         (unsigned char *)out);
      break;
    case 2:
      hipLaunchKernelGGL((k_take<unsigned short>), dim3(grid), dim3(kBlock), 0, mmpi::stream(),
                         (const unsigned short *)src, (long long)nsrc, ix, (long long)n,
                         (unsigned short *)out);
      break;
    case 4:
      hipLaunchKernelGGL((k_take<unsigned>), dim3(grid), dim3(kBlock), 0, mmpi::stream(),
                         (const unsigned *)src, (long long)nsrc, ix, (long long)n, (unsigned *)out);
      break;
    case 8:
      hipLaunchKernelGGL((k_take<unsigned long long>), dim3(grid), dim3(kBlock), 0,
                         mmpi::stream(), (const unsigned long long *)src, (long long)nsrc, ix,
                         (long long)n, (unsigned long long *)out);
      break;
    default:
      return mmpi::fail(MMP_E_ARG, "mmp_take: item size %d", itemsize);
  }
  return mmpi::check_launch("mmp_take");
}
