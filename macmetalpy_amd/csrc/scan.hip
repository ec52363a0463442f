// scan.hip -- cumsum / cumprod.
//
// Replaces the reference's three-pass Metal scan (_kernels.py:1263-1360,
// driven by ndarray._prefix_scan ndarray.py:2068-2152): block-local serial
// scans, then ONE thread scanning all block totals, then a propagation pass.
//
// Here a contiguous scan (any number of rows of length len) is a single
// pass of decoupled look-back:
//  * a tile's id is its workgroup id; a tile never waits without bound for
//    a predecessor (whose workgroup may not have started: AMD gives no
//    forward-progress guarantee to workgroups that have not started) --
//    after a few polls it sums that predecessor's input itself;
//  * a tile (16384 elements: 4 sub-tiles of 256 threads x 16 consecutive
//    elements) is loaded with 128-bit loads, all issued up front, and
//    redistributed through LDS into registers, scanned serially per thread
//    in the accumulator type, then across the wave64 with shuffles and
//    across the 4 waves through LDS;
//  * wave 0 publishes the tile aggregate, reads the 8 nearest predecessors'
//    descriptors at once and combines aggregates up to the nearest
//    inclusive prefix, then publishes its own inclusive prefix;
//  * descriptors carry a per-call generation tag, so they are never
//    cleared between calls;
//  * rows whose byte length is a multiple of 16 (and 16-byte aligned
//    operands) run their whole tiles through a guard-free kernel and each
//    row's partial tail through a second small launch; other layouts run a
//    guarded kernel.
// Accumulators: int64 for integers (int32 -> int64 output as NumPy),
// float64 for floats (rounded once per output element).  HBM-bound:
// sizeof(in) + sizeof(out) bytes per element.
// Strided scans (inner > 1) run one thread per column, coalesced across
// columns, with the axis cut into chunks (totals first, then a rescan from
// each chunk's carry-in) so that narrow arrays still fill the device.
#include "mmp_ops.h"
#include "mmp_internal.h"

namespace {

constexpr int kBlock = 256;
constexpr int kItems = 16;                // consecutive elements per thread per sub-tile
constexpr int kSubTile = kBlock * kItems; // 4096 elements staged through LDS at a time
constexpr int kPad = kSubTile / kItems;   // one pad word per thread row in LDS
// A tile (one ticket, one look-back) is kSub sub-tiles: 16384 elements for
// 1-, 2- and 4-byte inputs, 8192 for 8-byte inputs (register budget).  A
// same-address atomic ticket costs ~11 ns per workgroup on MI355X and the
// tickets serialise, so tiles must be large.
template <typename Ti> constexpr int sub_tiles() { return sizeof(Ti) >= 8 ? 2 : 4; }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct ScanAcc { typedef double type; };
template <> struct ScanAcc<mmp_i16> { typedef mmp_i64 type; };
template <> struct ScanAcc<mmp_i32> { typedef mmp_i64 type; };
template <> struct ScanAcc<mmp_i64> { typedef mmp_i64 type; };
template <> struct ScanAcc<bool> { typedef mmp_i64 type; };
template <> struct ScanAcc<mmp_u16> { typedef mmp_u64 type; };
template <> struct ScanAcc<mmp_u32> { typedef mmp_u64 type; };
template <> struct ScanAcc<mmp_u64> { typedef mmp_u64 type; };

template <int OP, typename T> struct ScanOp {
  typedef typename ScanAcc<T>::type A;
  static __device__ __forceinline__ A ident() { return OP == MMP_S_CUMSUM ? (A)0 : (A)1; }
  static __device__ __forceinline__ A map(T v) {
    if constexpr (mmp_t<T>::is_float) return (A)(typename mmp_t<T>::C)v;
    else return (A)v;
  }
  static __device__ __forceinline__ A comb(A a, A b) {
    if constexpr (mmp_t<T>::is_float) {
      return OP == MMP_S_CUMSUM ? a + b : a * b;
    } else {
      return OP == MMP_S_CUMSUM ? (A)((mmp_u64)a + (mmp_u64)b) : (A)((mmp_u64)a * (mmp_u64)b);
    }
  }
};

__device__ __forceinline__ int padded(int i) { return i + i / kItems; }

template <typename A> __device__ __forceinline__ A shfl_xor64(A v, int m) {
  unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  unsigned lo = __shfl_xor((unsigned)u, m, 64), hi = __shfl_xor((unsigned)(u >> 32), m, 64);
  return __builtin_bit_cast(A, ((unsigned long long)hi << 32) | lo);
}

template <typename A> __device__ __forceinline__ A shfl64(A v, int src) {
  unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  unsigned lo = __shfl((unsigned)u, src, 64), hi = __shfl((unsigned)(u >> 32), src, 64);
  return __builtin_bit_cast(A, ((unsigned long long)hi << 32) | lo);
}

// Lane `src` (wave-uniform) of v, read into scalar registers.
template <typename A> __device__ __forceinline__ A readlane64(A v, int src) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const unsigned lo = __builtin_amdgcn_readlane((unsigned)u, src);
  const unsigned hi = __builtin_amdgcn_readlane((unsigned)(u >> 32), src);
  return __builtin_bit_cast(A, ((unsigned long long)hi << 32) | lo);
}

template <typename A> __device__ __forceinline__ A shfl_up64(A v, int d) {
  unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  unsigned lo = __shfl_up((unsigned)u, d, 64), hi = __shfl_up((unsigned)(u >> 32), d, 64);
  return __builtin_bit_cast(A, ((unsigned long long)hi << 32) | lo);
}

// Tile descriptors are two 64-bit words, each = (tag << 32) | 32 payload
// bits, tag = generation << 2 | state (1 aggregate, 2 inclusive prefix).
// They are written and read with RELAXED agent-scope atomics; a reader only
// accepts a descriptor whose two tags agree and carry this call's
// generation.  No release/acquire fences: on multi-XCD CDNA those write
// back / invalidate the whole L2 and would serialise the look-back.
template <typename A>
__device__ __forceinline__ void publish(unsigned long long *d, A v, unsigned tag) {
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const unsigned long long hi = (unsigned long long)tag << 32;
  __hip_atomic_store(d, hi | (u & 0xffffffffull), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(d + 1, hi | (u >> 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct ScanScratch {
  unsigned long long *desc;   // 2 words per tile
  unsigned *timeout;          // pinned host word, set to 1 if a tail's prefix was missing
  unsigned read_gen;          // generation look-back readers expect (== gen unless forced)
  long long spin_limit;       // look-back polls before a tile sums a predecessor itself
};

template <bool B> struct Bool { static constexpr bool value = B; };

// An empty asm "redefinition": the value is only available where this is
// executed.  Used on the inputs in the output pass, so that the compiler
// neither hoists that pass's running sums above the barriers (which keeps
// all 64 wide accumulators of a thread live at once) nor keeps the widened
// inputs of the totals pass alive for it; either costs half the occupancy.
template <typename T> __device__ __forceinline__ T opaque(T v) {
  if constexpr (sizeof(T) == 4 || sizeof(T) == 8) {
    asm volatile("" : "+v"(v));
    return v;
  } else if constexpr (sizeof(T) == 2) {
    unsigned u = (unsigned)__builtin_bit_cast(unsigned short, v);
    asm volatile("" : "+v"(u));
    return __builtin_bit_cast(T, (unsigned short)u);
  } else {
    unsigned u = (unsigned)__builtin_bit_cast(unsigned char, v);
    asm volatile("" : "+v"(u));
    return __builtin_bit_cast(T, (unsigned char)u);
  }
}

// Decoupled look-back by wave 0: lanes 0..kLook-1 read the descriptors of
// the kLook (4 or 8, below) nearest predecessors at once (lane 0 = tile - 1).  The window is
// usable when every lane nearer than the nearest inclusive prefix holds a
// valid aggregate; otherwise it is re-read.  Tiles before the row's first
// tile count as an inclusive identity.  Returns the exclusive prefix of
// `tile` (lane 0's value is the one used).  The descriptor reads are
// agent-scope loads that contend with the other tiles' publications;
// measured on MI355X at 2^28 elements, int32 -> int64: 64 tiles per round
// 0.72 ms, 32: 0.64, 16: 0.60, 8: 0.58, 4: 0.57 (float32 best at 8), and
// 256 per round 1.03 ms.
//
// Tiles are numbered by workgroup id, so a predecessor may belong to a
// workgroup that has not started (nothing in the hardware promises that a
// lower id runs first, although dispatch is in id order in practice).  A
// tile therefore never waits for one without bound: after sc.spin_limit
// polls it reads the nearest missing predecessor's input and sums it
// itself (64 KiB for a float32 tile, a few microseconds), and goes on.
// Forward progress needs no other workgroup, and no atomic ticket is
// drawn (a same-address ticket per workgroup cost 6 % of the float32 scan).
// Integer prefixes are exact in any association.  A floating scan folds
// the values read in tile order, oldest first, so that every prefix is the
// same sequential fold whichever inclusive prefix a tile found: floating
// scans are bit-for-bit repeatable.
// Window per type, measured at 2^28 elements with the ticket-free look-back:
// int32 -> int64 (8-byte outputs) 4 (6.0 TB/s; 8: 5.9, 16: 5.8).  Floating
// scans fold in tile order (below), which lengthens the walk: a tile's
// look-back goes back 128 tiles on average against 58 with a tree over
// each read (per-tile counts at 2^28 float32); 16 per read then beats 8
// (0.398-0.405 ms against 0.409-0.414; 32: 0.42, 64: 0.51).
template <typename Ti, typename To> constexpr int scan_look() {
  if (mmp_t<Ti>::is_float) return 16;
  return (sizeof(Ti) == 4 && sizeof(To) == 8) ? 4 : 8;
}
constexpr int kLookMax = 16;
constexpr int kMaxWinTiles = 512;  // look-back reads kept for the fold
constexpr long long kPollsBeforeSum = 256;

// Aggregate of a whole tile (Q sub-tiles of kSubTile elements at p) by one
// wave, combined in exactly the order the tile's own workgroup combines it
// (k_scan_rows steps 1-2): thread t of wave w sums its 16 consecutive
// elements from the identity, the wave's inclusive shuffle scan gives lane
// 63's total, the four wave totals fold left from the identity per
// sub-tile, the sub-tile totals fold left from the identity.  A floating
// scan is then bit-identical whether a predecessor's aggregate came from
// its descriptor or from here.  Lane 63's result is the one used (every
// lane holds it after the final broadcast).
template <typename S, int Q, typename Ti>
__device__ typename S::A wave_aggregate(const Ti *__restrict__ p, int lane) {
  typedef typename S::A A;
  A total = S::ident();
#pragma unroll 1
  for (int q = 0; q < Q; ++q) {
    A qtot = S::ident();
#pragma unroll 1
    for (int w = 0; w < kBlock / 64; ++w) {
      const Ti *e = p + q * kSubTile + (w * 64 + lane) * kItems;
      A run = S::ident();
#pragma unroll 1
      for (int j = 0; j < kItems; ++j) run = S::comb(run, S::map(e[j]));
      A inc = run;
#pragma unroll
      for (int dd = 1; dd < 64; dd <<= 1) {
        const A o = shfl_up64(inc, dd);
        if (lane >= dd) inc = S::comb(o, inc);
      }
      qtot = S::comb(qtot, shfl64(inc, 63));
    }
    total = S::comb(total, qtot);
  }
  return total;
}

template <typename S, int kLook, int Q, typename Ti>
__device__ typename S::A look_back(const ScanScratch &sc, long long tile, long long t,
                                   typename S::A total, unsigned gen, int lane,
                                   const Ti *__restrict__ xrow, typename S::A *own_val,
                                   typename S::A *win) {
  constexpr long long tile_len = (long long)Q * kSubTile;
  typedef typename S::A A;
  constexpr bool kOrdered = __is_same(A, double);  // floating: fold in tile order
  constexpr int kMaxWin = kMaxWinTiles / kLook;
  A prefix = S::ident();
  unsigned long long *d = sc.desc;
  if (t > 0) {
    if (lane == 0) publish(d + 2 * tile, total, (gen << 2) | 1u);
    const long long first = tile - t;  // first tile of this row
    const unsigned long long in_window = kLook >= 64 ? ~0ull : ((1ull << kLook) - 1);
    // One descriptor: state 0 missing / stale, 1 aggregate, 2 inclusive
    // prefix; tiles before the row count as an inclusive identity.
    auto read = [&](long long j, bool want, unsigned &state, A &val) {
      state = 2u;
      val = S::ident();
      if (want && j >= first) {
        const unsigned long long w0 = __hip_atomic_load(d + 2 * j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned long long w1 = __hip_atomic_load(d + 2 * j + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned t0 = (unsigned)(w0 >> 32), t1 = (unsigned)(w1 >> 32);
        state = (t0 == t1 && (t0 >> 2) == sc.read_gen) ? (t0 & 3u) : 0u;
        val = __builtin_bit_cast(A, (w0 & 0xffffffffull) | (w1 << 32));
      }
    };
    long long top = tile - 1;
    long long spins = 0;
    int nwin = 0;  // windows read before this one (the first kMaxWin are kept in `win`)
    // lanes whose predecessor was summed here (wave-uniform), values in LDS
    unsigned long long own = 0;
    unsigned state;
    A val;
    int p;
    while (true) {
      read(top - lane, lane < kLook, state, val);
      if (lane < kLook && state == 0u && ((own >> lane) & 1ull)) {
        state = 1u;
        val = own_val[lane];
      }
      const unsigned long long incl = __ballot(state == 2u) & in_window;
      const unsigned long long bad = __ballot(state == 0u) & in_window;
      p = incl ? __ffsll((long long)incl) - 1 : kLook;  // nearest inclusive lane
      const unsigned long long nearer = p >= 63 ? ~0ull : ((1ull << (p + 1)) - 1);
      if (bad & nearer) {
        if (++spins <= sc.spin_limit) {
          __builtin_amdgcn_s_sleep(1);
          continue;
        }
        // the nearest predecessor still missing: sum its input here
        const int b = __ffsll((long long)(bad & nearer)) - 1;
        const A agg = wave_aggregate<S, Q>(xrow + (top - b - first) * tile_len, lane);
        if (lane == b) own_val[b] = agg;
        own |= 1ull << b;
        continue;
      }
      if constexpr (!kOrdered) {  // integers: any association is exact
        A part = lane <= p && lane < kLook ? val : S::ident();
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) part = S::comb(part, shfl_xor64(part, m));
        prefix = S::comb(part, prefix);
      }
      if (p < kLook) break;
      // a window walked past: kept for the fold (the last one stays in registers)
      if (kOrdered && nwin < kMaxWin && lane < kLook) win[nwin * kLook + lane] = val;
      top -= kLook;
      ++nwin;
      own = 0;
      spins = 0;
    }
    if constexpr (kOrdered) {
      // Fold oldest first: the inclusive prefix (lane p of the last window),
      // then every later tile's aggregate in tile order.  Each inclusive
      // prefix is then the sequential fold of the row's tile aggregates from
      // its start, whichever predecessor's prefix a tile started from, so a
      // floating scan rounds the same way in every run.
      A s = S::ident();
      if (nwin < kMaxWin) {
        // the window just read from registers (lane index uniform: readlane),
        // the newer ones from LDS
        s = readlane64(val, p);
        for (int L = p - 1; L >= 0; --L) s = S::comb(s, readlane64(val, L));
        for (int w = nwin - 1; w >= 0; --w)
#pragma unroll
          for (int L = kLook - 1; L >= 0; --L) s = S::comb(s, win[w * kLook + L]);
      } else {
        // More than kMaxWin windows back (rare): re-read the tiles after the
        // inclusive prefix, 64 at a time, folding as above; the newest
        // inclusive prefix in a read replaces the base, a missing aggregate is
        // summed here in the tile's own order (so its bits are the tile's).
        s = shfl64(val, p);
        long long k0 = top - p + 1;
        spins = 0;
        own = 0;
        A own_v = S::ident();
        while (k0 < tile) {
          const int cnt = tile - k0 < 64 ? (int)(tile - k0) : 64;
          unsigned st;
          A v;
          read(k0 + lane, lane < cnt, st, v);
          if ((own >> lane) & 1ull) {
            st = 1u;
            v = own_v;
          }
          const unsigned long long live = cnt >= 64 ? ~0ull : ((1ull << cnt) - 1);
          const unsigned long long incl = __ballot(st == 2u) & live;
          const int q = incl ? 63 - __clzll((long long)incl) : -1;  // newest inclusive lane
          const unsigned long long after =
              q < 0 ? live : (q >= 63 ? 0ull : (live & ~((2ull << q) - 1)));  // lanes after q
          const unsigned long long miss = __ballot(st == 0u) & after;
          if (miss) {
            if (++spins <= sc.spin_limit) {
              __builtin_amdgcn_s_sleep(1);
              continue;
            }
            const int b = __ffsll((long long)miss) - 1;
            const A agg = wave_aggregate<S, Q>(xrow + (k0 + b - first) * tile_len, lane);
            if (lane == b) own_v = agg;
            own |= 1ull << b;
            continue;
          }
          if (q >= 0) s = shfl64(v, q);
          for (int L = q + 1; L < cnt; ++L) s = S::comb(s, shfl64(v, L));
          k0 += cnt;
          own = 0;
          spins = 0;
        }
      }
      prefix = s;
    }
  }
  if (lane == 0) publish(d + 2 * tile, S::comb(prefix, total), (gen << 2) | 2u);
  return prefix;
}

// Prefix for a row's tail (MODE 2): the inclusive descriptor of the row's
// last whole tile, published by the preceding launch on the same stream.
template <typename S>
__device__ typename S::A tail_prefix(const ScanScratch &sc, long long pred, unsigned gen) {
  const unsigned long long w0 = __hip_atomic_load(sc.desc + 2 * pred, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned long long w1 = __hip_atomic_load(sc.desc + 2 * pred + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned t0 = (unsigned)(w0 >> 32), t1 = (unsigned)(w1 >> 32);
  if (!(t0 == t1 && t0 == ((sc.read_gen << 2) | 2u)))
    __hip_atomic_store(sc.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  return __builtin_bit_cast(typename S::A, (w0 & 0xffffffffull) | (w1 << 32));
}

// MODE 0: whole, 16-byte aligned tiles only (grid = rows x whole tiles per
//         row), guard-free streaming body, look-back.
// MODE 1: any layout (grid = rows x ceil tiles per row), guarded body,
//         look-back.
// MODE 2: the partial last tile of each row after a MODE 0 launch (grid =
//         rows); its prefix is the inclusive descriptor MODE 0 published for
//         the row's last whole tile.
// MODE 0 is compiled for at least two workgroups per CU (measured best:
// more concurrent tiles lengthen every look-back); keeping the guarded
// paths out of it keeps its registers down.
template <int OP, typename Ti, typename To, int MODE>
__global__ __launch_bounds__(kBlock, MODE == 0 ? 2 : 1) void k_scan_rows(
    const Ti *__restrict__ x, To *__restrict__ y, long long len, long long tiles_per_row,
    long long ntiles, ScanScratch sc, unsigned gen) {
  typedef ScanOp<OP, Ti> S;
  typedef typename S::A A;
  constexpr int Q = sub_tiles<Ti>();
  constexpr int kTile = Q * kSubTile;
  constexpr int kStage = (sizeof(Ti) > sizeof(To) ? sizeof(Ti) : sizeof(To));
  __shared__ __attribute__((aligned(16))) unsigned char stage[(kSubTile + kPad) * kStage];
  __shared__ A wsum[Q][kBlock / 64];
  __shared__ A s_prefix;
  __shared__ A s_own[kLookMax];  // predecessor aggregates the look-back summed itself
  __shared__ A s_win[kMaxWinTiles];  // the look-back's reads, folded oldest first
  __shared__ A s_excl[Q][kBlock];
  Ti *sx = reinterpret_cast<Ti *>(stage);
  To *sy = reinterpret_cast<To *>(stage);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // tile = workgroup id (rows x tiles per row, row-major); MODE 2: the
  // row's tail, one past its last whole tile
  const long long tile = MODE == 2 ? (long long)blockIdx.x * tiles_per_row + tiles_per_row
                                   : (long long)blockIdx.x;
  const long long row = MODE == 2 ? (long long)blockIdx.x : tile / tiles_per_row;
  const long long t = tile - row * tiles_per_row;
  const long long base = t * kTile;
  const long long rem = len - base;
  const int n = rem < kTile ? (int)rem : kTile;
  const Ti *xr = x + row * len + base;
  To *yr = y + row * len + base;

  // The tile body is instantiated twice: FULL (a whole tile with 16-byte
  // aligned input and output: 128-bit loads and stores, no per-element
  // guards) and the guarded general case (a row's last tile, unaligned
  // views).  Only the first is on the streaming path.
  auto body = [&](auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    constexpr int VI = 16 / sizeof(Ti);
    constexpr int NV = kSubTile / VI / kBlock;  // 16-byte input vectors per thread per sub-tile
    auto count = [&](int q) {  // valid elements of sub-tile q
      if constexpr (FULL) return kSubTile;
      const int r = n - q * kSubTile;
      return r < 0 ? 0 : (r < kSubTile ? r : kSubTile);
    };

    // 1. inputs: all of the tile's 128-bit loads are issued first (a whole
    //    tile in flight per workgroup), then each sub-tile is redistributed
    //    through LDS so that a thread holds 16 consecutive elements
    u32x4 raw[FULL ? Q : 1][FULL ? NV : 1];
    if constexpr (FULL) {
      const u32x4 *xv = reinterpret_cast<const u32x4 *>(xr);
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int k = 0; k < NV; ++k)
          raw[q][k] = __builtin_nontemporal_load(xv + q * (kSubTile / VI) + k * kBlock + tid);
    }
    Ti xin[Q][kItems];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      if (q) __syncthreads();
      if constexpr (FULL) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          const int vi = k * kBlock + tid;
          union { u32x4 v; Ti e[VI]; } u;
          u.v = raw[q][k];
#pragma unroll
          for (int e = 0; e < VI; ++e) sx[padded(vi * VI + e)] = u.e[e];
        }
      } else {
        const int qn = count(q);
        for (int i = tid; i < qn; i += kBlock) sx[padded(i)] = xr[q * kSubTile + i];
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kItems; ++j) {
        const int i = tid * kItems + j;
        xin[q][j] = (FULL || i < count(q)) ? sx[padded(i)] : (Ti)0;
      }
    }

    // 2. per-thread totals of each sub-tile, block scans across threads
    //    (wave64 shuffles, then the 4 wave totals through LDS)
    A excl[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      A run = S::ident();
#pragma unroll
      for (int j = 0; j < kItems; ++j)
        if (FULL || tid * kItems + j < count(q)) run = S::comb(run, S::map(xin[q][j]));
      A inc = run;
#pragma unroll
      for (int dd = 1; dd < 64; dd <<= 1) {
        const A o = shfl_up64(inc, dd);
        if (lane >= dd) inc = S::comb(o, inc);
      }
      A ex = shfl_up64(inc, 1);
      if (lane == 0) ex = S::ident();
      excl[q] = ex;
      if (lane == 63) wsum[q][wave] = inc;
    }
    __syncthreads();
    A total = S::ident();
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      A wpre = S::ident(), qtot = S::ident();
#pragma unroll
      for (int w = 0; w < kBlock / 64; ++w) {
        if (w < wave) wpre = S::comb(wpre, wsum[q][w]);
        qtot = S::comb(qtot, wsum[q][w]);
      }
      // prefix within the tile, parked in LDS (this thread's slot) so that
      // it holds no registers across the look-back
      s_excl[q][tid] = S::comb(total, S::comb(wpre, excl[q]));
      total = S::comb(total, qtot);
    }

    // 3. look-back (wave 0), prefix to every thread through LDS
    if constexpr (MODE == 2) {
      if (tid == 0) s_prefix = t > 0 ? tail_prefix<S>(sc, tile - 1, gen) : S::ident();
    } else if (wave == 0) {
      const A prefix = look_back<S, scan_look<Ti, To>(), Q>(sc, tile, t, total, gen, lane,
                                                            x + row * len, s_own, s_win);
      if (lane == 0) s_prefix = prefix;
    }
    __syncthreads();

    // 4. outputs per sub-tile through LDS, then coalesced stores
    constexpr int VO = 16 / sizeof(To);
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      const int qn = count(q);
      A run = S::comb(s_prefix, s_excl[q][tid]);
#pragma unroll
      for (int j = 0; j < kItems; ++j) {
        const int i = tid * kItems + j;
        if (FULL || i < qn) {
          run = S::comb(run, S::map(opaque(xin[q][j])));
          sy[padded(i)] = mmp_convert<To, A>(run);
        }
      }
      __syncthreads();
      if constexpr (FULL) {
        u32x4 *yv = reinterpret_cast<u32x4 *>(yr + q * kSubTile);
#pragma unroll
        for (int k = 0; k < kSubTile / VO / kBlock; ++k) {
          const int vi = k * kBlock + tid;
          union { u32x4 v; To e[VO]; } u;
#pragma unroll
          for (int e = 0; e < VO; ++e) u.e[e] = sy[padded(vi * VO + e)];
          __builtin_nontemporal_store(u.v, yv + vi);
        }
      } else {
        for (int i = tid; i < qn; i += kBlock) yr[q * kSubTile + i] = sy[padded(i)];
      }
      __syncthreads();
    }
  };

  if constexpr (MODE == 0)
    body(Bool<true>());
  else
    body(Bool<false>());
}

// Strided axis: one thread per column; the axis is cut into S chunks so
// that the launch fills the device.  Phase 1 writes each chunk's column
// totals; phase 2 starts every chunk from the combined totals of the chunks
// before it (in order) and scans it.  Traffic: input read twice, output
// written once.
constexpr int kColUnroll = 8;  // rows in flight per thread

template <int OP, typename Ti>
__global__ __launch_bounds__(kBlock) void k_scan_cols_part(const Ti *__restrict__ x,
                                                          typename ScanOp<OP, Ti>::A *__restrict__ part,
                                                          long long len, long long inner, int S) {
  typedef ScanOp<OP, Ti> Sc;
  const long long o = blockIdx.y;
  const int s = blockIdx.z;
  const long long c = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (c >= inner) return;
  const long long per = (len + S - 1) / S;
  const long long b0 = s * per;
  const long long b1 = b0 + per < len ? b0 + per : len;
  const Ti *p = x + o * len * inner + c;
  typename Sc::A acc = Sc::ident();
  long long l = b0;
  for (; l + kColUnroll <= b1; l += kColUnroll) {
    Ti q[kColUnroll];
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) q[u] = p[(l + u) * inner];
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) acc = Sc::comb(acc, Sc::map(q[u]));
  }
  for (; l < b1; ++l) acc = Sc::comb(acc, Sc::map(p[l * inner]));
  part[((long long)o * S + s) * inner + c] = acc;
}

template <int OP, typename Ti, typename To>
__global__ __launch_bounds__(kBlock) void k_scan_cols(const Ti *__restrict__ x, To *__restrict__ y,
                                                     const typename ScanOp<OP, Ti>::A *__restrict__ part,
                                                     long long len, long long inner, int S) {
  typedef ScanOp<OP, Ti> Sc;
  const long long o = blockIdx.y;
  const int s = blockIdx.z;
  const long long c = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (c >= inner) return;
  const long long per = (len + S - 1) / S;
  const long long b0 = s * per;
  const long long b1 = b0 + per < len ? b0 + per : len;
  typename Sc::A acc = Sc::ident();
  for (int k = 0; k < s; ++k) acc = Sc::comb(acc, part[((long long)o * S + k) * inner + c]);
  const long long off = o * len * inner + c;
  long long l = b0;
  for (; l + kColUnroll <= b1; l += kColUnroll) {
    Ti q[kColUnroll];
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) q[u] = x[off + (l + u) * inner];
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) {
      acc = Sc::comb(acc, Sc::map(q[u]));
      y[off + (l + u) * inner] = mmp_convert<To, typename Sc::A>(acc);
    }
  }
  for (; l < b1; ++l) {
    acc = Sc::comb(acc, Sc::map(x[off + l * inner]));
    y[off + l * inner] = mmp_convert<To, typename Sc::A>(acc);
  }
}

// Strided axis with 16-byte column vectors (input element of 2, 4 or 8
// bytes, inner extent a multiple of the vector, 16-byte aligned input and
// output): a thread owns VI = 16 / sizeof(Ti) adjacent columns, so a
// workgroup reads 256 x 16 bytes of every row and each lane keeps 16 bytes
// in flight per row.  Phase 1 writes the VI chunk totals, a carry pass turns
// each column's totals into exclusive prefixes in place, phase 2 rescans
// each chunk from its prefix.
template <typename Ti> constexpr int scan_col_vec() { return 16 / (int)sizeof(Ti); }

template <int OP, typename Ti>
__global__ __launch_bounds__(kBlock) void k_scan_cols_part_vec(
    const Ti *__restrict__ x, typename ScanOp<OP, Ti>::A *__restrict__ part, long long len,
    long long inner, int S) {
  typedef ScanOp<OP, Ti> Sc;
  typedef typename Sc::A A;
  constexpr int VI = scan_col_vec<Ti>();
  const long long o = blockIdx.y;
  const int s = blockIdx.z;
  const long long c = ((long long)blockIdx.x * kBlock + threadIdx.x) * VI;
  if (c >= inner) return;
  const long long per = (len + S - 1) / S;
  const long long b0 = s * per;
  const long long b1 = b0 + per < len ? b0 + per : len;
  const Ti *p = x + o * len * inner + c;
  A acc[VI];
#pragma unroll
  for (int e = 0; e < VI; ++e) acc[e] = Sc::ident();
  long long l = b0;
  for (; l + kColUnroll <= b1; l += kColUnroll) {
    u32x4 q[kColUnroll];
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) q[u] = *reinterpret_cast<const u32x4 *>(p + (l + u) * inner);
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) {
      union { u32x4 v; Ti e[VI]; } w;
      w.v = q[u];
#pragma unroll
      for (int e = 0; e < VI; ++e) acc[e] = Sc::comb(acc[e], Sc::map(w.e[e]));
    }
  }
  for (; l < b1; ++l) {
    union { u32x4 v; Ti e[VI]; } w;
    w.v = *reinterpret_cast<const u32x4 *>(p + l * inner);
#pragma unroll
    for (int e = 0; e < VI; ++e) acc[e] = Sc::comb(acc[e], Sc::map(w.e[e]));
  }
  A *dst = part + ((long long)o * S + s) * inner + c;
#pragma unroll
  for (int e = 0; e < VI; ++e) dst[e] = acc[e];
}

// Chunk totals -> exclusive chunk prefixes, per column, in place.
template <int OP, typename Ti>
__global__ __launch_bounds__(kBlock) void k_scan_cols_carry(typename ScanOp<OP, Ti>::A *__restrict__ part,
                                                           long long inner, int S) {
  typedef ScanOp<OP, Ti> Sc;
  typedef typename Sc::A A;
  const long long o = blockIdx.y;
  const long long c = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (c >= inner) return;
  A *p = part + (long long)o * S * inner + c;
  A run = Sc::ident();
  int k = 0;
  for (; k + 8 <= S; k += 8) {
    A v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(long long)(k + u) * inner];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      p[(long long)(k + u) * inner] = run;
      run = Sc::comb(run, v[u]);
    }
  }
  for (; k < S; ++k) {
    const A v = p[(long long)k * inner];
    p[(long long)k * inner] = run;
    run = Sc::comb(run, v);
  }
}

template <int OP, typename Ti, typename To>
__global__ __launch_bounds__(kBlock) void k_scan_cols_vec(const Ti *__restrict__ x, To *__restrict__ y,
                                                         const typename ScanOp<OP, Ti>::A *__restrict__ pre,
                                                         long long len, long long inner, int S) {
  typedef ScanOp<OP, Ti> Sc;
  typedef typename Sc::A A;
  constexpr int VI = scan_col_vec<Ti>();
  constexpr int VO = 16 / (int)sizeof(To);  // outputs per 16-byte store
  static_assert(VI % VO == 0, "a lane's outputs fill whole 16-byte stores");
  const long long o = blockIdx.y;
  const int s = blockIdx.z;
  const long long c = ((long long)blockIdx.x * kBlock + threadIdx.x) * VI;
  if (c >= inner) return;
  const long long per = (len + S - 1) / S;
  const long long b0 = s * per;
  const long long b1 = b0 + per < len ? b0 + per : len;
  A acc[VI];
#pragma unroll
  for (int e = 0; e < VI; ++e) acc[e] = pre ? pre[((long long)o * S + s) * inner + c + e] : Sc::ident();
  const long long off = o * len * inner + c;
  auto row = [&](const u32x4 &v, long long l) {
    union { u32x4 v; Ti e[VI]; } w;
    w.v = v;
    union { u32x4 v[VI / VO]; To e[VI]; } r;
#pragma unroll
    for (int e = 0; e < VI; ++e) {
      acc[e] = Sc::comb(acc[e], Sc::map(w.e[e]));
      r.e[e] = mmp_convert<To, A>(acc[e]);
    }
    u32x4 *dst = reinterpret_cast<u32x4 *>(y + off + l * inner);
#pragma unroll
    for (int k = 0; k < VI / VO; ++k) dst[k] = r.v[k];
  };
  long long l = b0;
  for (; l + kColUnroll <= b1; l += kColUnroll) {
    u32x4 q[kColUnroll];
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) q[u] = *reinterpret_cast<const u32x4 *>(x + off + (l + u) * inner);
#pragma unroll
    for (int u = 0; u < kColUnroll; ++u) row(q[u], l + u);
  }
  for (; l < b1; ++l) row(*reinterpret_cast<const u32x4 *>(x + off + l * inner), l);
}

template <int OP, typename Ti, typename To> constexpr bool scan_out_ok() {
  if (mmp_t<Ti>::is_float) return __is_same(Ti, To);
  if (mmp_t<Ti>::is_signed || mmp_t<Ti>::is_bool) return __is_same(To, mmp_i64);
  return __is_same(To, mmp_u64);
}

#ifndef MMP_SCAN_COL_TARGET
#define MMP_SCAN_COL_TARGET 512
#endif
// The column-vector strided scan: splits of the axis for about
// MMP_SCAN_COL_TARGET workgroups, each chunk at least 64 rows.
template <int OP, typename Ti, typename To>
int launch_scan_cols_vec(long long outer, long long len, long long inner, const void *x, void *y) {
  typedef typename ScanOp<OP, Ti>::A A;
  constexpr int VI = scan_col_vec<Ti>();
  const long long ncb = mmpi::ceil_div(inner / VI, kBlock);
  const long long want = (MMP_SCAN_COL_TARGET + outer * ncb - 1) / (outer * ncb);
  const long long maxs = len / 64 > 0 ? len / 64 : 1;
  long long S = want < maxs ? want : maxs;
  if (S < 1) S = 1;
  if (S > 256) S = 256;
  const dim3 grid((unsigned)ncb, (unsigned)outer, (unsigned)S);
  void *part = nullptr;
  if (S > 1) {
    if (int st = mmp_alloc((size_t)outer * S * inner * sizeof(A), &part)) return st;
    hipLaunchKernelGGL((k_scan_cols_part_vec<OP, Ti>), grid, dim3(kBlock), 0, mmpi::stream(),
                       (const Ti *)x, (A *)part, len, inner, (int)S);
    int st = mmpi::check_launch("mmp_scan(cols, totals)");
    if (!st) {
      hipLaunchKernelGGL((k_scan_cols_carry<OP, Ti>),
                         dim3((unsigned)mmpi::ceil_div(inner, kBlock), (unsigned)outer), dim3(kBlock), 0,
                         mmpi::stream(), (A *)part, inner, (int)S);
      st = mmpi::check_launch("mmp_scan(cols, carries)");
    }
    if (st) {
      (void)mmp_free(part);
      return st;
    }
  }
  hipLaunchKernelGGL((k_scan_cols_vec<OP, Ti, To>), grid, dim3(kBlock), 0, mmpi::stream(),
                     (const Ti *)x, (To *)y, (const A *)part, len, inner, (int)S);
  const int st = mmpi::check_launch("mmp_scan(cols)");
  if (part) (void)mmp_free(part);  // stream-ordered: reused only by later work
  return st;
}

template <int OP, typename Ti, typename To>
int launch_scan(long long outer, long long len, long long inner, const void *x, void *y) {
  if constexpr (!scan_out_ok<OP, Ti, To>()) {
    return mmpi::fail(MMP_E_UNSUPPORTED, "scan: unsupported output dtype");
  } else {
    typedef typename ScanOp<OP, Ti>::A A;
    {  // a tile may read its predecessors' inputs, so out must not overlap in
      const uintptr_t xb = (uintptr_t)x, yb = (uintptr_t)y;
      const uintptr_t xe = xb + (uintptr_t)(outer * len * inner) * sizeof(Ti);
      const uintptr_t ye = yb + (uintptr_t)(outer * len * inner) * sizeof(To);
      if (outer * len * inner > 0 && xb < ye && yb < xe)
        return mmpi::fail(MMP_E_ARG, "scan: output overlaps the input");
    }
    if (inner == 1) {
      constexpr long long kTile = (long long)sub_tiles<Ti>() * kSubTile;
      // streaming layout: every row starts 16-byte aligned in input and output
      const bool vec = ((uintptr_t)x & 15u) == 0 && ((uintptr_t)y & 15u) == 0 &&
                       (len * (long long)sizeof(Ti)) % 16 == 0 &&
                       (len * (long long)sizeof(To)) % 16 == 0;
      const long long tpr = vec ? len / kTile : mmpi::ceil_div(len, kTile);
      const long long ntiles = outer * tpr;
      if (ntiles > 0x7fffffffLL || outer > 0x7fffffffLL)
        return mmpi::fail(MMP_E_ARG, "scan too large");
      int st = MMP_OK;
      ScanScratch sc;
      sc.timeout = mmpi::wait_flags();
      sc.desc = (unsigned long long *)mmpi::scratch(mmpi::SCRATCH_SCAN_VALUES,
                                                      16ull * (ntiles > 0 ? ntiles : 1), &st);
      if (st) return st;
      const unsigned gen = mmpi::next_generation();
      const mmpi::WaitParams wp = mmpi::wait_params();
      sc.read_gen = (gen + wp.tag_offset) & 0x3fffffffu;
      // polls of a missing predecessor before summing it here: it normally
      // publishes within a few (its loads are in flight when we start)
      sc.spin_limit = wp.spin_limit < kPollsBeforeSum ? wp.spin_limit : kPollsBeforeSum;
      if (!vec) {
        hipLaunchKernelGGL((k_scan_rows<OP, Ti, To, 1>), dim3((unsigned)ntiles), dim3(kBlock), 0,
                           mmpi::stream(), (const Ti *)x, (To *)y, len, tpr, ntiles, sc, gen);
        return mmpi::check_launch("mmp_scan(rows)");
      }
      if (ntiles > 0) {
        hipLaunchKernelGGL((k_scan_rows<OP, Ti, To, 0>), dim3((unsigned)ntiles), dim3(kBlock), 0,
                           mmpi::stream(), (const Ti *)x, (To *)y, len, tpr, ntiles, sc, gen);
        if (int e = mmpi::check_launch("mmp_scan(rows)")) return e;
      }
      if (len % kTile) {
        hipLaunchKernelGGL((k_scan_rows<OP, Ti, To, 2>), dim3((unsigned)outer), dim3(kBlock), 0,
                           mmpi::stream(), (const Ti *)x, (To *)y, len, tpr, ntiles, sc, gen);
        return mmpi::check_launch("mmp_scan(row tails)");
      }
      return MMP_OK;
    }
    if (outer > 65535) return mmpi::fail(MMP_E_ARG, "strided scan: outer extent %lld > 65535", outer);
    if constexpr (sizeof(Ti) >= 2) {
      constexpr int VI = scan_col_vec<Ti>();
      if (inner % VI == 0 && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)y & 15u) == 0)
        return launch_scan_cols_vec<OP, Ti, To>(outer, len, inner, x, y);
    }
    const long long ncb = mmpi::ceil_div(inner, kBlock);
    long long want = (2048 + outer * ncb - 1) / (outer * ncb);
    long long maxs = len / 64 > 0 ? len / 64 : 1;
    int S = (int)(want < maxs ? want : maxs);
    if (S < 1) S = 1;
    if (S > 256) S = 256;
    const dim3 grid((unsigned)ncb, (unsigned)outer, (unsigned)S);
    void *part = nullptr;
    if (S > 1) {
      if (int st = mmp_alloc((size_t)outer * S * inner * sizeof(A), &part)) return st;
      hipLaunchKernelGGL((k_scan_cols_part<OP, Ti>), grid, dim3(kBlock), 0, mmpi::stream(),
                         (const Ti *)x, (A *)part, len, inner, S);
      if (int st = mmpi::check_launch("mmp_scan(cols, totals)")) {
        (void)mmp_free(part);
        return st;
      }
    }
    hipLaunchKernelGGL((k_scan_cols<OP, Ti, To>), grid, dim3(kBlock), 0, mmpi::stream(),
                       (const Ti *)x, (To *)y, (const A *)part, len, inner, S);
    const int st = mmpi::check_launch("mmp_scan(cols)");
    if (part) (void)mmp_free(part);  // stream-ordered: reused only by later work
    return st;
  }
}

template <int OP, typename Ti>
int scan_out(int out_dtype, long long outer, long long len, long long inner, const void *x, void *y) {
  switch (out_dtype) {
    case MMP_F32: return launch_scan<OP, Ti, float>(outer, len, inner, x, y);
    case MMP_F64: return launch_scan<OP, Ti, double>(outer, len, inner, x, y);
    case MMP_F16: return launch_scan<OP, Ti, mmp_half>(outer, len, inner, x, y);
    case MMP_I64: return launch_scan<OP, Ti, mmp_i64>(outer, len, inner, x, y);
    case MMP_U64: return launch_scan<OP, Ti, mmp_u64>(outer, len, inner, x, y);
    default: return mmpi::fail(MMP_E_UNSUPPORTED, "scan output dtype %d", out_dtype);
  }
}

}  // namespace

extern "C" int mmp_scan(int op, int dtype, int out_dtype, int64_t outer, int64_t len,
                        int64_t inner, const void *x, void *out) {
  if (int st = mmpi::ensure_init()) return st;
  if (outer < 0 || len < 0 || inner < 0) return mmpi::fail(MMP_E_ARG, "negative extent");
  if (outer * len * inner == 0) return MMP_OK;
  if (!x || !out) return mmpi::fail(MMP_E_ARG, "null pointer");
  std::lock_guard<std::mutex> lk(mmpi::launch_mutex());
  MMP_DISPATCH_ALL(dtype, {
    if (op == MMP_S_CUMSUM) return scan_out<MMP_S_CUMSUM, T>(out_dtype, outer, len, inner, x, out);
    if (op == MMP_S_CUMPROD) return scan_out<MMP_S_CUMPROD, T>(out_dtype, outer, len, inner, x, out);
    return mmpi::fail(MMP_E_ARG, "unknown scan op %d", op);
  })
}
