// scan.hip -- cumsum / cumprod.
//
// Replaces the reference's three-pass Metal scan (_kernels.py:1263-1360,
// driven by ndarray._prefix_scan ndarray.py:2068-2152): block-local serial
// scans, then ONE thread scanning all block totals, then a propagation pass.
//
// Here a contiguous scan (any number of rows of length len) is a single
// pass of decoupled look-back:
//  * workgroups take tile ids from an atomic counter in launch order, so a
//    tile only ever waits for tiles that are already running (AMD gives no
//    forward-progress guarantee to workgroups that have not started);
//  * a tile (16384 elements: 4 sub-tiles of 256 threads x 16 consecutive
//    elements) is staged through LDS with 128-bit loads into registers,
//    scanned serially per thread in the accumulator type, then across the
//    wave64 with shuffles and across the 4 waves through LDS;
//  * wave 0 publishes the tile aggregate, reads the 64 nearest
//    predecessors' descriptors at once and combines aggregates up to the
//    nearest inclusive prefix, then publishes its own inclusive prefix;
//  * descriptors carry a per-call generation tag, so they are never
//    cleared between calls; waits are bounded and a timeout is recorded
//    instead of hanging.
// Accumulators: int64 for integers (int32 -> int64 output as NumPy),
// float64 for floats (rounded once per output element).  HBM-bound:
// sizeof(in) + sizeof(out) bytes per element.
// Strided scans (inner > 1) run one thread per column, coalesced across
// columns.
#include "mmp_ops.h"
#include "mmp_internal.h"

namespace {

constexpr int kBlock = 256;
constexpr int kItems = 16;                // consecutive elements per thread per sub-tile
constexpr int kSubTile = kBlock * kItems; // 4096 elements staged through LDS at a time
constexpr int kPad = kSubTile / kItems;   // one pad word per thread row in LDS
constexpr long long kSpinLimit = 1ll << 26;
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
  unsigned *counter;          // tile ticket (left at 0 by the last tile)
  unsigned long long *desc;   // 2 words per tile
  unsigned *timeout;          // set to 1 if a look-back wait ran out
};

template <int OP, typename Ti, typename To>
__global__ __launch_bounds__(kBlock) void k_scan_rows(const Ti *__restrict__ x, To *__restrict__ y,
                                                     long long len, long long tiles_per_row,
                                                     long long ntiles, ScanScratch sc,
                                                     unsigned gen) {
  typedef ScanOp<OP, Ti> S;
  typedef typename S::A A;
  constexpr int Q = sub_tiles<Ti>();
  constexpr int kTile = Q * kSubTile;
  constexpr int kStage = (sizeof(Ti) > sizeof(To) ? sizeof(Ti) : sizeof(To));
  __shared__ __attribute__((aligned(16))) unsigned char stage[(kSubTile + kPad) * kStage];
  __shared__ A wsum[Q][kBlock / 64];
  __shared__ A s_prefix;
  __shared__ unsigned s_tile;
  Ti *sx = reinterpret_cast<Ti *>(stage);
  To *sy = reinterpret_cast<To *>(stage);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  if (tid == 0) {
    const unsigned t = __hip_atomic_fetch_add(sc.counter, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
    s_tile = t;
    // every other workgroup has already drawn its id: re-arm for the next call
    if ((long long)t == ntiles - 1)
      __hip_atomic_store(sc.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const long long tile = s_tile;
  const long long row = tile / tiles_per_row;
  const long long t = tile - row * tiles_per_row;
  const long long base = t * kTile;
  const long long rem = len - base;
  const int n = rem < kTile ? (int)rem : kTile;
  const Ti *xr = x + row * len + base;
  To *yr = y + row * len + base;

  // 1. stage each sub-tile through LDS (128-bit loads when whole and
  //    aligned); each thread keeps its 16 consecutive inputs in registers
  constexpr int VI = 16 / sizeof(Ti);
  Ti xin[Q][kItems];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int qb = q * kSubTile;
    const int qn = n - qb < 0 ? 0 : (n - qb < kSubTile ? n - qb : kSubTile);
    if (q) __syncthreads();
    if (qn == kSubTile && ((uintptr_t)(xr + qb) & 15u) == 0) {
      const u32x4 *xv = reinterpret_cast<const u32x4 *>(xr + qb);
#pragma unroll
      for (int k = 0; k < kSubTile / VI / kBlock; ++k) {
        const int vi = k * kBlock + tid;
        union { u32x4 v; Ti e[VI]; } u;
        u.v = __builtin_nontemporal_load(xv + vi);
#pragma unroll
        for (int e = 0; e < VI; ++e) sx[padded(vi * VI + e)] = u.e[e];
      }
    } else {
      for (int i = tid; i < qn; i += kBlock) sx[padded(i)] = xr[qb + i];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
      const int i = tid * kItems + j;
      xin[q][j] = i < qn ? sx[padded(i)] : (Ti)0;
    }
  }

  // 2. per-thread totals of each sub-tile, block scans across threads
  //    (wave64 shuffles, then the 4 wave totals through LDS)
  A excl[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int qn = n - q * kSubTile;
    A run = S::ident();
#pragma unroll
    for (int j = 0; j < kItems; ++j)
      if (tid * kItems + j < qn) run = S::comb(run, S::map(xin[q][j]));
    A inc = run;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const A o = shfl_up64(inc, d);
      if (lane >= d) inc = S::comb(o, inc);
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
    excl[q] = S::comb(total, S::comb(wpre, excl[q]));  // prefix within the tile
    total = S::comb(total, qtot);
  }

  // 3. decoupled look-back by wave 0: its 64 lanes read the descriptors of
  //    the 64 nearest predecessors at once (lane 0 = tile - 1).  The window
  //    is usable when every lane nearer than the nearest inclusive prefix
  //    holds a valid aggregate; otherwise it is re-read (bounded).  Tiles
  //    before the row's first tile count as an inclusive identity.
  if (wave == 0) {
    A prefix = S::ident();
    unsigned long long *d = sc.desc;
    if (t > 0) {
      if (lane == 0) publish(d + 2 * tile, total, (gen << 2) | 1u);
      const long long first = tile - t;  // first tile of this row
      long long top = tile - 1;
      long long spins = 0;
      while (true) {
        const long long j = top - lane;
        unsigned state = 2u;
        A val = S::ident();
        if (j >= first) {
          const unsigned long long w0 = __hip_atomic_load(d + 2 * j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const unsigned long long w1 = __hip_atomic_load(d + 2 * j + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const unsigned t0 = (unsigned)(w0 >> 32), t1 = (unsigned)(w1 >> 32);
          state = (t0 == t1 && (t0 >> 2) == gen) ? (t0 & 3u) : 0u;
          val = __builtin_bit_cast(A, (w0 & 0xffffffffull) | (w1 << 32));
        }
        const unsigned long long incl = __ballot(state == 2u);
        const unsigned long long bad = __ballot(state == 0u);
        const int p = incl ? __ffsll((long long)incl) - 1 : 64;  // nearest inclusive lane
        const unsigned long long nearer = p >= 63 ? ~0ull : ((1ull << (p + 1)) - 1);
        if (bad & nearer) {
          if (++spins > kSpinLimit) {
            if (lane == 0) __hip_atomic_store(sc.timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          continue;
        }
        A part = lane <= p ? val : S::ident();
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) part = S::comb(part, shfl_xor64(part, m));
        prefix = S::comb(part, prefix);
        if (p < 64) break;
        top -= 64;
      }
    }
    if (lane == 0) {
      publish(d + 2 * tile, S::comb(prefix, total), (gen << 2) | 2u);
      s_prefix = prefix;
    }
  }
  __syncthreads();

  // 4. outputs per sub-tile through LDS, then coalesced stores
  constexpr int VO = 16 / sizeof(To);
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int qb = q * kSubTile;
    const int qn = n - qb < 0 ? 0 : (n - qb < kSubTile ? n - qb : kSubTile);
    A run = S::comb(s_prefix, excl[q]);
#pragma unroll
    for (int j = 0; j < kItems; ++j) {
      const int i = tid * kItems + j;
      if (i < qn) {
        run = S::comb(run, S::map(xin[q][j]));
        sy[padded(i)] = mmp_convert<To, A>(run);
      }
    }
    __syncthreads();
    if (qn == kSubTile && ((uintptr_t)(yr + qb) & 15u) == 0) {
      u32x4 *yv = reinterpret_cast<u32x4 *>(yr + qb);
#pragma unroll
      for (int k = 0; k < kSubTile / VO / kBlock; ++k) {
        const int vi = k * kBlock + tid;
        union { u32x4 v; To e[VO]; } u;
#pragma unroll
        for (int e = 0; e < VO; ++e) u.e[e] = sy[padded(vi * VO + e)];
        __builtin_nontemporal_store(u.v, yv + vi);
      }
    } else {
      for (int i = tid; i < qn; i += kBlock) yr[qb + i] = sy[padded(i)];
    }
    __syncthreads();
  }
}

// Strided axis: one thread per column, serial along the axis.
template <int OP, typename Ti, typename To>
__global__ __launch_bounds__(kBlock) void k_scan_cols(const Ti *__restrict__ x, To *__restrict__ y,
                                                     long long len, long long inner) {
  typedef ScanOp<OP, Ti> S;
  const long long o = blockIdx.y;
  const long long c = (long long)blockIdx.x * kBlock + threadIdx.x;
  if (c >= inner) return;
  const long long off = o * len * inner + c;
  typename S::A acc = S::ident();
  for (long long l = 0; l < len; ++l) {
    acc = S::comb(acc, S::map(x[off + l * inner]));
    y[off + l * inner] = mmp_convert<To, typename S::A>(acc);
  }
}

template <int OP, typename Ti, typename To> constexpr bool scan_out_ok() {
  if (mmp_t<Ti>::is_float) return __is_same(Ti, To);
  if (mmp_t<Ti>::is_signed || mmp_t<Ti>::is_bool) return __is_same(To, mmp_i64);
  return __is_same(To, mmp_u64);
}

template <int OP, typename Ti, typename To>
int launch_scan(long long outer, long long len, long long inner, const void *x, void *y) {
  if constexpr (!scan_out_ok<OP, Ti, To>()) {
    return mmpi::fail(MMP_E_UNSUPPORTED, "scan: unsupported output dtype");
  } else {
    typedef typename ScanOp<OP, Ti>::A A;
    if (inner == 1) {
      const long long tpr = mmpi::ceil_div(len, (long long)sub_tiles<Ti>() * kSubTile);
      const long long ntiles = outer * tpr;
      if (ntiles > 0x7fffffffLL) return mmpi::fail(MMP_E_ARG, "scan too large");
      int st = MMP_OK;
      ScanScratch sc;
      sc.counter = (unsigned *)mmpi::scratch(mmpi::SCRATCH_SCAN_COUNTER, 64, &st);
      if (st) return st;
      sc.timeout = sc.counter + 1;
      sc.desc = (unsigned long long *)mmpi::scratch(mmpi::SCRATCH_SCAN_VALUES, 16ull * ntiles, &st);
      if (st) return st;
      const unsigned gen = mmpi::next_generation();
      hipLaunchKernelGGL((k_scan_rows<OP, Ti, To>), dim3((unsigned)ntiles), dim3(kBlock), 0,
                         mmpi::stream(), (const Ti *)x, (To *)y, len, tpr, ntiles, sc, gen);
      return mmpi::check_launch("mmp_scan(rows)");
    }
    if (outer > 65535) return mmpi::fail(MMP_E_ARG, "strided scan: outer extent %lld > 65535", outer);
    hipLaunchKernelGGL((k_scan_cols<OP, Ti, To>),
                       dim3((unsigned)mmpi::ceil_div(inner, kBlock), (unsigned)outer), dim3(kBlock),
                       0, mmpi::stream(), (const Ti *)x, (To *)y, len, inner);
    return mmpi::check_launch("mmp_scan(cols)");
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
  MMP_DISPATCH_ALL(dtype, {
    if (op == MMP_S_CUMSUM) return scan_out<MMP_S_CUMSUM, T>(out_dtype, outer, len, inner, x, out);
    if (op == MMP_S_CUMPROD) return scan_out<MMP_S_CUMPROD, T>(out_dtype, outer, len, inner, x, out);
    return mmpi::fail(MMP_E_ARG, "unknown scan op %d", op);
  })
}
