// matmul.hip -- C[b] = A[b] @ B[b] on MFMA (gfx950).
//
// Replaces the reference's naive Metal matmul_op (_kernels.py:740-759: one
// thread per output, no tiling, float16 accumulating in half) and the CPU
// np.matmul it uses for batched products (linalg_top.py:105-106).
//
// Row-major operands: A (M, K) row stride lda, B (K, N) row stride ldb,
// C (M, N) row stride ldc; batch strides sA, sB, sC (0 broadcasts).
//
// Floating kernels: a 128 x 128 output tile per 256-thread workgroup, four
// wave64s in a 2 x 2 arrangement, each owning 64 x 64 = 4 x 4 MFMA 16x16
// tiles (64 fp32 accumulators per lane).  K advances in 128-byte slabs
// (BK = 64 halves / 32 floats / 16 doubles) through two LDS buffers: the
// next slab is fetched into registers while the current one feeds the
// MFMAs, then written to the other buffer (one barrier per slab).
//  * float16 / bfloat16: v_mfma_f32_16x16x32_{f16,bf16}.  A lane's operand
//    is 8 consecutive k of one row (A) or one column (B), so both LDS tiles
//    are k-contiguous; B arrives n-contiguous from HBM and is transposed in
//    registers (each thread owns an 8(k) x 4(n) block) before the LDS store.
//    Accumulation in fp32 (the reference accumulates float16 in half).
//    Products with 256-divisible extents, 16-byte aligned rows and at least
//    128 output tiles of 256 x 256 use k_gemm16_dma instead (256 x 256
//    tiles, operands copied global -> LDS without passing through VGPRs).
//  * float32 / float64: v_mfma_f32_16x16x4f32 / v_mfma_f64_16x16x4f64.  The
//    k slot a lane feeds is permuted (MFMA step t, lane group g consumes
//    k = KG*g + t), so a lane's A values for a whole slab are contiguous in
//    LDS and B keeps its natural n-contiguous layout.  float32 products with
//    128-divisible extents and 16-byte aligned rows copy operands global ->
//    LDS into swizzled stages: k_gemm4_dma3 (256 x 128 tiles, persistent,
//    three stages) when the tiles fill whole rounds of the CUs, else
//    k_gemm4_dma (128 x 128 tiles).
// Partial tiles and unaligned operands use guarded scalar loads (zero fill)
// and guarded stores.  Integer matmul: LDS-tiled exact kernel with
// wrap-around arithmetic (NumPy's integer matmul wraps).
#include "mmp_ops.h"
#include "mmp_internal.h"

namespace {

constexpr int kBlock = 256;
constexpr int BM = 128, BN = 128;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef double d4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------- 16-bit inputs
template <typename T> struct Half16;
template <> struct Half16<mmp_half> {
  typedef h8 vec;
  static __device__ __forceinline__ f4 mfma(vec a, vec b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Half16<__bf16> {
  typedef b8 vec;
  static __device__ __forceinline__ f4 mfma(vec a, vec b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <typename T> __device__ __forceinline__ T from_f32(float v) {
  if constexpr (sizeof(T) == 2 && !__is_same(T, mmp_half)) {
    return (T)v;  // bfloat16 (round to nearest even)
  } else {
    return (T)v;
  }
}

template <typename T, bool EDGE>
__global__ __launch_bounds__(kBlock, 2) void k_gemm16(const T *__restrict__ A,
                                                     const T *__restrict__ B, T *__restrict__ C,
                                                     int M, int N, int K, long long lda,
                                                     long long ldb, long long ldc, long long sA,
                                                     long long sB, long long sC, int tiles_n) {
  constexpr int BK = 64, LDK = BK + 8;
  typedef typename Half16<T>::vec V;
  __shared__ __attribute__((aligned(16))) unsigned short As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) unsigned short Bs[2][BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  const long long bz = blockIdx.y;
  const int m0 = tm * BM, n0 = tn * BN;
  const unsigned short *Ag = reinterpret_cast<const unsigned short *>(A + bz * sA);
  const unsigned short *Bg = reinterpret_cast<const unsigned short *>(B + bz * sB);

  // register staging: A 4 x 16B (rows tid/8 + 32p, k-vector tid%8);
  // B 8 x 8B (k rows 8*(tid/32) + kk, n columns 4*(tid%32) .. +3)
  u32x4 ra[4];
  u32x2 rb[8];
  const int a_row = tid >> 3, a_kv = tid & 7;
  const int b_k8 = tid >> 5, b_n4 = tid & 31;

  auto load = [&](int k0) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int r = m0 + a_row + 32 * p, k = k0 + a_kv * 8;
      if constexpr (!EDGE) {
        ra[p] = *reinterpret_cast<const u32x4 *>(Ag + (long long)r * lda + k);
      } else {
        unsigned short h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          h[e] = (r < M && k + e < K) ? Ag[(long long)r * lda + k + e] : (unsigned short)0;
        ra[p] = u32x4{h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16),
                      h[4] | ((unsigned)h[5] << 16), h[6] | ((unsigned)h[7] << 16)};
      }
    }
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
      const int k = k0 + b_k8 * 8 + kk, n = n0 + b_n4 * 4;
      if constexpr (!EDGE) {
        rb[kk] = *reinterpret_cast<const u32x2 *>(Bg + (long long)k * ldb + n);
      } else {
        unsigned short h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          h[e] = (k < K && n + e < N) ? Bg[(long long)k * ldb + n + e] : (unsigned short)0;
        rb[kk] = u32x2{h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16)};
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
      *reinterpret_cast<u32x4 *>(&As[buf][(a_row + 32 * p) * LDK + a_kv * 8]) = ra[p];
    // transpose the 8(k) x 4(n) block: column c gathers half c of each row
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      unsigned w[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const unsigned lo = rb[2 * d][c >> 1], hi = rb[2 * d + 1][c >> 1];
        w[d] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
      }
      *reinterpret_cast<u32x4 *>(&Bs[buf][(b_n4 * 4 + c) * LDK + b_k8 * 8]) =
          u32x4{w[0], w[1], w[2], w[3]};
    }
  };

  f4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int nk = (K + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * BK);
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      V af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const V *>(&As[cur][(wm * 64 + i * 16 + fr) * LDK + s * 32 + fk]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = *reinterpret_cast<const V *>(&Bs[cur][(wn * 64 + j * 16 + fr) * LDK + s * 32 + fk]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Half16<T>::mfma(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < nk) store(cur ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds rows 4*(lane/16)+r, column lane%16 of each tile
  T *Cb = C + bz * sC;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + r;
        const int col = n0 + wn * 64 + j * 16 + fr;
        if (!EDGE || (row < M && col < N)) Cb[(long long)row * ldc + col] = from_f32<T>(acc[i][j][r]);
      }
}

// ---------------------------- 16-bit inputs, large tiles, global -> LDS DMA
// 256 x 256 output tile per workgroup for operands whose extents divide
// the tile and whose rows are 16-byte aligned.  Eight waves (2 x 4, two per
// SIMD), each owning a 128 x 64 sub-tile with its 128 fp32 accumulators in
// VGPRs; one workgroup per CU.  Per 64-deep k slab a workgroup moves 64 KiB
// L2 -> LDS for 256 x 256 x 64 MACs.  Every operand byte goes HBM/L2 -> LDS
// with global_load_lds_dwordx4 (lane L of a wave's load lands at 16 B x L of
// the destination), so there is no register staging, no ds_write and no
// register transposition:
//  * Loading: waves 0-3 fill B, waves 4-7 fill A, eight 1 KiB loads per
//    wave per slab.
//  * A stage: 256 rows x 128 B (k-contiguous, as in HBM), 16-byte chunk c
//    of row r at c ^ ((r >> 1) & 7); a load instruction fills 8 rows, each
//    lane fetching the global chunk that belongs at its landing slot.
//  * B stage: 64 k-rows x 512 B (n-contiguous, as in HBM), 16-byte chunk c
//    of row k at c ^ fb(k), fb(k) = 2 * ((k & 3) | ((k >> 3) & 3) << 2), so
//    that the 16 rows one transposed read touches fall in distinct 32 B
//    slots.  B fragments come from ds_read_b64_tr_b16 (measured on gfx950:
//    within each 16-lane group, result element j of lane 4a + b is element
//    b of the 8 bytes addressed by lane a + 4j): two reads give a lane the
//    8 consecutive k of one column that the MFMA operand needs.  Both
//    layouts read without LDS bank conflicts (SQ_LDS_BANK_CONFLICT = 0).
//  * Two stages as separate LDS arrays, k loop unrolled by two, so the
//    compiler can tell that the MFMA reads of one stage never alias the
//    loads in flight into the other; slab kt + 1 is loaded while slab kt
//    runs, and the barrier in the middle of each slab waits for this
//    wave's loads (vmcnt) before publishing the stage.  LDS reads run one
//    half-slab ahead of the MFMAs, across the barrier.
//  * The MFMA is issued as C^T = B^T A^T (operands swapped), so a lane's
//    four accumulators are four consecutive columns of one C row: the
//    epilogue writes 8 B per lane per 16 x 16 tile.
//  * Workgroup ids are remapped so that the tiles one XCD runs together
//    (ids are dealt round-robin over the eight XCDs) form 4-row groups:
//    concurrent workgroups on an XCD share A and B panels in its L2.
// Measured at 8192^3 float16 on MI355X: 1.21-1.24 PF/s (0.89-0.91 ms);
// torch.matmul (hipBLASLt) on the same device 1.22 PF/s.  Register-staged loading
// (global -> VGPR -> ds_write, B transposed with v_perm) reached 0.88 PF/s;
// a four-stage 32-deep variant of this kernel 1.10 PF/s (twice the
// barriers).
typedef short s16x4 __attribute__((ext_vector_type(4)));

template <typename T>
__global__ __launch_bounds__(512, 1) void k_gemm16_dma(
    const T *__restrict__ A, const T *__restrict__ B, T *__restrict__ C, int M, int N, int K,
    long long lda, long long ldb, long long ldc, long long sA, long long sB, long long sC,
    int tiles_m, int tiles_n) {
  constexpr int WN = 4, TB = 256, BK = 64;
  constexpr int TM = 128, TN = 64, I = TM / 16, J = TN / 16;
  typedef typename Half16<T>::vec V;
  __shared__ __attribute__((aligned(16))) unsigned short As0[TB * BK], As1[TB * BK];
  __shared__ __attribute__((aligned(16))) unsigned short Bs0[BK * TB], Bs1[BK * TB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  const int nblk = tiles_m * tiles_n;
  int b = blockIdx.x;
  if ((nblk & 7) == 0) b = (b & 7) * (nblk >> 3) + (b >> 3);
  constexpr int GM = 4;
  const int group = b / (GM * tiles_n), first_m = group * GM;
  const int gm = min(tiles_m - first_m, GM);
  const int rem = b - group * GM * tiles_n;
  const int tm = first_m + rem % gm, tn = rem / gm;

  const long long bz = blockIdx.y;
  const int m0 = tm * TB, n0 = tn * TB;
  const unsigned short *Ag = reinterpret_cast<const unsigned short *>(A + bz * sA) +
                             (long long)m0 * lda;
  const unsigned short *Bg = reinterpret_cast<const unsigned short *>(B + bz * sB) + n0;

  auto swz = [](int r) { return (r >> 1) & 7; };
  auto fb = [](int k) { return 2 * ((k & 3) | (((k >> 3) & 3) << 2)); };

  // Loads: waves 0-3 fill B (each wave 8 instructions x 2 rows of 512 B),
  // waves 4-7 fill A (each wave 8 instructions x 8 rows of 128 B).  The
  // XOR swizzle of instruction p depends on p only through (p & 1) for A
  // and (p & 1, p >> 2) for B, so a lane keeps 4 per-lane offsets (32-bit:
  // the host keeps lda and ldb below 2^28) and the rest is wave-uniform.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int w4 = wv & 3;
  const bool b_role = wv < 4;
  unsigned loff[4];
  if (b_role) {
    const int h = lane >> 5, slot = lane & 31;  // row 16 w4 + 2p + h
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int f = 2 * ((2 * (v & 1) + h) | (((2 * w4 + (v >> 1)) & 3) << 2));  // fb(row)
      loff[v] = (unsigned)h * (unsigned)ldb + (unsigned)((slot ^ f) * 8);
    }
  } else {
    const int l3 = lane >> 3, slot = lane & 7;  // row 64 w4 + 8p + l3
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int sw = (4 * (v & 1) + (lane >> 4)) & 7;  // swz(row); entries 2, 3 repeat 0, 1
      loff[v] = (unsigned)l3 * (unsigned)lda + (unsigned)((slot ^ sw) * 8);
    }
  }
  auto issue = [&](unsigned short *As_, unsigned short *Bs_, int k0) {
    // operands selected, one product: hipcc branches on the role when each
    // side has its own multiply, and the branch splits the copies' block
    const unsigned short *g = (b_role ? Bg : Ag) + (long long)k0 * (b_role ? ldb : 1LL);
    unsigned short *dst = b_role ? Bs_ : As_;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const long long sp = b_role ? (long long)(16 * w4 + 2 * p) * ldb
                                  : (long long)(64 * w4 + 8 * p) * lda;
      const unsigned lo = loff[(p & 1) | ((p >> 2) << 1)];
      __builtin_amdgcn_global_load_lds(g + sp + lo, dst + (w4 * 8 + p) * 512, 16, 0, 0);
    }
  };

  f4 acc[I][J];
#pragma unroll
  for (int i = 0; i < I; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, grp = lane >> 4;
  const int fch[2] = {((grp + 0) ^ swz(fr)) * 8, ((grp + 4) ^ swz(fr)) * 8};
  // The fragments of one 32-deep half-slab: I A and J B fragments.
  auto read_half = [&](const unsigned short *As_, const unsigned short *Bs_, int s, V (&af)[I],
                       V (&bf)[J]) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      // lane (group grp, index q) addresses k row 32s + 8grp + q/4 (+4),
      // columns 4 (q % 4) .. +3 of the 16-column tile
      const int q = fr;
      const int col = wn * TN + j * 16 + 4 * (q & 3);
      const int k1 = s * 32 + grp * 8 + (q >> 2), k2 = k1 + 4;
      const int c8 = col >> 3, w = col & 7;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4 *)(Bs_ + k1 * TB + ((c8 ^ fb(k1)) << 3) + w));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4 *)(Bs_ + k2 * TB + ((c8 ^ fb(k2)) << 3) + w));
      typedef short s16x8 __attribute__((ext_vector_type(8)));
      const s16x8 v8 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      bf[j] = __builtin_bit_cast(V, v8);
    }
#pragma unroll
    for (int i = 0; i < I; ++i)
      af[i] = *reinterpret_cast<const V *>(&As_[(wm * TM + i * 16 + fr) * BK + fch[s]]);
  };
  auto mfma_half = [&](const V (&af)[I], const V (&bf)[J]) {
#pragma unroll
    for (int i = 0; i < I; ++i)
#pragma unroll
      for (int j = 0; j < J; ++j) acc[i][j] = Half16<T>::mfma(bf[j], af[i], acc[i][j]);
  };
  // A half-slab's 32 MFMAs with the 16 LDS reads of the next half-slab
  // placed one after each of the first 16 (the reads are done well before
  // the barrier or the MFMAs that need them).  The empty asm after each
  // half keeps those reads in the half (the compiler would otherwise sink
  // the reads of the next slab below the loop test, into a burst).
  auto sched_half = [&]() {
#pragma unroll
    for (int m = 0; m < 32; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      if (m < 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
  };

  // Pipeline: each 64-deep slab is two halves with one barrier between
  // them.  Before the barrier: MFMAs of the first half, reads of the second
  // half.  The barrier (which waits for this wave's copies) publishes the
  // other stage, so after it: the copy of the slab two ahead into the stage
  // just consumed, then MFMAs of the second half with the reads of the next
  // slab's first half.  Copies past the last slab reload the last slab into
  // a stage that is no longer read; reads past it read a stale stage and
  // are never used.  (1.17-1.18 -> 1.21-1.24 PF/s at 8192^3 over a single
  // read burst after each barrier.)
  const int nk = K / BK;
  V f0a[I], f0b[J], f1a[I], f1b[J];
  issue(As0, Bs0, 0);
  __syncthreads();
  issue(As1, Bs1, min(1, nk - 1) * BK);
  read_half(As0, Bs0, 0, f0a, f0b);
  for (int kt = 0; kt < nk; kt += 2) {
    // slab kt in stage 0
    mfma_half(f0a, f0b);
    read_half(As0, Bs0, 1, f1a, f1b);
    sched_half();
    asm volatile("" ::: "memory");
    __syncthreads();
    issue(As0, Bs0, min(kt + 2, nk - 1) * BK);
    mfma_half(f1a, f1b);
    read_half(As1, Bs1, 0, f0a, f0b);
    sched_half();
    asm volatile("" ::: "memory");
    if (kt + 1 < nk) {
      // slab kt + 1 in stage 1
      mfma_half(f0a, f0b);
      read_half(As1, Bs1, 1, f1a, f1b);
      sched_half();
      asm volatile("" ::: "memory");
      __syncthreads();
      issue(As1, Bs1, min(kt + 3, nk - 1) * BK);
      mfma_half(f1a, f1b);
      read_half(As0, Bs0, 0, f0a, f0b);
      sched_half();
      asm volatile("" ::: "memory");
    }
  }
  __syncthreads();  // no copy into LDS may be in flight when the workgroup ends

  T *Cb = C + bz * sC;
  const int cr = lane & 15, cc = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < I; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int row = m0 + wm * TM + i * 16 + cr;
      const int col = n0 + wn * TN + j * 16 + cc;
      unsigned short h[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) h[r] = __builtin_bit_cast(unsigned short, from_f32<T>(acc[i][j][r]));
      *reinterpret_cast<u32x2 *>(Cb + (long long)row * ldc + col) =
          u32x2{h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16)};
    }
}

// ------------------------------------------------------ fp32 / fp64
// Output element r of lane group g (= lane / 16) holds tile row
// 4*g + r for the fp32 MFMA but g + 4*r for the fp64 one (measured on
// gfx950 with a single-wave probe); the column is lane % 16 for both.
template <typename T> struct Mfma4;
template <> struct Mfma4<float> {
  typedef f4 acc_t;
  static __device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int out_row(int g, int r) { return 4 * g + r; }
};
template <> struct Mfma4<double> {
  typedef d4 acc_t;
  static __device__ __forceinline__ d4 mfma(double a, double b, d4 c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int out_row(int g, int r) { return g + 4 * r; }
};

template <typename T, bool EDGE>
__global__ __launch_bounds__(kBlock, 2) void k_gemm4(const T *__restrict__ A, const T *__restrict__ B,
                                                    T *__restrict__ C, int M, int N, int K,
                                                    long long lda, long long ldb, long long ldc,
                                                    long long sA, long long sB, long long sC,
                                                    int tiles_n) {
  constexpr int V = 16 / sizeof(T);        // elements per 16-byte vector
  constexpr int BK = 128 / sizeof(T);      // 32 floats / 16 doubles per slab
  constexpr int KG = BK / 4;               // k per lane group per slab
  constexpr int LDA = BK + V;              // padded A row (k-contiguous)
  constexpr int LDB = BN + V;              // padded B row (n-contiguous)
  constexpr int AV = BM * BK / V / kBlock; // A vectors per thread (4)
  constexpr int BV = BK * BN / V / kBlock; // B vectors per thread (4)
  typedef typename Mfma4<T>::acc_t ACC;
  __shared__ __attribute__((aligned(16))) T As[2][BM * LDA];
  __shared__ __attribute__((aligned(16))) T Bs[2][BK * LDB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  const long long bz = blockIdx.y;
  const int m0 = tm * BM, n0 = tn * BN;
  const T *Ag = A + bz * sA;
  const T *Bg = B + bz * sB;

  constexpr int A_VPR = BK / V;   // vectors per A row (8)
  constexpr int B_VPR = BN / V;   // vectors per B row (32 / 64)
  u32x4 ra[AV], rb[BV];

  auto load = [&](int k0) {
#pragma unroll
    for (int p = 0; p < AV; ++p) {
      const int idx = tid + p * kBlock;
      const int r = m0 + idx / A_VPR, k = k0 + (idx % A_VPR) * V;
      if constexpr (!EDGE) {
        ra[p] = *reinterpret_cast<const u32x4 *>(Ag + (long long)r * lda + k);
      } else {
        T h[V];
#pragma unroll
        for (int e = 0; e < V; ++e) h[e] = (r < M && k + e < K) ? Ag[(long long)r * lda + k + e] : (T)0;
        __builtin_memcpy(&ra[p], h, 16);
      }
    }
#pragma unroll
    for (int p = 0; p < BV; ++p) {
      const int idx = tid + p * kBlock;
      const int k = k0 + idx / B_VPR, n = n0 + (idx % B_VPR) * V;
      if constexpr (!EDGE) {
        rb[p] = *reinterpret_cast<const u32x4 *>(Bg + (long long)k * ldb + n);
      } else {
        T h[V];
#pragma unroll
        for (int e = 0; e < V; ++e) h[e] = (k < K && n + e < N) ? Bg[(long long)k * ldb + n + e] : (T)0;
        __builtin_memcpy(&rb[p], h, 16);
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int p = 0; p < AV; ++p) {
      const int idx = tid + p * kBlock;
      *reinterpret_cast<u32x4 *>(&As[buf][(idx / A_VPR) * LDA + (idx % A_VPR) * V]) = ra[p];
    }
#pragma unroll
    for (int p = 0; p < BV; ++p) {
      const int idx = tid + p * kBlock;
      *reinterpret_cast<u32x4 *>(&Bs[buf][(idx / B_VPR) * LDB + (idx % B_VPR) * V]) = rb[p];
    }
  };

  ACC acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = ACC{0, 0, 0, 0};

  const int nk = (K + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();
  const int fr = lane & 15, g = lane >> 4;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * BK);
    T af[4][KG], bf[4][KG];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const T *src = &As[cur][(wm * 64 + i * 16 + fr) * LDA + g * KG];
#pragma unroll
      for (int t = 0; t < KG; t += V)
        *reinterpret_cast<u32x4 *>(&af[i][t]) = *reinterpret_cast<const u32x4 *>(src + t);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < KG; ++t) bf[j][t] = Bs[cur][(g * KG + t) * LDB + wn * 64 + j * 16 + fr];
#pragma unroll
    for (int t = 0; t < KG; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = Mfma4<T>::mfma(af[i][t], bf[j][t], acc[i][j]);
    if (kt + 1 < nk) store(cur ^ 1);
    __syncthreads();
  }

  T *Cb = C + bz * sC;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + Mfma4<T>::out_row(g, r);
        const int col = n0 + wn * 64 + j * 16 + fr;
        if (!EDGE || (row < M && col < N)) Cb[(long long)row * ldc + col] = acc[i][j][r];
      }
}

// ------------------------------------------- float32, global -> LDS DMA
// 128 x 128 output tile per workgroup of four waves (two along M, two
// along N, each 64 x 64 = 4 x 4 MFMA tiles of v_mfma_f32_16x16x4f32; two
// workgroups per CU) for operands whose extents divide the tile and the
// 32-float slab and whose rows are 16-byte aligned, where the 256 x 128
// kernel below does not fill the CUs.  Operands are copied HBM/L2 -> LDS
// with global_load_lds_dwordx4 (lane L of a wave's copy lands at 16 B x L
// of its destination): no register staging, no ds_write.  Two LDS stages;
// waves 0-1 copy A (eight 1 KiB copies each per slab), waves 2-3 copy B.
// The MFMA's k slot is permuted as in k_gemm4 (lane group g feeds
// k = 8 g + t), so a lane's A values of a half-slab are one 16-byte chunk.
//  * A stage: 128 rows x 32 floats (128 B, k-contiguous as in HBM); chunk c
//    of row r sits at slot c ^ ((r >> 1) & 7), so the 16 rows of a fragment
//    read spread over all 64 banks.
//  * B stage: 32 k-rows x 128 floats (512 B, n-contiguous); chunk c of row
//    k sits at slot c ^ (4 ((k >> 3) & 3)), so the four lane groups of a
//    scalar fragment read (rows 8 apart) fall in different bank quarters.
//  * Pipeline as in k_gemm16_dma: one barrier per slab (it waits for this
//    wave's copies), the copy of the slab two ahead issued right after it
//    into the stage just consumed, fragment reads half a slab ahead of the
//    MFMAs.
__global__ __launch_bounds__(256, 2) void k_gemm4_dma(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int M, int N,
    int K, long long lda, long long ldb, long long ldc, long long sA, long long sB, long long sC,
    int tiles_n) {
  constexpr int WM = 2, BK = 32, TM = 64 * WM;  // tile rows: WM waves of 64 rows along M
  __shared__ __attribute__((aligned(16))) float As0[TM * BK], As1[TM * BK];
  __shared__ __attribute__((aligned(16))) float Bs0[BK * BN], Bs1[BK * BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  const long long bz = blockIdx.y;
  const int m0 = tm * TM, n0 = tn * BN;
  const float *Ag = A + bz * sA + (long long)m0 * lda;
  const float *Bg = B + bz * sB + n0;

  // Copies.  Wave w copies q = 8 (w & 1) + p, p = 0-7.  A: copy q fills
  // rows 8q .. 8q + 7, lane L row 8q + L/8, slot L % 8; its swizzle
  // (r >> 1) & 7 = ((L >> 4) + 4q) & 7 depends on q only through p & 1.
  // B: copy q fills k-rows 2q, 2q + 1, lane L row 2q + L/32, slot L % 32;
  // swizzle 4 ((q >> 2) & 3) = 4 (2 (w & 1) + (p >> 2)).  A lane keeps the
  // two offsets its copies use, indexed by the unrolled p (32-bit: the host
  // keeps lda and ldb below 2^28).
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const bool b_role = wv >= WM;  // the first WM waves copy A, the rest B
  const int w2 = b_role ? wv - WM : wv;
  unsigned loff[2];
  if (b_role) {
    const int h = lane >> 5, slot = lane & 31;
#pragma unroll
    for (int u = 0; u < 2; ++u)
      loff[u] = (unsigned)h * (unsigned)ldb + (unsigned)((slot ^ (4 * (2 * w2 + u))) * 4);
  } else {
    const int r8 = lane >> 3, slot = lane & 7;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int sw = ((lane >> 4) + 4 * u) & 7;
      loff[u] = (unsigned)r8 * (unsigned)lda + (unsigned)((slot ^ sw) * 4);
    }
  }
  // The role is selected, not branched on: a branch per copy splits the
  // block the copies and MFMAs share.
  auto issue = [&](float *As_, float *Bs_, int k0) {
    const float *base = b_role ? Bg + (long long)k0 * ldb : Ag + k0;
    const long long step = b_role ? 2 * ldb : 8 * lda;  // rows per copy
    float *dst = b_role ? Bs_ : As_;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int q = w2 * 8 + p;
      const unsigned lo = b_role ? loff[p >> 2] : loff[p & 1];
      __builtin_amdgcn_global_load_lds(base + q * step + lo, dst + q * 256, 16, 0, 0);
    }
  };

  f4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, g = lane >> 4;
  // Fragments of half-slab s (k = 8 g + 4 s .. + 3 of each lane group).
  auto read_half = [&](const float *As_, const float *Bs_, int s, f4 (&af)[4], f4 (&bf)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wm * 64 + i * 16 + fr;
      af[i] = *reinterpret_cast<const f4 *>(As_ + r * BK + (((2 * g + s) ^ ((r >> 1) & 7)) * 4));
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int k = g * 8 + s * 4 + t;
      const int sw = 4 * ((k >> 3) & 3);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = wn * 64 + j * 16 + fr;
        bf[j][t] = Bs_[k * BN + (((n >> 2) ^ sw) * 4) + (n & 3)];
      }
    }
  };
  auto mfma_half = [&](const f4 (&af)[4], const f4 (&bf)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][t], bf[j][t], acc[i][j], 0, 0, 0);
  };
  // A half-slab's 64 MFMAs with the next half-slab's LDS reads placed one
  // after each of the first 20 (4 A reads, 16 B reads).
  auto sched_half = [&]() {
#pragma unroll
    for (int m = 0; m < 64; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);             // MFMA
      if (m < 20) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
  };

  // As in k_gemm16_dma: before each slab's barrier the MFMAs of its first
  // half and the reads of its second half; after it the copy of the slab
  // two ahead, the MFMAs of the second half and the reads of the next
  // slab's first half.  Copies past the last slab reload the last slab
  // into a stage no longer read; reads past it are never used.
  const int nk = K / BK;
  f4 f0a[4], f0b[4], f1a[4], f1b[4];
  issue(As0, Bs0, 0);
  __syncthreads();
  issue(As1, Bs1, min(1, nk - 1) * BK);
  read_half(As0, Bs0, 0, f0a, f0b);
  for (int kt = 0; kt < nk; kt += 2) {
    mfma_half(f0a, f0b);
    read_half(As0, Bs0, 1, f1a, f1b);
    sched_half();
    asm volatile("" ::: "memory");
    __syncthreads();
    issue(As0, Bs0, min(kt + 2, nk - 1) * BK);
    mfma_half(f1a, f1b);
    read_half(As1, Bs1, 0, f0a, f0b);
    sched_half();
    asm volatile("" ::: "memory");
    if (kt + 1 < nk) {
      mfma_half(f0a, f0b);
      read_half(As1, Bs1, 1, f1a, f1b);
      sched_half();
      asm volatile("" ::: "memory");
      __syncthreads();
      issue(As1, Bs1, min(kt + 3, nk - 1) * BK);
      mfma_half(f1a, f1b);
      read_half(As0, Bs0, 0, f0a, f0b);
      sched_half();
      asm volatile("" ::: "memory");
    }
  }
  __syncthreads();  // no copy into LDS may be in flight when the workgroup ends

  float *Cb = C + bz * sC;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm * 64 + i * 16 + 4 * g + r;
        const int col = n0 + wn * 64 + j * 16 + fr;
        Cb[(long long)row * ldc + col] = acc[i][j][r];
      }
}

// 256 x 128 tiles with three LDS stages of 48 KiB (A's 256 x 32 floats,
// then B's 32 x 128), same layouts and swizzles as k_gemm4_dma.  A slab's
// 48 one-KiB copies (32 of A, 16 of B) are split six per wave, so every
// wave copies and none branches on its role inside the loop.
//
// Persistent: one workgroup per CU walks a list of tiles, and its slabs
// form one stream across them.  The copy of stream slab s + 3 is issued
// after the barrier that ends the reads of slab s, into that slab's stage,
// and waited for two slabs later: each barrier waits until at most this
// wave's six newest copies (slab s + 2) are in flight (vmcnt(6)), not for
// all of them.  So the next tile's first slabs are in flight while the
// current tile finishes, and a tile's C stores overlap the next tile's
// MFMAs; the barrier after a tile's stores waits for everything (vmcnt(0):
// stores and copies need not complete in issue order).  Copies past the
// last slab reload the last slab into a stage never read again, so every
// wave always has six copies per slab in flight and the count stays exact.
__global__ __launch_bounds__(512, 1) void k_gemm4_dma3(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int K,
    long long lda, long long ldb, long long ldc, long long sA, long long sB, long long sC,
    int tiles_n, int per_b, int T) {
  constexpr int BK = 32, TM = 256, AS = TM * BK, ST = AS + BK * BN;  // floats per stage
  __shared__ __attribute__((aligned(16))) float S0[ST], S1[ST], S2[ST];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // Tile order.  Workgroups are dispatched to the eight XCDs round-robin
  // (workgroup w to XCD w % 8); when the tile count and the grid divide by
  // 8, the workgroups of XCD x share the contiguous range x T/8 .. (x + 1)
  // T/8 - 1 of the order below, in turn, instead of every eighth tile.  The
  // order runs batch by batch and, within a batch, over groups of four tile
  // rows, column by column, so the 32 workgroups an XCD runs at a time
  // share their operand slabs in its L2 (a 4 x 8 block of one product, or
  // one whole product of a batch of small ones).
  const int P = gridDim.x, w = blockIdx.x;
  int tfirst, tstep, nt;
  if ((T & 7) == 0 && (P & 7) == 0) {
    const int q = T >> 3, ps = P >> 3, s = w >> 3;
    tfirst = (w & 7) * q + s;
    tstep = ps;
    nt = s < q ? (q - 1 - s) / ps + 1 : 0;
  } else {
    tfirst = w;
    tstep = P;
    nt = w < T ? (T - 1 - w) / P + 1 : 0;
  }
  if (nt == 0) return;  // the whole workgroup, before any barrier
  auto decode = [&](int i, long long &bz, int &m0, int &n0) {
    const int t = tfirst + i * tstep;
    bz = t / per_b;
    const int r = t - (int)bz * per_b;
    const int tiles_m = per_b / tiles_n;
    const int first = (r / (4 * tiles_n)) * 4, gsize = min(4, tiles_m - first);
    const int local = r - first * tiles_n;
    m0 = (first + local % gsize) * TM;
    n0 = (local / gsize) * BN;
  };

  // Copy c = 6 w + p lands at 1 KiB x c of a stage.  c < 32: rows 8c .. 8c
  // + 7 of A, lane L row 8c + L/8, slot L % 8 holding chunk slot ^ sw with
  // sw = ((L >> 4) + 4c) & 7.  c >= 32, q = c - 32: k-rows 2q, 2q + 1 of B,
  // lane L row 2q + L/32, slot L % 32 holding chunk slot ^ 4 ((q >> 2) & 3).
  // The wave-uniform part of each source (panel, row and slab offsets)
  // stays scalar; the lane part is a 32-bit byte offset (the host keeps lda
  // and ldb below 2^27, so 7 lda + 32 floats fit).
  //
  // The copies are written as instructions (scalar base + lane offset form;
  // M0 holds the LDS destination, and an LDS copy may not read M0 in the
  // cycle after it is written, hence the s_nop) rather than through the
  // compiler's builtin: the compiler cannot tell which stage an in-flight
  // copy writes across the loop's back edge and would wait for every copy
  // before the first LDS read of each pass.  The waits here are the
  // explicit ones.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  bool isA[6];
  long long off[6], ks[6];
  unsigned vo[6];
#pragma unroll
  for (int p = 0; p < 6; ++p) {
    const int c = wv * 6 + p;
    isA[p] = c < 32;
    if (c < 32) {
      off[p] = (long long)(8 * c) * lda;
      ks[p] = 1;
      const int sw = ((lane >> 4) + 4 * c) & 7;
      vo[p] = ((unsigned)(lane >> 3) * (unsigned)lda + (unsigned)(((lane & 7) ^ sw) * 4)) * 4u;
    } else {
      const int q = c - 32;
      off[p] = (long long)(2 * q) * ldb;
      ks[p] = ldb;
      const int sw = 4 * ((q >> 2) & 3);
      vo[p] = ((unsigned)(lane >> 5) * (unsigned)ldb + (unsigned)(((lane & 31) ^ sw) * 4)) * 4u;
    }
  }
  const int nk = K / BK;
  // The copy stream: tile ci of the list, its slab ck, and that tile's
  // operand panels.
  int ci = 0, ck = 0;
  const float *cA, *cB;
  auto copy_tile = [&]() {
    long long bz;
    int m0, n0;
    decode(ci, bz, m0, n0);
    cA = A + bz * sA + (long long)m0 * lda;
    cB = B + bz * sB + n0;
  };
  copy_tile();
  // src: this wave's six sources in the copy stream's next slab.  advance()
  // steps them one slab along k, or to the next tile's panels; after the
  // last slab of the last tile the stream stays on it.  It runs at the end
  // of a slab, beside the compute stream's tile-end branch: a branch inside
  // a half-slab splits its block, and the scheduler then cannot interleave
  // that half's LDS reads with its MFMAs (the first half's reads went after
  // all 64 of its MFMAs, then waited out their latency before the barrier:
  // 2-2.5 % of the kernel).
  const float *src[6];
  auto panel_sources = [&]() {
#pragma unroll
    for (int p = 0; p < 6; ++p) src[p] = (isA[p] ? cA : cB) + off[p];
  };
  panel_sources();
  auto advance = [&]() {
    if (ck + 1 < nk) {
      ++ck;
#pragma unroll
      for (int p = 0; p < 6; ++p) src[p] += BK * ks[p];
    } else if (ci + 1 < nt) {
      ++ci;
      ck = 0;
      copy_tile();
      panel_sources();
    }
  };
  auto issue = [&](float *S, const float *(&src)[6]) {
#pragma unroll
    for (int p = 0; p < 6; ++p) {
      const unsigned dst =
          (unsigned)(uintptr_t)(__attribute__((address_space(3))) float *)(S + (wv * 6 + p) * 256);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
      asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                   :
                   : "s"(dst), "v"(vo[p]), "s"(src[p])
                   : "memory", "m0");
#pragma clang diagnostic pop
    }
  };

  f4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, g = lane >> 4;
  auto read_half = [&](const float *S, int s, f4 (&af)[4], f4 (&bf)[4]) {
    const float *Bs_ = S + AS;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = wm * 64 + i * 16 + fr;
      af[i] = *reinterpret_cast<const f4 *>(S + r * BK + (((2 * g + s) ^ ((r >> 1) & 7)) * 4));
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int k = g * 8 + s * 4 + t;
      const int sw = 4 * ((k >> 3) & 3);
      // columns 4 fr .. 4 fr + 3 of the wave's 64: one 16-byte chunk
      const f4 v = *reinterpret_cast<const f4 *>(Bs_ + k * BN + (((wn * 16 + fr) ^ sw) * 4));
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j][t] = v[j];
    }
  };
  auto mfma_half = [&](const f4 (&af)[4], const f4 (&bf)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i][t], bf[j][t], acc[i][j], 0, 0, 0);
  };
  constexpr int kReads = 8;  // LDS reads of a half-slab's fragments (4 of A, 4 of B)
  auto sched_half = [&]() {
#pragma unroll
    for (int m = 0; m < 64; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // MFMA
      if (m < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
  };

  f4 f0a[4], f0b[4], f1a[4], f1b[4];
  issue(S0, src);
  advance();
  issue(S1, src);
  advance();
  issue(S2, src);
  advance();
  asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");  // slab 0 landed everywhere
  read_half(S0, 0, f0a, f0b);
  int kt = 0, ti = 0;  // the compute stream: slab kt of tile ti
  bool stored = false;  // C stores issued since the last barrier
  // One slab: the MFMAs of its first half with the reads of its second; a
  // barrier once the next slab has landed and every wave has read this one;
  // the copy three slabs ahead into this slab's stage; the second half's
  // MFMAs with the reads of the first half of the next slab; after a tile's
  // last slab, its C stores; the copy stream's next sources.
  auto slab = [&](float *cur, const float *nxt) {
    mfma_half(f0a, f0b);
    read_half(cur, 1, f1a, f1b);
    sched_half();
    __builtin_amdgcn_sched_barrier(0);  // the half's MFMAs stay ahead of the barrier
    if (stored)
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    stored = false;
    issue(cur, src);
    mfma_half(f1a, f1b);
    read_half(nxt, 0, f0a, f0b);
    sched_half();
    asm volatile("" ::: "memory");
    if (kt + 1 < nk) {
      ++kt;
    } else {
      long long bz;
      int m0, n0;
      decode(ti, bz, m0, n0);
      float *Cb = C + bz * sC;
      // lane fr holds columns 4 fr .. 4 fr + 3: one 16-byte store per row
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = m0 + wm * 64 + i * 16 + 4 * g + r;
          *reinterpret_cast<f4 *>(Cb + (long long)row * ldc + n0 + wn * 64 + 4 * fr) =
              f4{acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]};
        }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
      ++ti;
      kt = 0;
      stored = true;
    }
    advance();
  };
  const int total = nt * nk;
  for (int s = 0; s < total; s += 3) {
    slab(S0, S1);
    if (s + 1 < total) {
      slab(S1, S2);
      if (s + 2 < total) slab(S2, S0);
    }
  }
  // no copy into LDS may be in flight when the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
}

// ----------------------------------------------------------- integers
template <typename T>
__global__ __launch_bounds__(kBlock) void k_gemm_int(const T *__restrict__ A, const T *__restrict__ B,
                                                    T *__restrict__ C, int M, int N, int K,
                                                    long long lda, long long ldb, long long ldc,
                                                    long long sA, long long sB, long long sC,
                                                    int tiles_n) {
  constexpr int TS = 16;
  __shared__ T As[TS][TS + 1], Bs[TS][TS + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x - tm * tiles_n;
  const long long bz = blockIdx.y;
  const int row = tm * TS + ty, col = tn * TS + tx;
  const T *Ag = A + bz * sA;
  const T *Bg = B + bz * sB;
  T acc = 0;
  for (int k0 = 0; k0 < K; k0 += TS) {
    As[ty][tx] = (row < M && k0 + tx < K) ? Ag[(long long)row * lda + k0 + tx] : (T)0;
    Bs[ty][tx] = (k0 + ty < K && col < N) ? Bg[(long long)(k0 + ty) * ldb + col] : (T)0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < TS; ++k) acc = op_add(acc, op_multiply(As[ty][k], Bs[k][tx]));
    __syncthreads();
  }
  if (row < M && col < N) C[bz * sC + (long long)row * ldc + col] = acc;
}

// -------------------------------------------------------------- launch
inline bool al(const void *p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

// The 256 x 256 kernel is used once the product has at least
// MMP_GEMM16_BIG_MIN_TILES tiles (fewer leave CUs idle).
#ifndef MMP_GEMM16_BIG_MIN_TILES
#define MMP_GEMM16_BIG_MIN_TILES 128
#endif

template <typename T>
int launch16(long long batch, int M, int N, int K, const void *A, long long lda, long long sA,
             const void *B, long long ldb, long long sB, void *C, long long ldc, long long sC) {
  if (M % 256 == 0 && N % 256 == 0 && K % 64 == 0 && lda % 8 == 0 && ldb % 8 == 0 &&
      lda < (1ll << 28) && ldb < (1ll << 28) &&
      ldc % 4 == 0 && sA % 8 == 0 && sB % 8 == 0 && sC % 4 == 0 && al(A, 16) && al(B, 16) &&
      al(C, 8) && (long long)(M / 256) * (N / 256) * batch >= MMP_GEMM16_BIG_MIN_TILES) {
    const int tm = M / 256, tn = N / 256;
    hipLaunchKernelGGL((k_gemm16_dma<T>), dim3((unsigned)(tm * tn), (unsigned)batch), dim3(512), 0,
                       mmpi::stream(), (const T *)A, (const T *)B, (T *)C, M, N, K, lda, ldb,
                       ldc, sA, sB, sC, tm, tn);
    return mmpi::check_launch("mmp_matmul(mfma16 256x256)");
  }
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const bool fast = M % BM == 0 && N % BN == 0 && K % 64 == 0 && lda % 8 == 0 && ldb % 4 == 0 &&
                    sA % 8 == 0 && sB % 4 == 0 && al(A, 16) && al(B, 8);
  dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)batch);
  if (fast)
    hipLaunchKernelGGL((k_gemm16<T, false>), grid, dim3(kBlock), 0, mmpi::stream(), (const T *)A,
                       (const T *)B, (T *)C, M, N, K, lda, ldb, ldc, sA, sB, sC, tiles_n);
  else
    hipLaunchKernelGGL((k_gemm16<T, true>), grid, dim3(kBlock), 0, mmpi::stream(), (const T *)A,
                       (const T *)B, (T *)C, M, N, K, lda, ldb, ldc, sA, sB, sC, tiles_n);
  return mmpi::check_launch("mmp_matmul(mfma16)");
}

template <typename T>
int launch4(long long batch, int M, int N, int K, const void *A, long long lda, long long sA,
            const void *B, long long ldb, long long sB, void *C, long long ldc, long long sC) {
  constexpr int V = 16 / sizeof(T), BK = 128 / sizeof(T);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const bool fast = M % BM == 0 && N % BN == 0 && K % BK == 0 && lda % V == 0 && ldb % V == 0 &&
                    sA % V == 0 && sB % V == 0 && al(A, 16) && al(B, 16);
  dim3 grid((unsigned)(tiles_m * tiles_n), (unsigned)batch);
  if constexpr (__is_same(T, float)) {
    // the DMA kernel's per-lane copy offsets are 32-bit (7 lda + 28 floats)
    if (fast && lda < (1LL << 28) && ldb < (1LL << 28)) {
      // 256 x 128 tiles (one persistent workgroup per CU) when the tiles fill
      // whole rounds of the CUs, or nearly; otherwise 128 x 128 tiles, whose
      // finer grain leaves fewer CUs idle in the last round (2048^2: 128
      // wide tiles for 256 CUs; 6144^2: 4.5 rounds).
      const long long cus = mmpi::cu_count() > 0 ? mmpi::cu_count() : 256;
      const long long wide_tiles = M % 256 == 0 ? (long long)(M / 256) * tiles_n * batch : 0;
      const long long rounds = (wide_tiles + cus - 1) / cus;
      const bool c16 = al(C, 16) && ldc % 4 == 0 && sC % 4 == 0;  // 16-byte C rows
      if (wide_tiles > 0 && wide_tiles < (1LL << 30) && lda < (1LL << 27) && ldb < (1LL << 27) &&
          c16 && wide_tiles * 100 >= rounds * cus * 97) {
        const long long P = wide_tiles > cus ? cus : wide_tiles;
        hipLaunchKernelGGL(k_gemm4_dma3, dim3((unsigned)P), dim3(512), 0, mmpi::stream(),
                           (const float *)A, (const float *)B, (float *)C, K, lda, ldb, ldc, sA,
                           sB, sC, tiles_n, (int)((M / 256) * tiles_n), (int)wide_tiles);
      } else {
        hipLaunchKernelGGL(k_gemm4_dma, grid, dim3(kBlock), 0, mmpi::stream(),
                           (const float *)A, (const float *)B, (float *)C, M, N, K, lda, ldb, ldc,
                           sA, sB, sC, tiles_n);
      }
      return mmpi::check_launch("mmp_matmul(mfma4 dma)");
    }
  }
  if (fast)
    hipLaunchKernelGGL((k_gemm4<T, false>), grid, dim3(kBlock), 0, mmpi::stream(), (const T *)A,
                       (const T *)B, (T *)C, M, N, K, lda, ldb, ldc, sA, sB, sC, tiles_n);
  else
    hipLaunchKernelGGL((k_gemm4<T, true>), grid, dim3(kBlock), 0, mmpi::stream(), (const T *)A,
                       (const T *)B, (T *)C, M, N, K, lda, ldb, ldc, sA, sB, sC, tiles_n);
  return mmpi::check_launch("mmp_matmul(mfma4)");
}

template <typename T>
int launch_int(long long batch, int M, int N, int K, const void *A, long long lda, long long sA,
               const void *B, long long ldb, long long sB, void *C, long long ldc, long long sC) {
  const int tiles_m = (M + 15) / 16, tiles_n = (N + 15) / 16;
  hipLaunchKernelGGL((k_gemm_int<T>), dim3((unsigned)(tiles_m * tiles_n), (unsigned)batch),
                     dim3(kBlock), 0, mmpi::stream(), (const T *)A, (const T *)B, (T *)C, M, N, K,
                     lda, ldb, ldc, sA, sB, sC, tiles_n);
  return mmpi::check_launch("mmp_matmul(int)");
}

}  // namespace

extern "C" int mmp_matmul(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K, const void *A,
                          int64_t lda, int64_t sA, const void *B, int64_t ldb, int64_t sB, void *C,
                          int64_t ldc, int64_t sC) {
  if (int st = mmpi::ensure_init()) return st;
  if (batch < 0 || M < 0 || N < 0 || K < 0) return mmpi::fail(MMP_E_ARG, "negative extent");
  if (batch == 0 || M == 0 || N == 0) return MMP_OK;
  if (K == 0) return mmpi::fail(MMP_E_ARG, "K == 0: fill the output instead");
  if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff)
    return mmpi::fail(MMP_E_ARG, "matmul extent exceeds 2^31 - 1");
  if (batch > 65535) return mmpi::fail(MMP_E_ARG, "batch %lld > 65535", (long long)batch);
  if (!A || !B || !C) return mmpi::fail(MMP_E_ARG, "null pointer");
  if (lda < K || ldb < N || ldc < N) return mmpi::fail(MMP_E_ARG, "leading dimension too small");
  const long long tiles = ((M + 127) / 128) * ((N + 127) / 128);
  if (tiles > 0x7fffffffLL) return mmpi::fail(MMP_E_ARG, "matmul grid too large");
  const int m = (int)M, n = (int)N, k = (int)K;
  switch (dtype) {
    case MMP_F16: return launch16<mmp_half>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    case MMP_BF16: return launch16<__bf16>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    case MMP_F32: return launch4<float>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    case MMP_F64: return launch4<double>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    case MMP_I16: return launch_int<mmp_i16>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    case MMP_U16: return launch_int<mmp_u16>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    case MMP_I32: return launch_int<mmp_i32>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    case MMP_U32: return launch_int<mmp_u32>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    case MMP_I64: return launch_int<mmp_i64>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    case MMP_U64: return launch_int<mmp_u64>(batch, m, n, k, A, lda, sA, B, ldb, sB, C, ldc, sC);
    default: return mmpi::fail(MMP_E_UNSUPPORTED, "matmul dtype %d", dtype);
  }
}
