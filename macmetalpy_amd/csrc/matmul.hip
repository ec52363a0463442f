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
//  * float32 / float64: v_mfma_f32_16x16x4f32 / v_mfma_f64_16x16x4f64.  The
//    k slot a lane feeds is permuted (MFMA step t, lane group g consumes
//    k = KG*g + t), so a lane's A values for a whole slab are contiguous in
//    LDS and B keeps its natural n-contiguous layout.
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

// ------------------------------------------- 16-bit inputs, large tiles
// 256 x 256 output tile per workgroup for operands whose extents divide
// the tile and whose rows are 16-byte aligned.  WM x WN waves (2 x 4 by
// default: eight waves, two per SIMD, each owning a 128 x 64 sub-tile with
// its 128 fp32 accumulators in VGPRs); one workgroup per CU.  Per 64-deep
// k slab a workgroup moves 64 KiB L2 -> LDS for 256 x 256 x 64 MACs, half
// the L2 traffic per flop of a 128 x 128 tile.
//  * Loading (eight waves): waves 0-3 fetch B, waves 4-7 fetch A, every
//    thread as eight 16-byte row pieces.  A is stored unchanged
//    (k-contiguous); a B thread owns an 8(k) x 8(n) block and transposes it
//    in registers (v_perm) into eight k-contiguous columns.  Eight
//    consecutive lanes cover one 128 B row segment in HBM and one LDS row.
//  * LDS: two buffers of 256 rows x 128 B for each operand, 16-byte chunks
//    XOR-swizzled per row (see swz below): conflict-free fragment reads and
//    stores.
//  * Pipeline per slab kt: store slab kt + 1 (already in registers) to the
//    idle buffer, issue the global loads of slab kt + 2, run slab kt's
//    MFMAs with the loads spread between them, one barrier.
//  * The MFMA is issued as C^T = B^T A^T (operands swapped), so a lane's
//    four accumulators are four consecutive columns of one C row: the
//    epilogue writes 8 B per lane per 16 x 16 tile.
//  * Workgroup ids are remapped so that the tiles one XCD runs together
//    (ids are dealt round-robin over the eight XCDs) form 4-row groups:
//    concurrent workgroups on an XCD share A and B panels in its L2.
// Measured at 8192^3 float16 on MI355X: 0.85 PF/s (1.31 ms).  The same loop
// without global loads reaches 1.4 PF/s and a register-fed MFMA loop with
// random operands 1.6 PF/s (operand-dependent power limits the clock), so
// the remaining gap is the global->LDS path.
#ifndef MMP_GEMM16_SPLIT
#define MMP_GEMM16_SPLIT 1
#endif
#ifndef MMP_GEMM16_INTERLEAVE
#define MMP_GEMM16_INTERLEAVE 1
#endif

template <int BW> struct BRow;
template <> struct BRow<8> { typedef u32x4 type; };
template <> struct BRow<4> { typedef u32x2 type; };

template <typename T, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN, 1) void k_gemm16_big(
    const T *__restrict__ A, const T *__restrict__ B, T *__restrict__ C, int M, int N, int K,
    long long lda, long long ldb, long long ldc, long long sA, long long sB, long long sC,
    int tiles_m, int tiles_n) {
  constexpr int NT = 64 * WM * WN;
  constexpr int TB = 256, BK = 64, LDK = BK;
  constexpr int TM = TB / WM, TN = TB / WN;   // wave tile
  constexpr int I = TM / 16, J = TN / 16;     // 16 x 16 MFMA tiles per wave
  constexpr int AV = TB * (BK / 8) / NT;      // A vectors per thread
  constexpr int BW = TB * BK / (NT * 8);      // B block width (n)
  static_assert(BW == 4 || BW == 8, "B block width");
  typedef typename Half16<T>::vec V;
  typedef typename BRow<BW>::type BR;
  __shared__ __attribute__((aligned(16))) unsigned short As[2][TB * LDK];
  __shared__ __attribute__((aligned(16))) unsigned short Bs[2][TB * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // XCD-aware, 4-row grouped tile order
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

  u32x4 ra[AV];
  BR rb[8];
  const int a_row = tid >> 3, a_kv = tid & 7;
  const int b_k8 = tid & 7, b_nb = tid >> 3;
  // LDS rows are 128 B (64 k); 16-byte chunk c of row r is stored at
  // chunk c ^ ((r >> 1) & 7).  Measured on gfx950: ds_read_b128 serves
  // 16 lanes per cycle (lanes sharing bits 1 and 5 of the lane id) and
  // conflicts when two of them hit the same 16 B slot modulo 512 B; with
  // this swizzle the fragment reads (16 rows x 2 chunks per lane group)
  // and the row-contiguous stores are conflict-free, where a 144 B row
  // pitch gave 2-way conflicts on every fragment read.
  auto swz = [](int r) { return (r >> 1) & 7; };
  const int a_swz = swz(a_row);

  // With eight waves, the first four load B and the last four load A, each
  // thread as eight 16-byte row pieces (a B thread owns an 8(k) x 8(n)
  // block, an A thread eight row segments): every global load is 16 bytes
  // wide and each wave issues eight, instead of twelve half of which move
  // only 8 bytes per lane.  The role test is uniform per wave.
  constexpr bool SPLIT = NT == 512 && MMP_GEMM16_SPLIT;
  const bool b_role = tid < 256;
  const int t2 = tid & 255;
  const int s_k8 = t2 & 7, s_nb = t2 >> 3;     // B role: 8 x 8 block
  const int s_row = t2 >> 3, s_kv = t2 & 7;    // A role: rows s_row + 32p
  const int s_swz = swz(s_row);
  u32x4 rs[8];
  auto load_split = [&](int k0) {
    if (b_role) {
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        rs[kk] = *reinterpret_cast<const u32x4 *>(Bg + (long long)(k0 + s_k8 * 8 + kk) * ldb + s_nb * 8);
    } else {
#pragma unroll
      for (int p = 0; p < 8; ++p)
        rs[p] = *reinterpret_cast<const u32x4 *>(Ag + (long long)(s_row + 32 * p) * lda + k0 + s_kv * 8);
    }
  };
  auto store_split = [&](int buf) {
    if (b_role) {
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const unsigned sel = (c & 1) ? 0x07060302u : 0x05040100u;
        u32x4 w;
#pragma unroll
        for (int d = 0; d < 4; ++d)
          w[d] = __builtin_amdgcn_perm(rs[2 * d + 1][c >> 1], rs[2 * d][c >> 1], sel);
        *reinterpret_cast<u32x4 *>(&Bs[buf][(s_nb * 8 + c) * LDK + (s_k8 ^ swz(s_nb * 8 + c)) * 8]) = w;
      }
    } else {
#pragma unroll
      for (int p = 0; p < 8; ++p)
        *reinterpret_cast<u32x4 *>(&As[buf][(s_row + 32 * p) * LDK + (s_kv ^ s_swz) * 8]) = rs[p];
    }
  };

  auto load = [&](int k0) {
    if constexpr (SPLIT) {
      load_split(k0);
      return;
    }
#pragma unroll
    for (int p = 0; p < AV; ++p)
      ra[p] = *reinterpret_cast<const u32x4 *>(Ag + (long long)(a_row + (NT / 8) * p) * lda +
                                               k0 + a_kv * 8);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
      rb[kk] = *reinterpret_cast<const BR *>(Bg + (long long)(k0 + b_k8 * 8 + kk) * ldb +
                                             b_nb * BW);
  };
  auto store = [&](int buf) {
    if constexpr (SPLIT) {
      store_split(buf);
      return;
    }
#pragma unroll
    for (int p = 0; p < AV; ++p)
      *reinterpret_cast<u32x4 *>(&As[buf][(a_row + (NT / 8) * p) * LDK + (a_kv ^ a_swz) * 8]) = ra[p];
    // column c of the 8 x BW block: half c of each of the eight rows
#pragma unroll
    for (int c = 0; c < BW; ++c) {
      const unsigned sel = (c & 1) ? 0x07060302u : 0x05040100u;
      u32x4 w;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        w[d] = __builtin_amdgcn_perm(rb[2 * d + 1][c >> 1], rb[2 * d][c >> 1], sel);
      *reinterpret_cast<u32x4 *>(&Bs[buf][(b_nb * BW + c) * LDK + (b_k8 ^ swz(b_nb * BW + c)) * 8]) = w;
    }
  };

  f4 acc[I][J];
#pragma unroll
  for (int i = 0; i < I; ++i)
#pragma unroll
    for (int j = 0; j < J; ++j) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};

  const int nk = K / BK;
  const int fr = lane & 15;
  // fragment chunk offsets (halves) of sub-steps 0 and 1 for this lane
  const int fch[2] = {(((lane >> 4) + 0) ^ swz(fr)) * 8, (((lane >> 4) + 4) ^ swz(fr)) * 8};
  auto mfmas = [&](int cur) {
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      V af[I], bf[J];
#pragma unroll
      for (int i = 0; i < I; ++i)
        af[i] = *reinterpret_cast<const V *>(&As[cur][(wm * TM + i * 16 + fr) * LDK + fch[s]]);
#pragma unroll
      for (int j = 0; j < J; ++j)
        bf[j] = *reinterpret_cast<const V *>(&Bs[cur][(wn * TN + j * 16 + fr) * LDK + fch[s]]);
#pragma unroll
      for (int i = 0; i < I; ++i)
#pragma unroll
        for (int j = 0; j < J; ++j) acc[i][j] = Half16<T>::mfma(bf[j], af[i], acc[i][j]);
    }
  };

  // Pipeline: slab kt + 1 sits in registers when step kt begins.  The step
  // writes it to the idle LDS buffer, refills the registers with slab
  // kt + 2 (clamped to the last slab; the surplus copy is never read) and
  // then runs slab kt's MFMAs from the other buffer, so the LDS stores and
  // the global-load latency overlap the MFMAs instead of separating them;
  // one barrier per slab.  Straight-line steps let the scheduler interleave
  // loads, LDS traffic and MFMAs.
  load(0);
  store(0);
  load(min(1, nk - 1) * BK);
  __syncthreads();
  constexpr int NLOAD = SPLIT ? 8 : AV + 8;  // global loads per thread per slab
  constexpr int NMFMA = 2 * I * J;          // MFMAs per wave per slab
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    store(cur ^ 1);
    load(min(kt + 2, nk - 1) * BK);
    mfmas(cur);
#if MMP_GEMM16_INTERLEAVE
    // spread the global loads over the MFMA stream: a wave that issues all
    // of them back to back stalls on the full address queue and starves
    // the matrix core
#pragma unroll
    for (int g = 0; g < NLOAD; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                // 1 VMEM read
      __builtin_amdgcn_sched_group_barrier(0x008, NMFMA / NLOAD, 0);    // MFMAs
    }
#endif
    __syncthreads();
  }

  // epilogue: accumulator r of lane l is C[row l % 16][col 4 * (l / 16) + r]
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

// Large-tile kernel: 2 = 2 x 4 waves of 128 x 64 (default), 1 = 2 x 2
// waves of 128 x 128 (slower: the compiler shuffles its 256 accumulators
// between register files), 0 = off.  Used once the product has at least
// MMP_GEMM16_BIG_MIN_TILES 256 x 256 tiles (fewer leave CUs idle).
#ifndef MMP_GEMM16_BIG
#define MMP_GEMM16_BIG 2
#endif
#ifndef MMP_GEMM16_BIG_MIN_TILES
#define MMP_GEMM16_BIG_MIN_TILES 128
#endif

template <typename T>
int launch16(long long batch, int M, int N, int K, const void *A, long long lda, long long sA,
             const void *B, long long ldb, long long sB, void *C, long long ldc, long long sC) {
  if (MMP_GEMM16_BIG && M % 256 == 0 && N % 256 == 0 && K % 64 == 0 && lda % 8 == 0 &&
      ldb % 8 == 0 && ldc % 4 == 0 && sA % 8 == 0 && sB % 8 == 0 && sC % 4 == 0 && al(A, 16) &&
      al(B, 16) && al(C, 8) &&
      (long long)(M / 256) * (N / 256) * batch >= MMP_GEMM16_BIG_MIN_TILES) {
    const int tm = M / 256, tn = N / 256;
    dim3 grid((unsigned)(tm * tn), (unsigned)batch);
    if (MMP_GEMM16_BIG == 2)
      hipLaunchKernelGGL((k_gemm16_big<T, 2, 4>), grid, dim3(512), 0, mmpi::stream(),
                         (const T *)A, (const T *)B, (T *)C, M, N, K, lda, ldb, ldc, sA, sB, sC,
                         tm, tn);
    else
      hipLaunchKernelGGL((k_gemm16_big<T, 2, 2>), grid, dim3(256), 0, mmpi::stream(),
                         (const T *)A, (const T *)B, (T *)C, M, N, K, lda, ldb, ldc, sA, sB, sC,
                         tm, tn);
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
