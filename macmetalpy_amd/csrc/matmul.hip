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

template <typename T>
int launch16(long long batch, int M, int N, int K, const void *A, long long lda, long long sA,
             const void *B, long long ldb, long long sB, void *C, long long ldc, long long sC) {
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
