// linalg.hip -- batched dense factorizations for cp.linalg, one workgroup
// per matrix of a contiguous row-major batch, float32 and float64.
//
// Replaces the reference's NumPy/LAPACK host calls in linalg.py
// (solve / inv / det / slogdet :37-61, 149-159; cholesky :83-88; qr
// :97-105; eigh / eigvalsh :63-69, 122-127; svd / svdvals / pinv /
// matrix_rank / cond / lstsq :71-81, 129-183, 269-274).
//
//  * mmp_lu: right-looking LU with partial pivoting (the first row of
//    largest |a| in the column, as LAPACK's getrf picks), unit-lower L and
//    U packed in place, pivots as LAPACK's 0-based row swaps, info = first
//    exactly-zero pivot (1-based) or 0.
//  * mmp_lu_solve: row swaps, forward then backward substitution for nrhs
//    right-hand sides (threads over rows x rhs per elimination step).
//  * mmp_cholesky: right-looking lower Cholesky; info = first non-positive
//    pivot (1-based); the strict upper triangle is zeroed.
//  * mmp_qr / mmp_qr_q: Householder QR with LAPACK's reflector convention
//    (beta = -sign(alpha) * ||x||, tau = (beta - alpha) / beta, v(0) = 1),
//    R in the upper triangle, reflectors below it, then Q accumulated
//    backwards into the first qcols columns of I (one wavefront per column).
//  * mmp_eigh: cyclic two-sided Jacobi for symmetric matrices, disjoint
//    rotation pairs per round (round-robin ordering), rows then columns
//    updated per round, eigenvectors accumulated in V.
//  * mmp_svd: one-sided (Hestenes) Jacobi orthogonalising the rows of W
//    (rows <= len), one wavefront per row pair, row rotations mirrored in
//    VT; the row norms are the singular values.
// Every loop is bounded (the Jacobi sweeps by kMaxSweeps), so each
// workgroup exits.
#include <limits>

#include "mmp_ops.h"
#include "mmp_internal.h"

namespace {

constexpr int kT = 256;           // LU / Cholesky / QR workgroup
constexpr int kJ = 1024;          // Jacobi workgroup (16 wavefronts)
constexpr int kMaxSweeps = 60;
constexpr int kMaxEighN = 2048;   // rotation table in LDS: kMaxEighN / 2 pairs
constexpr int kMaxSvdRows = 8192;
constexpr int kNb = 64;             // panel width of the blocked LU
constexpr int kBlockedMinN = 256;   // from this order a few matrices use the blocked LU
constexpr int kBlockedMaxBatch = 64;
constexpr int kRhsChunk = 32;       // right-hand sides per workgroup in the substitution

// dst[r] -= src[r] * f for rows r = r0, r0 + S, ... < m of two columns of
// row-major matrices (leading dimensions ldd, lds): eight rows are loaded
// before any is stored (the stores never touch the loaded source column),
// so the loads overlap instead of waiting one by one.
template <typename T, int S>
__device__ __forceinline__ void axpy_rows(T *__restrict__ dst, long long ldd, const T *__restrict__ src,
                                          long long lds, int r0, int m, T f) {
  constexpr int U = 8;
  int r = r0;
  for (; r + (U - 1) * S < m; r += U * S) {
    T x[U], y[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      x[u] = src[(long long)(r + u * S) * lds];
      y[u] = dst[(long long)(r + u * S) * ldd];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) dst[(long long)(r + u * S) * ldd] = y[u] - x[u] * f;
  }
  for (; r < m; r += S) dst[(long long)r * ldd] -= src[(long long)r * lds] * f;
}

// Rows x, y (length len) := (c x - s y, s x + c y), lanes striding by 64,
// eight elements per lane loaded before any is stored.
template <typename T>
__device__ __forceinline__ void rotate_rows(T *__restrict__ x, T *__restrict__ y, int len, int lane, T c,
                                            T s) {
  constexpr int U = 8;
  int j = lane;
  for (; j + (U - 1) * 64 < len; j += U * 64) {
    T a[U], b[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      a[u] = x[j + u * 64];
      b[u] = y[j + u * 64];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      x[j + u * 64] = c * a[u] - s * b[u];
      y[j + u * 64] = s * a[u] + c * b[u];
    }
  }
  for (; j < len; j += 64) {
    const T a = x[j], b = y[j];
    x[j] = c * a - s * b;
    y[j] = s * a + c * b;
  }
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over the workgroup, the same value in every thread (fixed order).
template <int NT, typename T>
__device__ T block_sum(T v, T *lds) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
  __syncthreads();
  T r = T(0);
  for (int i = 0; i < NT / 64; ++i) r += lds[i];
  return r;
}

// Round-robin pairing of N (even) indices: N - 1 rounds, N / 2 disjoint
// pairs per round, every pair met once per sweep.
__device__ __forceinline__ void pair_of(int r, int pi, int N, int &p, int &q) {
  if (pi == 0) {
    p = N - 1;
    q = r;
  } else {
    p = (r + pi) % (N - 1);
    q = (r - pi + (N - 1)) % (N - 1);
  }
}

// ------------------------------------------------------------------- LU
template <typename T>
__global__ __launch_bounds__(kT) void k_getrf(T *__restrict__ a, int n, int *__restrict__ piv,
                                              int *__restrict__ info) {
  T *A = a + (long long)blockIdx.x * n * n;
  int *P = piv + (long long)blockIdx.x * n;
  __shared__ T sval[kT / 64];
  __shared__ int sidx[kT / 64];
  const int tid = threadIdx.x;
  int first_zero = 0;
  for (int k = 0; k < n; ++k) {
    T best = T(-1);
    int bi = n;
    for (int i = k + tid; i < n; i += kT) {
      const T v = fabs(A[(long long)i * n + k]);
      if (v > best) {
        best = v;
        bi = i;
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const T ov = __shfl_xor(best, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > best || (ov == best && oi < bi)) {
        best = ov;
        bi = oi;
      }
    }
    __syncthreads();
    if ((tid & 63) == 0) {
      sval[tid >> 6] = best;
      sidx[tid >> 6] = bi;
    }
    __syncthreads();
    best = sval[0];
    bi = sidx[0];
    for (int w = 1; w < kT / 64; ++w)
      if (sval[w] > best || (sval[w] == best && sidx[w] < bi)) {
        best = sval[w];
        bi = sidx[w];
      }
    const int p = bi < n ? bi : k;  // an all-NaN column keeps its row
    if (tid == 0) P[k] = p;
    if (p != k)
      for (int j = tid; j < n; j += kT) {
        const T t = A[(long long)k * n + j];
        A[(long long)k * n + j] = A[(long long)p * n + j];
        A[(long long)p * n + j] = t;
      }
    __syncthreads();
    const T d = A[(long long)k * n + k];
    if (d == T(0)) {  // the whole column is zero: nothing to eliminate
      if (!first_zero) first_zero = k + 1;
      continue;
    }
    for (int i = k + 1 + tid; i < n; i += kT) A[(long long)i * n + k] /= d;
    __syncthreads();
    const int m = n - k - 1;
    const long long mm = (long long)m * m;
    for (long long t = tid; t < mm; t += kT) {
      const int i = k + 1 + (int)(t / m), j = k + 1 + (int)(t % m);
      A[(long long)i * n + j] -= A[(long long)i * n + k] * A[(long long)k * n + j];
    }
    __syncthreads();
  }
  if (tid == 0) info[blockIdx.x] = first_zero;
}

// Workgroup (b, y) handles right-hand sides [y * kRhsChunk, ...) of matrix b.
template <typename T>
__global__ __launch_bounds__(kT) void k_getrs(const T *__restrict__ lu, const int *__restrict__ piv,
                                              T *__restrict__ b, int n, int nrhs) {
  const T *A = lu + (long long)blockIdx.x * n * n;
  const int *P = piv + (long long)blockIdx.x * n;
  const int c0 = blockIdx.y * kRhsChunk;
  const int cw = nrhs - c0 < kRhsChunk ? nrhs - c0 : kRhsChunk;
  T *B = b + (long long)blockIdx.x * n * nrhs + c0;
  const int tid = threadIdx.x;
  for (int c = tid; c < cw; c += kT)
    for (int k = 0; k < n; ++k) {
      const int p = P[k];
      if (p != k) {
        const T t = B[(long long)k * nrhs + c];
        B[(long long)k * nrhs + c] = B[(long long)p * nrhs + c];
        B[(long long)p * nrhs + c] = t;
      }
    }
  __syncthreads();
  // thread -> (row group r0, column c) once, no division per element; the
  // r0 < rstep threads cover every (row group, column) pair exactly once
  const int c = tid % cw, r0 = tid / cw, rstep = kT / cw;
  for (int k = 0; k < n - 1; ++k) {
    if (r0 < rstep) {
      const T bk = B[(long long)k * nrhs + c];
      for (int i = k + 1 + r0; i < n; i += rstep) B[(long long)i * nrhs + c] -= A[(long long)i * n + k] * bk;
    }
    __syncthreads();
  }
  for (int k = n - 1; k >= 0; --k) {
    if (tid < cw) B[(long long)k * nrhs + tid] /= A[(long long)k * n + k];
    __syncthreads();
    if (r0 < rstep) {
      const T bk = B[(long long)k * nrhs + c];
      for (int i = r0; i < k; i += rstep) B[(long long)i * nrhs + c] -= A[(long long)i * n + k] * bk;
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------ blocked LU
// One n x n matrix (leading dimension n), panels of kNb columns:
// k_getf2_panel factors rows j0.., columns j0..j0+jb with partial pivoting
// (one workgroup), k_laswp applies its row swaps to the other columns,
// k_trsm_ll forms U12 = L11^-1 A12 (one thread per column), and the
// trailing update A22 -= L21 U12 is a device matmul into scratch followed
// by k_sub_block.
template <typename T>
__global__ __launch_bounds__(kT) void k_getf2_panel(T *__restrict__ a, int n, int j0, int jb,
                                                    int *__restrict__ piv, int *__restrict__ info) {
  T *P = a + (long long)j0 * n + j0;
  const int m = n - j0;
  __shared__ T sval[kT / 64];
  __shared__ int sidx[kT / 64];
  const int tid = threadIdx.x;
  int first_zero = 0;
  for (int k = 0; k < jb; ++k) {
    T best = T(-1);
    int bi = m;
    for (int i = k + tid; i < m; i += kT) {
      const T v = fabs(P[(long long)i * n + k]);
      if (v > best) {
        best = v;
        bi = i;
      }
    }
    for (int o = 32; o > 0; o >>= 1) {
      const T ov = __shfl_xor(best, o, 64);
      const int oi = __shfl_xor(bi, o, 64);
      if (ov > best || (ov == best && oi < bi)) {
        best = ov;
        bi = oi;
      }
    }
    __syncthreads();
    if ((tid & 63) == 0) {
      sval[tid >> 6] = best;
      sidx[tid >> 6] = bi;
    }
    __syncthreads();
    best = sval[0];
    bi = sidx[0];
    for (int w = 1; w < kT / 64; ++w)
      if (sval[w] > best || (sval[w] == best && sidx[w] < bi)) {
        best = sval[w];
        bi = sidx[w];
      }
    const int p = bi < m ? bi : k;
    if (tid == 0) piv[j0 + k] = j0 + p;
    if (p != k)
      for (int j = tid; j < jb; j += kT) {
        const T t = P[(long long)k * n + j];
        P[(long long)k * n + j] = P[(long long)p * n + j];
        P[(long long)p * n + j] = t;
      }
    __syncthreads();
    const T d = P[(long long)k * n + k];
    if (d == T(0)) {
      if (!first_zero) first_zero = j0 + k + 1;
      continue;
    }
    for (int i = k + 1 + tid; i < m; i += kT) P[(long long)i * n + k] /= d;
    __syncthreads();
    // rank-1 update: lane = column (jb <= 64), wavefronts take rows in turn
    const int lane = tid & 63, wave = tid >> 6;
    if (lane < jb - k - 1) {
      const int j = k + 1 + lane;
      const T ukj = P[(long long)k * n + j];
      axpy_rows<T, kT / 64>(P + j, n, P + k, n, k + 1 + wave, m, ukj);
    }
    __syncthreads();
  }
  if (tid == 0) {
    if (j0 == 0) info[0] = first_zero;
    else if (info[0] == 0) info[0] = first_zero;
  }
}

template <typename T>
__global__ __launch_bounds__(kT) void k_laswp(T *__restrict__ a, int n, const int *__restrict__ piv,
                                              int k0, int k1) {
  const int c = blockIdx.x * kT + threadIdx.x;
  if (c >= n || (c >= k0 && c < k1)) return;  // the panel's own columns are swapped already
  for (int k = k0; k < k1; ++k) {
    const int p = piv[k];
    if (p != k) {
      const T t = a[(long long)k * n + c];
      a[(long long)k * n + c] = a[(long long)p * n + c];
      a[(long long)p * n + c] = t;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kT) void k_trsm_ll(T *__restrict__ a, int n, int j0, int jb) {
  const int c = j0 + jb + blockIdx.x * kT + threadIdx.x;
  if (c >= n) return;
  const T *L = a + (long long)j0 * n + j0;
  T *B = a + (long long)j0 * n;
  for (int i = 1; i < jb; ++i) {
    T s = B[(long long)i * n + c];
    for (int k = 0; k < i; ++k) s -= L[(long long)i * n + k] * B[(long long)k * n + c];
    B[(long long)i * n + c] = s;
  }
}

template <typename T>
__global__ __launch_bounds__(kT) void k_sub_block(T *__restrict__ a, int n, int r0, int mr, int nc,
                                                  const T *__restrict__ c) {
  const long long tot = (long long)mr * nc;
  for (long long t = (long long)blockIdx.x * kT + threadIdx.x; t < tot; t += (long long)gridDim.x * kT) {
    const int i = (int)(t / nc), j = (int)(t % nc);
    a[(long long)(r0 + i) * n + r0 + j] -= c[t];
  }
}

template <typename T>
int lu_blocked(int dtype, T *a, long long batch, int n, int *piv, int *info) {
  const long long m2max = (long long)(n - kNb);
  void *tmp = nullptr;
  if (m2max > 0)
    if (int st = mmp_alloc((size_t)(m2max * m2max) * sizeof(T), &tmp)) return st;
  int st = MMP_OK;
  const unsigned cgrid = (unsigned)mmpi::ceil_div(n, kT);
  for (long long b = 0; b < batch && st == MMP_OK; ++b) {
    T *A = a + b * (long long)n * n;
    int *P = piv + b * n;
    int *I = info + b;
    for (int j0 = 0; j0 < n && st == MMP_OK; j0 += kNb) {
      const int jb = n - j0 < kNb ? n - j0 : kNb;
      hipLaunchKernelGGL(k_getf2_panel<T>, dim3(1), dim3(kT), 0, mmpi::stream(), A, n, j0, jb, P, I);
      hipLaunchKernelGGL(k_laswp<T>, dim3(cgrid), dim3(kT), 0, mmpi::stream(), A, n, (const int *)P, j0,
                         j0 + jb);
      const int n2 = n - j0 - jb;
      if (n2 > 0) {
        hipLaunchKernelGGL(k_trsm_ll<T>, dim3((unsigned)mmpi::ceil_div(n2, kT)), dim3(kT), 0,
                           mmpi::stream(), A, n, j0, jb);
        st = mmp_matmul(dtype, 1, n2, n2, jb, A + (long long)(j0 + jb) * n + j0, n, 0,
                        A + (long long)j0 * n + j0 + jb, n, 0, tmp, n2, 0);
        if (st == MMP_OK) {
          const long long tot = (long long)n2 * n2;
          const long long g = mmpi::ceil_div(tot, kT);
          hipLaunchKernelGGL(k_sub_block<T>, dim3((unsigned)(g < 4096 ? g : 4096)), dim3(kT), 0,
                             mmpi::stream(), A, n, j0 + jb, n2, n2, (const T *)tmp);
        }
      }
      if (st == MMP_OK) st = mmpi::check_launch("mmp_lu (blocked)");
    }
  }
  if (tmp) {
    const int fs = mmp_free(tmp);
    if (st == MMP_OK) st = fs;
  }
  return st;
}

// -------------------------------------------------------------- Cholesky
template <typename T>
__global__ __launch_bounds__(kT) void k_potrf(T *__restrict__ a, int n, int *__restrict__ info) {
  T *A = a + (long long)blockIdx.x * n * n;
  const int tid = threadIdx.x;
  int bad = 0;
  for (int k = 0; k < n; ++k) {
    const T d = A[(long long)k * n + k];
    if (!(d > T(0))) {  // same value in every thread: a uniform exit
      bad = k + 1;
      break;
    }
    const T l = sqrt(d);
    __syncthreads();
    if (tid == 0) A[(long long)k * n + k] = l;
    for (int i = k + 1 + tid; i < n; i += kT) A[(long long)i * n + k] /= l;
    __syncthreads();
    const int m = n - k - 1;
    const long long mm = (long long)m * m;
    for (long long t = tid; t < mm; t += kT) {
      const int i = k + 1 + (int)(t / m), j = k + 1 + (int)(t % m);
      if (j <= i) A[(long long)i * n + j] -= A[(long long)i * n + k] * A[(long long)j * n + k];
    }
    __syncthreads();
  }
  const long long nn = (long long)n * n;
  for (long long t = tid; t < nn; t += kT)
    if ((int)(t % n) > (int)(t / n)) A[t] = T(0);
  if (tid == 0) info[blockIdx.x] = bad;
}

// ------------------------------------------------------ blocked Cholesky
// One n x n matrix, panels of kNb columns: the diagonal block is factored
// by one workgroup (k_potrf_diag), L21 = A21 L11^-T row by row
// (k_trsm_rlt, one thread per row), A22 -= L21 L21^T through the device
// matmul (L21^T staged by k_transpose_block) and k_sub_block; the strict
// upper triangle is zeroed at the end.
template <typename T>
__global__ __launch_bounds__(kT) void k_potrf_diag(T *__restrict__ a, int n, int j0, int jb,
                                                   int *__restrict__ info) {
  T *A = a + (long long)j0 * n + j0;
  const int tid = threadIdx.x;
  int bad = 0;
  if (info[0] != 0) return;  // an earlier panel failed: leave the rest
  for (int k = 0; k < jb; ++k) {
    const T d = A[(long long)k * n + k];
    if (!(d > T(0))) {
      bad = j0 + k + 1;
      break;
    }
    const T l = sqrt(d);
    __syncthreads();
    if (tid == 0) A[(long long)k * n + k] = l;
    for (int i = k + 1 + tid; i < jb; i += kT) A[(long long)i * n + k] /= l;
    __syncthreads();
    const int m = jb - k - 1;
    for (int t = tid; t < m * m; t += kT) {
      const int i = k + 1 + t / m, j = k + 1 + t % m;
      if (j <= i) A[(long long)i * n + j] -= A[(long long)i * n + k] * A[(long long)j * n + k];
    }
    __syncthreads();
  }
  if (tid == 0 && bad) info[0] = bad;
}

template <typename T>
__global__ __launch_bounds__(kT) void k_trsm_rlt(T *__restrict__ a, int n, int j0, int jb) {
  const int r = j0 + jb + blockIdx.x * kT + threadIdx.x;
  if (r >= n) return;
  const T *L = a + (long long)j0 * n + j0;
  T *X = a + (long long)r * n + j0;
  for (int k = 0; k < jb; ++k) {
    T s = X[k];
    for (int l = 0; l < k; ++l) s -= X[l] * L[(long long)k * n + l];
    X[k] = s / L[(long long)k * n + k];
  }
}

// out (jb x m2, contiguous) = transpose of A[r0 .. r0+m2)[j0 .. j0+jb)
template <typename T>
__global__ __launch_bounds__(kT) void k_transpose_block(const T *__restrict__ a, int n, int r0, int j0,
                                                        int m2, int jb, T *__restrict__ out) {
  const long long tot = (long long)m2 * jb;
  for (long long t = (long long)blockIdx.x * kT + threadIdx.x; t < tot; t += (long long)gridDim.x * kT) {
    const int k = (int)(t / m2), i = (int)(t % m2);
    out[t] = a[(long long)(r0 + i) * n + j0 + k];
  }
}

template <typename T>
__global__ __launch_bounds__(kT) void k_zero_upper(T *__restrict__ a, int n) {
  const long long tot = (long long)n * n;
  for (long long t = (long long)blockIdx.x * kT + threadIdx.x; t < tot; t += (long long)gridDim.x * kT)
    if ((int)(t % n) > (int)(t / n)) a[t] = T(0);
}

template <typename T>
__global__ void k_set_zero(int *__restrict__ p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0;
}

template <typename T>
int cholesky_blocked(int dtype, T *a, long long batch, int n, int *info) {
  const long long m2max = (long long)(n - kNb);
  void *tmp = nullptr, *tr = nullptr;
  if (m2max > 0) {
    if (int st = mmp_alloc((size_t)(m2max * m2max) * sizeof(T), &tmp)) return st;
    if (int st = mmp_alloc((size_t)(m2max * kNb) * sizeof(T), &tr)) {
      mmp_free(tmp);
      return st;
    }
  }
  hipLaunchKernelGGL(k_set_zero<T>, dim3(1), dim3(kT), 0, mmpi::stream(), info, (int)batch);
  int st = mmpi::check_launch("mmp_cholesky (blocked)");
  for (long long b = 0; b < batch && st == MMP_OK; ++b) {
    T *A = a + b * (long long)n * n;
    int *I = info + b;
    for (int j0 = 0; j0 < n && st == MMP_OK; j0 += kNb) {
      const int jb = n - j0 < kNb ? n - j0 : kNb;
      hipLaunchKernelGGL(k_potrf_diag<T>, dim3(1), dim3(kT), 0, mmpi::stream(), A, n, j0, jb, I);
      const int m2 = n - j0 - jb;
      if (m2 > 0) {
        hipLaunchKernelGGL(k_trsm_rlt<T>, dim3((unsigned)mmpi::ceil_div(m2, kT)), dim3(kT), 0,
                           mmpi::stream(), A, n, j0, jb);
        const long long g1 = mmpi::ceil_div((long long)m2 * jb, kT);
        hipLaunchKernelGGL(k_transpose_block<T>, dim3((unsigned)(g1 < 4096 ? g1 : 4096)), dim3(kT), 0,
                           mmpi::stream(), (const T *)A, n, j0 + jb, j0, m2, jb, (T *)tr);
        st = mmp_matmul(dtype, 1, m2, m2, jb, A + (long long)(j0 + jb) * n + j0, n, 0, tr, m2, 0, tmp,
                        m2, 0);
        if (st == MMP_OK) {
          const long long g = mmpi::ceil_div((long long)m2 * m2, kT);
          hipLaunchKernelGGL(k_sub_block<T>, dim3((unsigned)(g < 4096 ? g : 4096)), dim3(kT), 0,
                             mmpi::stream(), A, n, j0 + jb, m2, m2, (const T *)tmp);
        }
      }
      if (st == MMP_OK) st = mmpi::check_launch("mmp_cholesky (blocked)");
    }
    if (st == MMP_OK) {
      const long long g = mmpi::ceil_div((long long)n * n, kT);
      hipLaunchKernelGGL(k_zero_upper<T>, dim3((unsigned)(g < 4096 ? g : 4096)), dim3(kT), 0,
                         mmpi::stream(), A, n);
      st = mmpi::check_launch("mmp_cholesky (blocked)");
    }
  }
  if (tmp) mmp_free(tmp);
  if (tr) mmp_free(tr);
  return st;
}

// -------------------------------------------------------------------- QR
template <typename T>
__global__ __launch_bounds__(kT) void k_geqrf(T *__restrict__ a, int m, int n, T *__restrict__ tau) {
  const int kmin = m < n ? m : n;
  T *A = a + (long long)blockIdx.x * m * n;
  T *TAU = tau + (long long)blockIdx.x * kmin;
  __shared__ T red[kT / 64];
  __shared__ T part_lds[kT / 64][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int k = 0; k < kmin; ++k) {
    T part = T(0);
    for (int i = k + 1 + tid; i < m; i += kT) {
      const T v = A[(long long)i * n + k];
      part += v * v;
    }
    const T xn2 = block_sum<kT>(part, red);
    const T alpha = A[(long long)k * n + k];
    T t = T(0);
    if (xn2 != T(0)) {
      const T beta = -copysign(sqrt(alpha * alpha + xn2), alpha);
      t = (beta - alpha) / beta;
      const T sc = T(1) / (alpha - beta);
      __syncthreads();  // alpha read everywhere before A[k][k] changes
      for (int i = k + 1 + tid; i < m; i += kT) A[(long long)i * n + k] *= sc;
      if (tid == 0) A[(long long)k * n + k] = beta;
    }
    if (tid == 0) TAU[k] = t;
    __syncthreads();
    if (t != T(0)) {
      // lane = column of a 64-column chunk, wavefronts split the rows; the
      // four partial dot products meet in LDS
      for (int jc = k + 1; jc < n; jc += 64) {
        const int j = jc + lane;
        T part = T(0);
        if (j < n) {
#pragma unroll 8
          for (int i = k + 1 + wave; i < m; i += kT / 64) part += A[(long long)i * n + k] * A[(long long)i * n + j];
        }
        // A[k][j] is read by every wavefront before the barrier and
        // written by wavefront 0 after it
        const T akj = j < n ? A[(long long)k * n + j] : T(0);
        part_lds[wave][lane] = part;
        __syncthreads();
        if (j < n) {
          T w = akj;
          for (int q = 0; q < kT / 64; ++q) w += part_lds[q][lane];
          axpy_rows<T, kT / 64>(A + j, n, A + k, n, k + 1 + wave, m, t * w);
          if (wave == 0) A[(long long)k * n + j] = akj - t * w;
        }
        __syncthreads();
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kT) void k_orgqr(const T *__restrict__ a, const T *__restrict__ tau, int m,
                                              int n, int qc, T *__restrict__ q) {
  const int kmin = m < n ? m : n;
  const T *A = a + (long long)blockIdx.x * m * n;
  const T *TAU = tau + (long long)blockIdx.x * kmin;
  T *Q = q + (long long)blockIdx.x * m * qc;
  __shared__ T part_lds[kT / 64][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long long tot = (long long)m * qc;
  for (long long t = tid; t < tot; t += kT) Q[t] = (t / qc == t % qc) ? T(1) : T(0);
  __syncthreads();
  for (int k = kmin - 1; k >= 0; --k) {
    const T t = TAU[k];
    if (t == T(0)) continue;
    for (int jc = k; jc < qc; jc += 64) {
      const int j = jc + lane;
      T part = T(0);
      if (j < qc) {
#pragma unroll 8
        for (int i = k + 1 + wave; i < m; i += kT / 64) part += A[(long long)i * n + k] * Q[(long long)i * qc + j];
      }
      const T qkj = j < qc ? Q[(long long)k * qc + j] : T(0);
      part_lds[wave][lane] = part;
      __syncthreads();
      if (j < qc) {
        T w = qkj;
        for (int q = 0; q < kT / 64; ++q) w += part_lds[q][lane];
        axpy_rows<T, kT / 64>(Q + j, qc, A + k, n, k + 1 + wave, m, t * w);
        if (wave == 0) Q[(long long)k * qc + j] = qkj - t * w;
      }
      __syncthreads();
    }
  }
}

// ------------------------------------------------------ symmetric Jacobi
template <typename T>
__global__ __launch_bounds__(kJ) void k_syevj(T *__restrict__ a, T *__restrict__ v, int n,
                                              int *__restrict__ sweeps_out) {
  T *A = a + (long long)blockIdx.x * n * n;
  T *V = v + (long long)blockIdx.x * n * n;
  __shared__ T cs[kMaxEighN];  // (c, s) of each pair of the round
  __shared__ int s_rot;
  const int tid = threadIdx.x;
  const int N = n + (n & 1);
  const int npair = N / 2;
  const T eps = std::numeric_limits<T>::epsilon();
  const long long nn = (long long)n * n;
  for (long long t = tid; t < nn; t += kJ) V[t] = (t / n == t % n) ? T(1) : T(0);
  int sweep = 0;
  for (; sweep < kMaxSweeps; ++sweep) {
    if (tid == 0) s_rot = 0;
    __syncthreads();
    for (int r = 0; r < N - 1; ++r) {
      for (int pi = tid; pi < npair; pi += kJ) {
        int p, q;
        pair_of(r, pi, N, p, q);
        T c = T(1), s = T(0);
        if (p < n && q < n) {
          const T app = A[(long long)p * n + p], aqq = A[(long long)q * n + q];
          const T apq = A[(long long)p * n + q];
          if (apq != T(0) && fabs(apq) > eps * sqrt(fabs(app * aqq))) {
            const T th = (aqq - app) / (T(2) * apq);
            const T tt = (th >= T(0) ? T(1) : T(-1)) / (fabs(th) + sqrt(T(1) + th * th));
            c = T(1) / sqrt(T(1) + tt * tt);
            s = tt * c;
            if (s != T(0)) s_rot = 1;
          }
        }
        cs[2 * pi] = c;
        cs[2 * pi + 1] = s;
      }
      __syncthreads();
      const int work = npair * n;  // <= 2^21
      for (int t = tid; t < work; t += kJ) {
        const int pi = t / n, j = t - pi * n;  // lanes along a row: coalesced
        const T s = cs[2 * pi + 1];
        if (s == T(0)) continue;
        int p, q;
        pair_of(r, pi, N, p, q);
        const T c = cs[2 * pi];
        const T x = A[(long long)p * n + j], y = A[(long long)q * n + j];
        A[(long long)p * n + j] = c * x - s * y;
        A[(long long)q * n + j] = s * x + c * y;
      }
      __syncthreads();
      for (int t = tid; t < work; t += kJ) {
        // lanes over consecutive pairs of one row: the round-robin pairs
        // are runs of consecutive columns, so the accesses coalesce
        const int i = t / npair, pi = t - i * npair;
        const T s = cs[2 * pi + 1];
        if (s == T(0)) continue;
        int p, q;
        pair_of(r, pi, N, p, q);
        const T c = cs[2 * pi];
        const T x = A[(long long)i * n + p], y = A[(long long)i * n + q];
        A[(long long)i * n + p] = c * x - s * y;
        A[(long long)i * n + q] = s * x + c * y;
        const T vx = V[(long long)i * n + p], vy = V[(long long)i * n + q];
        V[(long long)i * n + p] = c * vx - s * vy;
        V[(long long)i * n + q] = s * vx + c * vy;
      }
      __syncthreads();
    }
    const int rotated = s_rot;
    __syncthreads();
    if (!rotated) break;
  }
  if (tid == 0) sweeps_out[blockIdx.x] = sweep;
}

// ------------------------------------------------------ one-sided Jacobi
template <typename T>
__global__ __launch_bounds__(kJ) void k_gesvj(T *__restrict__ w, T *__restrict__ vt, int r, int L,
                                              int *__restrict__ sweeps_out) {
  T *W = w + (long long)blockIdx.x * r * L;
  T *VT = vt + (long long)blockIdx.x * r * r;
  __shared__ int s_rot;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = r + (r & 1);
  const int npair = N / 2;
  const T eps = std::numeric_limits<T>::epsilon();
  const long long rr = (long long)r * r;
  for (long long t = tid; t < rr; t += kJ) VT[t] = (t / r == t % r) ? T(1) : T(0);
  int sweep = 0;
  for (; sweep < kMaxSweeps; ++sweep) {
    if (tid == 0) s_rot = 0;
    __syncthreads();
    for (int rd = 0; rd < N - 1; ++rd) {
      for (int pi = wave; pi < npair; pi += kJ / 64) {
        int p, q;
        pair_of(rd, pi, N, p, q);
        if (p >= r || q >= r) continue;
        T al = T(0), be = T(0), ga = T(0);
#pragma unroll 8
        for (int j = lane; j < L; j += 64) {
          const T x = W[(long long)p * L + j], y = W[(long long)q * L + j];
          al += x * x;
          be += y * y;
          ga += x * y;
        }
        al = wave_sum(al);
        be = wave_sum(be);
        ga = wave_sum(ga);
        if (ga != T(0) && fabs(ga) > eps * sqrt(al * be)) {
          const T ze = (be - al) / (T(2) * ga);
          const T tt = (ze >= T(0) ? T(1) : T(-1)) / (fabs(ze) + sqrt(T(1) + ze * ze));
          const T c = T(1) / sqrt(T(1) + tt * tt), s = c * tt;
          if (s != T(0)) {
            rotate_rows(W + (long long)p * L, W + (long long)q * L, L, lane, c, s);
            rotate_rows(VT + (long long)p * r, VT + (long long)q * r, r, lane, c, s);
            if (lane == 0) s_rot = 1;
          }
        }
      }
      __syncthreads();
    }
    const int rotated = s_rot;
    __syncthreads();
    if (!rotated) break;
  }
  if (tid == 0) sweeps_out[blockIdx.x] = sweep;
}

int check_common(const char *what, int dtype, long long batch) {
  if (dtype != MMP_F32 && dtype != MMP_F64)
    return mmpi::fail(MMP_E_UNSUPPORTED, "%s: dtype %d (float32 / float64 only)", what, dtype);
  if (batch < 0 || batch > 0x7fffffffll) return mmpi::fail(MMP_E_ARG, "%s: batch %lld", what, batch);
  return MMP_OK;
}

}  // namespace

extern "C" int mmp_lu(int dtype, void *a, int64_t batch, int64_t n, int32_t *piv, int32_t *info) {
  if (int st = mmpi::ensure_init()) return st;
  if (int st = check_common("mmp_lu", dtype, batch)) return st;
  if (n < 0 || n > 32768) return mmpi::fail(MMP_E_ARG, "mmp_lu: n %lld", (long long)n);
  if (batch == 0 || n == 0) return MMP_OK;
  if (!a || !piv || !info) return mmpi::fail(MMP_E_ARG, "mmp_lu: null pointer");
  if (n >= kBlockedMinN && batch <= kBlockedMaxBatch)
    return dtype == MMP_F32 ? lu_blocked<float>(dtype, (float *)a, batch, (int)n, (int *)piv, (int *)info)
                            : lu_blocked<double>(dtype, (double *)a, batch, (int)n, (int *)piv, (int *)info);
  if (dtype == MMP_F32)
    hipLaunchKernelGGL(k_getrf<float>, dim3((unsigned)batch), dim3(kT), 0, mmpi::stream(), (float *)a,
                       (int)n, (int *)piv, (int *)info);
  else
    hipLaunchKernelGGL(k_getrf<double>, dim3((unsigned)batch), dim3(kT), 0, mmpi::stream(), (double *)a,
                       (int)n, (int *)piv, (int *)info);
  return mmpi::check_launch("mmp_lu");
}

extern "C" int mmp_lu_solve(int dtype, const void *lu, const int32_t *piv, void *b, int64_t batch,
                            int64_t n, int64_t nrhs) {
  if (int st = mmpi::ensure_init()) return st;
  if (int st = check_common("mmp_lu_solve", dtype, batch)) return st;
  if (n < 0 || n > 32768 || nrhs < 0 || nrhs > 0x7fffffffll)
    return mmpi::fail(MMP_E_ARG, "mmp_lu_solve: n %lld nrhs %lld", (long long)n, (long long)nrhs);
  if (batch == 0 || n == 0 || nrhs == 0) return MMP_OK;
  if (!lu || !piv || !b) return mmpi::fail(MMP_E_ARG, "mmp_lu_solve: null pointer");
  const dim3 grid((unsigned)batch, (unsigned)mmpi::ceil_div(nrhs, kRhsChunk));
  if (grid.y > 65535) return mmpi::fail(MMP_E_ARG, "mmp_lu_solve: nrhs %lld too large", (long long)nrhs);
  if (dtype == MMP_F32)
    hipLaunchKernelGGL(k_getrs<float>, grid, dim3(kT), 0, mmpi::stream(),
                       (const float *)lu, (const int *)piv, (float *)b, (int)n, (int)nrhs);
  else
    hipLaunchKernelGGL(k_getrs<double>, grid, dim3(kT), 0, mmpi::stream(),
                       (const double *)lu, (const int *)piv, (double *)b, (int)n, (int)nrhs);
  return mmpi::check_launch("mmp_lu_solve");
}

extern "C" int mmp_cholesky(int dtype, void *a, int64_t batch, int64_t n, int32_t *info) {
  if (int st = mmpi::ensure_init()) return st;
  if (int st = check_common("mmp_cholesky", dtype, batch)) return st;
  if (n < 0 || n > 32768) return mmpi::fail(MMP_E_ARG, "mmp_cholesky: n %lld", (long long)n);
  if (batch == 0 || n == 0) return MMP_OK;
  if (!a || !info) return mmpi::fail(MMP_E_ARG, "mmp_cholesky: null pointer");
  if (n >= kBlockedMinN && batch <= kBlockedMaxBatch)
    return dtype == MMP_F32 ? cholesky_blocked<float>(dtype, (float *)a, batch, (int)n, (int *)info)
                            : cholesky_blocked<double>(dtype, (double *)a, batch, (int)n, (int *)info);
  if (dtype == MMP_F32)
    hipLaunchKernelGGL(k_potrf<float>, dim3((unsigned)batch), dim3(kT), 0, mmpi::stream(), (float *)a,
                       (int)n, (int *)info);
  else
    hipLaunchKernelGGL(k_potrf<double>, dim3((unsigned)batch), dim3(kT), 0, mmpi::stream(), (double *)a,
                       (int)n, (int *)info);
  return mmpi::check_launch("mmp_cholesky");
}

extern "C" int mmp_qr(int dtype, void *a, void *tau, int64_t batch, int64_t m, int64_t n) {
  if (int st = mmpi::ensure_init()) return st;
  if (int st = check_common("mmp_qr", dtype, batch)) return st;
  if (m < 0 || n < 0 || m > 0x7fffffffll || n > 0x7fffffffll)
    return mmpi::fail(MMP_E_ARG, "mmp_qr: shape %lld x %lld", (long long)m, (long long)n);
  if (batch == 0 || m == 0 || n == 0) return MMP_OK;
  if (!a || !tau) return mmpi::fail(MMP_E_ARG, "mmp_qr: null pointer");
  if (dtype == MMP_F32)
    hipLaunchKernelGGL(k_geqrf<float>, dim3((unsigned)batch), dim3(kT), 0, mmpi::stream(), (float *)a,
                       (int)m, (int)n, (float *)tau);
  else
    hipLaunchKernelGGL(k_geqrf<double>, dim3((unsigned)batch), dim3(kT), 0, mmpi::stream(), (double *)a,
                       (int)m, (int)n, (double *)tau);
  return mmpi::check_launch("mmp_qr");
}

extern "C" int mmp_qr_q(int dtype, const void *a, const void *tau, int64_t batch, int64_t m, int64_t n,
                        int64_t qcols, void *q) {
  if (int st = mmpi::ensure_init()) return st;
  if (int st = check_common("mmp_qr_q", dtype, batch)) return st;
  const long long kmin = m < n ? m : n;
  if (m < 0 || n < 0 || m > 0x7fffffffll || n > 0x7fffffffll || qcols < kmin || qcols > m)
    return mmpi::fail(MMP_E_ARG, "mmp_qr_q: shape %lld x %lld, qcols %lld", (long long)m,
                      (long long)n, (long long)qcols);
  if (batch == 0 || m == 0 || qcols == 0) return MMP_OK;
  if (!a || !tau || !q) return mmpi::fail(MMP_E_ARG, "mmp_qr_q: null pointer");
  if (dtype == MMP_F32)
    hipLaunchKernelGGL(k_orgqr<float>, dim3((unsigned)batch), dim3(kT), 0, mmpi::stream(),
                       (const float *)a, (const float *)tau, (int)m, (int)n, (int)qcols, (float *)q);
  else
    hipLaunchKernelGGL(k_orgqr<double>, dim3((unsigned)batch), dim3(kT), 0, mmpi::stream(),
                       (const double *)a, (const double *)tau, (int)m, (int)n, (int)qcols, (double *)q);
  return mmpi::check_launch("mmp_qr_q");
}

extern "C" int mmp_eigh(int dtype, void *a, void *v, int64_t batch, int64_t n, int32_t *sweeps) {
  if (int st = mmpi::ensure_init()) return st;
  if (int st = check_common("mmp_eigh", dtype, batch)) return st;
  if (n < 0 || n > kMaxEighN) return mmpi::fail(MMP_E_ARG, "mmp_eigh: n %lld (at most %d)", (long long)n, kMaxEighN);
  if (batch == 0 || n == 0) return MMP_OK;
  if (!a || !v || !sweeps) return mmpi::fail(MMP_E_ARG, "mmp_eigh: null pointer");
  if (dtype == MMP_F32)
    hipLaunchKernelGGL(k_syevj<float>, dim3((unsigned)batch), dim3(kJ), 0, mmpi::stream(), (float *)a,
                       (float *)v, (int)n, (int *)sweeps);
  else
    hipLaunchKernelGGL(k_syevj<double>, dim3((unsigned)batch), dim3(kJ), 0, mmpi::stream(), (double *)a,
                       (double *)v, (int)n, (int *)sweeps);
  return mmpi::check_launch("mmp_eigh");
}

extern "C" int mmp_svd(int dtype, void *w, void *vt, int64_t batch, int64_t rows, int64_t len,
                       int32_t *sweeps) {
  if (int st = mmpi::ensure_init()) return st;
  if (int st = check_common("mmp_svd", dtype, batch)) return st;
  if (rows < 0 || rows > kMaxSvdRows || len < rows || len > 0x7fffffffll)
    return mmpi::fail(MMP_E_ARG, "mmp_svd: rows %lld len %lld (rows <= len, rows <= %d)", (long long)rows,
                      (long long)len, kMaxSvdRows);
  if (batch == 0 || rows == 0) return MMP_OK;
  if (!w || !vt || !sweeps) return mmpi::fail(MMP_E_ARG, "mmp_svd: null pointer");
  if (dtype == MMP_F32)
    hipLaunchKernelGGL(k_gesvj<float>, dim3((unsigned)batch), dim3(kJ), 0, mmpi::stream(), (float *)w,
                       (float *)vt, (int)rows, (int)len, (int *)sweeps);
  else
    hipLaunchKernelGGL(k_gesvj<double>, dim3((unsigned)batch), dim3(kJ), 0, mmpi::stream(), (double *)w,
                       (double *)vt, (int)rows, (int)len, (int *)sweeps);
  return mmpi::check_launch("mmp_svd");
}
