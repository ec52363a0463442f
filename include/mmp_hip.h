/*
 * mmp_hip.h -- C ABI of libmmp_hip.so, the MI355X (gfx950) compute library
 * behind macmetalpy_amd's `import macmetalpy as cp` array API.
 *
 * The reference drives its GPU through eleven ctypes-bound symbols of the
 * external metalgpu dylib (src/macmetalpy/_metal_backend.py:221-263):
 * init / deleteInstance / createBuffer / releaseBuffer / getBufferPointer /
 * createLibrary / createLibraryFromString / setFunction / runFunction /
 * maxThreadsPerGroup / threadExecutionWidth.  That ABI is stateful ("current
 * library", "current function"), has no error channel and ships kernel
 * *source* per call.  This header replaces it with typed, stateless entry
 * points: each one names the reference call it stands in for.
 *
 * Conventions
 *  - Every function returns 0 on success, a nonzero MMP_E* code on failure;
 *    mmp_last_error() then returns a message (thread-local).
 *  - Pointers named x/a/b/out are device pointers from mmp_alloc (or views
 *    into them).  Strides and offsets are in ELEMENTS, like the reference's
 *    ndarray._strides (src/macmetalpy/ndarray.py:254-260).
 *  - All work is enqueued on one in-order HIP stream owned by the library;
 *    mmp_sync() waits for it.  Calls are asynchronous unless noted.
 *  - Scalars travel BY VALUE (pointer to host bytes of the given dtype); the
 *    reference uploads them as 1-element buffers (e.g. ndarray.py:1026).
 */
#ifndef MMP_HIP_H
#define MMP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define MMP_OK 0
#define MMP_E_NODEVICE 1   /* no HIP device / mmp_init failed            */
#define MMP_E_HIP 2        /* a HIP runtime call failed                   */
#define MMP_E_OOM 3        /* device allocation failed                    */
#define MMP_E_ARG 4        /* invalid argument (shape, size, null, ...)   */
#define MMP_E_UNSUPPORTED 5 /* op / dtype combination not implemented     */
#define MMP_E_RTC 6        /* hiprtc compile failed (log in last_error)   */
#define MMP_E_INJECTED 7   /* failure forced by mmp_debug_fail_next       */
#define MMP_E_WAIT 8       /* a device-side bounded wait ran out (a scan or
                              reduction result since the last sync may be
                              wrong); reported by mmp_sync / mmp_d2h      */

/* ---- dtype codes (numpy dtype -> code, see macmetalpy_amd/_abi.py) ---- */
#define MMP_BOOL 0
#define MMP_I16 1
#define MMP_U16 2
#define MMP_I32 3
#define MMP_U32 4
#define MMP_I64 5
#define MMP_U64 6
#define MMP_F16 7
#define MMP_F32 8
#define MMP_F64 9
#define MMP_BF16 10        /* matmul operands only */
#define MMP_NDTYPES 11

/* ---- unary elementwise ops (reference _kernels.py:84-331 names) ------- */
#define MMP_U_NEG 0
#define MMP_U_POSITIVE 1
#define MMP_U_ABS 2
#define MMP_U_SIGN 3
#define MMP_U_SQUARE 4
#define MMP_U_RECIPROCAL 5
#define MMP_U_SQRT 6
#define MMP_U_CBRT 7
#define MMP_U_EXP 8
#define MMP_U_EXP2 9
#define MMP_U_EXPM1 10
#define MMP_U_LOG 11
#define MMP_U_LOG2 12
#define MMP_U_LOG10 13
#define MMP_U_LOG1P 14
#define MMP_U_SIN 15
#define MMP_U_COS 16
#define MMP_U_TAN 17
#define MMP_U_ASIN 18
#define MMP_U_ACOS 19
#define MMP_U_ATAN 20
#define MMP_U_SINH 21
#define MMP_U_COSH 22
#define MMP_U_TANH 23
#define MMP_U_ASINH 24
#define MMP_U_ACOSH 25
#define MMP_U_ATANH 26
#define MMP_U_FLOOR 27
#define MMP_U_CEIL 28
#define MMP_U_RINT 29
#define MMP_U_TRUNC 30
#define MMP_U_DEGREES 31
#define MMP_U_RADIANS 32
#define MMP_NUNARY 33

/* ---- binary elementwise ops (reference _kernels.py:49-82, 220-250, 335-402) */
#define MMP_B_ADD 0
#define MMP_B_SUB 1
#define MMP_B_MUL 2
#define MMP_B_DIV 3           /* true_divide (floating dtypes only)          */
#define MMP_B_FLOOR_DIVIDE 4  /* numpy floor semantics, not truncation       */
#define MMP_B_MOD 5           /* numpy remainder: sign of the divisor        */
#define MMP_B_POWER 6
#define MMP_B_MAXIMUM 7
#define MMP_B_MINIMUM 8
#define MMP_B_FMAX 9
#define MMP_B_FMIN 10
#define MMP_B_ATAN2 11
#define MMP_B_HYPOT 12
#define MMP_B_FMOD 13
#define MMP_B_COPYSIGN 14
#define MMP_B_NEXTAFTER 15
#define MMP_B_LOGADDEXP 16
#define MMP_B_LOGADDEXP2 17
#define MMP_B_HEAVISIDE 18
#define MMP_NBINARY 19

/* ---- reductions and scans ---------------------------------------------- */
#define MMP_R_SUM 0
#define MMP_R_PROD 1
#define MMP_R_MAX 2
#define MMP_R_MIN 3
#define MMP_R_MEAN 4
#define MMP_R_ARGMAX 5
#define MMP_R_ARGMIN 6
/* NaN-ignoring variants (the reference's nan_reduction_shader and
 * nan_ops.nansum/nanprod/nanmax/nanmin/nanmean/nanargmax/nanargmin,
 * _kernels.py:599-732, nan_ops.py:112-612).  A slice with no non-NaN
 * element gives NaN for max/min/mean, 0 for sum, 1 for prod and, for the
 * arg ops, the index INT64_MAX (numpy raises "All-NaN slice"). */
#define MMP_R_NANSUM 7
#define MMP_R_NANPROD 8
#define MMP_R_NANMAX 9
#define MMP_R_NANMIN 10
#define MMP_R_NANMEAN 11
#define MMP_R_NANARGMAX 12
#define MMP_R_NANARGMIN 13
#define MMP_NREDUCE 14

#define MMP_S_CUMSUM 0
#define MMP_S_CUMPROD 1

/* ======================================================================== */
/* Runtime: replaces MetalBackend (_metal_backend.py:179-372)                */
/* ======================================================================== */

/* Select and initialise a device; creates the library's stream.
 * Replaces metalgpu `init()` (_metal_backend.py:221) called from
 * MetalBackend.__new__ (_metal_backend.py:197-219).  Idempotent. */
int mmp_init(int device);

/* Number of visible HIP devices (0 when none; never fails for that). */
int mmp_device_count(int *count);

/* Device facts: name (gcnArchName), CU count, total HBM bytes, wave size,
 * max threads per block.  Replaces maxThreadsPerGroup / threadExecutionWidth
 * (_metal_backend.py:259-263). */
int mmp_device_info(char *arch, int arch_len, int *cu_count,
                    int64_t *total_mem, int *wave_size, int *max_threads);

/* Message for the last failing call on this thread ("" if none).  The
 * reference has no error channel (metalgpu returns void). */
const char *mmp_last_error(void);

/* Device allocation from a caching pool.  Replaces createBuffer /
 * releaseBuffer (_metal_backend.py:225-231) and _BufferPool
 * (_metal_backend.py:23-77).  Frees are stream-ordered: a freed block is
 * reused only by work enqueued later on the same stream. */
int mmp_alloc(size_t bytes, void **ptr);
int mmp_free(void *ptr);
/* Return all cached (free) blocks to the driver (synchronises first). */
int mmp_empty_cache(void);
/* Bytes currently handed out / held in the cache. */
int mmp_memory_stats(size_t *in_use, size_t *cached);

/* Host<->device copies.  The reference reads unified memory through
 * getBufferPointer (_metal_backend.py:233-236, ndarray.py:576-618); HBM is
 * discrete, so get()/set() become explicit copies.  h2d/d2h are synchronous
 * with respect to the host buffer (it may be reused as soon as they return);
 * d2d is stream-ordered.  mmp_h2d of at most 1 MiB copies the bytes into
 * page-locked staging memory and queues the transfer on the library stream
 * without waiting for it (work queued later sees the data; the transfer is
 * a small copy kernel reading the mapped staging memory); larger copies
 * wait for the transfer.  mmp_d2h of
 * less than 32 KiB (48 KiB into pageable memory) runs a copy kernel into
 * mapped page-locked memory,
 * waits for the word the kernel writes after the bytes (the kernel runs
 * after all work queued before it) and copies out on the host; larger ones
 * are a DMA and a stream wait.  mmp_d2h returns
 * MMP_E_WAIT (after completing the copy) when a device-side bounded wait
 * ran out since the last check -- see mmp_wait_status. */
int mmp_h2d(void *dst, const void *src, size_t bytes);
int mmp_d2h(void *dst, const void *src, size_t bytes);
int mmp_d2d(void *dst, const void *src, size_t bytes);

/* Page-locked host blocks (cached by size) for arrays copied back to the
 * host: mmp_d2h into one runs at the link rate instead of being staged
 * through the runtime's bounce buffers.  The reference's get() reads
 * unified memory (ndarray.py:576-603), so it has no counterpart.
 * MMP_E_OOM when more than 4 GiB would be handed out at once (callers
 * then use pageable memory). */
int mmp_host_alloc(size_t bytes, void **ptr);
int mmp_host_free(void *ptr);

/* Wait for all enqueued work.  Replaces MetalBackend.synchronize
 * (_metal_backend.py:359-372: dispatch of `_sync` with wait=True).  Returns
 * MMP_E_WAIT when a device-side bounded wait ran out since the last check
 * (the flags live in pinned host memory, so the check costs no copy). */
int mmp_sync(void);

/* The library stream as an opaque hipStream_t (null before mmp_init), for
 * callers that order their own work against the library's, or that record
 * library calls into a HIP graph: hipStreamBeginCapture on this stream,
 * the calls, hipStreamEndCapture, then replay with hipGraphLaunch on it.
 * Only calls that neither allocate nor wait can be captured
 * (mmp_reduce_noalloc is one).  The reference keeps metalgpu's command
 * queue private (_metal_backend.py:197-221), so it has no counterpart. */
int mmp_stream(void **stream);

/* Stream-ordered timing events on the library stream (benchmarks). */
int mmp_event_create(void **ev);
int mmp_event_record(void *ev);
int mmp_event_elapsed_ms(void *start, void *end, float *ms);
int mmp_event_destroy(void *ev);

/* ======================================================================== */
/* Elementwise: replaces execute_kernel(elementwise_shader, "<op>_op", n,    */
/* [a, b, out]) from ndarray._binary_op / _unary_op (ndarray.py:960-1243)   */
/* ======================================================================== */

/* out[i] = op(x[i]) for contiguous x, out of `dtype` (MMP_U_*).
 * Reference: ndarray._unary_op -> elementwise_shader "<op>_op"
 * (ndarray.py:1237-1243, _kernels.py:84-331). */
int mmp_unary(int op, int dtype, int64_t n, const void *x, void *out);

/* out[i] = op(a[i], b[i]) for contiguous same-shape a, b, out (MMP_B_*).
 * Reference: ndarray._binary_op (ndarray.py:1105-1113). */
int mmp_binary(int op, int dtype, int64_t n, const void *a, const void *b,
               void *out);

/* Array-scalar form: scalar_side 0 => out = op(s, b[i]); 1 => op(a[i], s).
 * `scalar` points to one host value of `dtype`.  The reference instead
 * materialises creation.full(shape, s) on the host and uploads it
 * (ndarray.py:995-1026). */
int mmp_binary_scalar(int op, int dtype, int64_t n, const void *arr,
                      const void *scalar, int scalar_side, void *out);

/* Strided cast/copy: out (C-contiguous, `dst_dtype`) = (dst)x viewed with
 * `shape` / `x_strides` (elements, may be 0 for broadcast) from x + 0.
 * Covers astype (cast_op, _kernel_cache.py:44-58), copy (copy_buf :61-71),
 * broadcast materialisation (broadcast_nd :74-97) and view -> contiguous
 * (strided_copy :100-122).  ndim <= 8. */
int mmp_copy(int src_dtype, int dst_dtype, int ndim, const int64_t *shape,
             const void *x, const int64_t *x_strides, void *out);

/* Strided write: dst view (shape, dst_strides) = (dst)src view (shape,
 * src_strides).  Covers setitem on views (strided_write, offset_copy,
 * scalar_write: _kernel_cache.py:125-189). ndim <= 8. */
int mmp_copy_strided(int src_dtype, int dst_dtype, int ndim,
                     const int64_t *shape, const void *src,
                     const int64_t *src_strides, void *dst,
                     const int64_t *dst_strides);

/* out[i] = value for i < n (value: host bytes of dtype).  Replaces the
 * reference's fill_scalar kernel (_kernels.py:114-118). */
int mmp_fill(int dtype, int64_t n, const void *value, void *out);

/* ======================================================================== */
/* Reductions: replace ndarray._reduce (ndarray.py:1895-1963), _reduce_axis */
/* (ndarray.py:2015-2066) and reductions._parallel_argmax (:314-343)        */
/* ======================================================================== */

/* Input viewed as C-contiguous (outer, len, inner); reduces the middle
 * axis -> out (outer, inner) of `out_dtype`.  axis=None is
 * (1, n, 1).  op: MMP_R_SUM/PROD/MAX/MIN/MEAN and their MMP_R_NAN*
 * variants.  Floating sums/means accumulate in float64 and round once;
 * integer sums accumulate in 64-bit (numpy promotes int32 sums to int64).
 * max/min propagate NaN; the NaN variants skip it. */
int mmp_reduce(int op, int dtype, int out_dtype, int64_t outer, int64_t len,
               int64_t inner, const void *x, void *out);

/* mmp_reduce for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, kernels
 * and results as mmp_reduce, but the cross-workgroup partials and tickets
 * live in a static device array of 4 MiB (16 KiB of tickets + 4 MiB -
 * 16 KiB of partial words) set up by mmp_init, one copy per device held
 * until the process ends; the call itself allocates nothing and never
 * initialises the library (returns MMP_E_ARG before mmp_init).  Reductions
 * along the last axis split exactly as mmp_reduce does (at most 2047
 * partials: they always fit); strided reductions lower their split count
 * until the partials fit, so a floating sum may round differently from
 * mmp_reduce there.  A layout whose partials still do not fit is rejected
 * with MMP_E_ARG.  Each call first zeroes the partial words it will use
 * with a small kernel on the stream (not a memset, so a capture records a
 * kernel node): a captured call replays with the tag fixed at capture time,
 * and the clear keeps the previous replay's partials, which carry the same
 * tag, from being combined.  Every call on a device shares its array: direct calls,
 * from any host thread, are serialised and run in order on the library
 * stream; work that replays a captured call on another stream must not
 * overlap another use of the array on that device. */
int mmp_reduce_noalloc(int op, int dtype, int out_dtype, int64_t outer, int64_t len,
                       int64_t inner, const void *x, void *out);

/* Same view; out (outer, inner) int64 indices of the first max/min
 * (MMP_R_ARGMAX / MMP_R_ARGMIN); a NaN counts as the extreme (first NaN
 * wins), as np.argmax does.  MMP_R_NANARGMAX / MMP_R_NANARGMIN skip NaNs
 * (np.nanargmax); an all-NaN slice gives INT64_MAX. */
int mmp_argreduce(int op, int dtype, int64_t outer, int64_t len,
                  int64_t inner, const void *x, int64_t *out);

/* ======================================================================== */
/* Scan: replaces ndarray._prefix_scan (ndarray.py:2068-2152) and the 3-pass */
/* parallel_scan_shader (_kernels.py:1263-1360)                              */
/* ======================================================================== */

/* Inclusive scan along the middle axis of (outer, len, inner).
 * MMP_S_CUMSUM / MMP_S_CUMPROD.  out_dtype follows numpy (int32 -> int64,
 * float32 -> float32); floating scans carry a float64 running value whose
 * additions run in one fixed order, so repeated calls on the same input
 * give the same bits.  out must not overlap x (MMP_E_ARG): a tile may read
 * its predecessors' input. */
int mmp_scan(int op, int dtype, int out_dtype, int64_t outer, int64_t len,
             int64_t inner, const void *x, void *out);

/* ======================================================================== */
/* Sorting: replaces sorting._bitonic_sort_1d (sorting.py:59-196, behind    */
/* sort / argsort :21-56) and searchsorted's GPU path (sorting.py:218-263)   */
/* ======================================================================== */

/* Sort each of `rows` contiguous rows of `len` elements ascending (NaN
 * last).  out_values (rows*len of dtype) and / or out_indices (int64,
 * positions within the row, as np.argsort) may be null, not both.  With
 * out_indices, rows > 1 or stable != 0 the order is stable (equal to
 * kind='stable'; -0.0 == +0.0) and values are gathered from x bit for bit;
 * a 1-D values-only sort keeps every value's bits except the sign of NaNs.
 * rows*len <= 2^32 - 8192.  x must not alias the outputs. */
int mmp_sort(int dtype, int64_t rows, int64_t len, const void *x, void *out_values,
             int64_t *out_indices, int stable);

/* out[i] = insertion index of values[i] into sorted[0..n) (ascending, NaN
 * last): the first such index (side_right = 0) or the last (1). */
int mmp_searchsorted(int dtype, int64_t n, const void *sorted, int64_t m,
                     const void *values, int side_right, int64_t *out);

/* out[i] = src[indices[i]] for elements of `itemsize` (1, 2, 4, 8) bytes;
 * an index outside [0, nsrc) reads nothing and yields 0 (callers check
 * ranges).  Replaces the host gathers of take / fancy indexing
 * (indexing.py) on the sort path. */
int mmp_take(int itemsize, int64_t nsrc, const void *src, int64_t n,
             const int64_t *indices, void *out);

/* ---------------------------------------------------------- indexing
 * Advanced indexing and the indexing routines on the device.  Replace the
 * reference's host paths: ndarray.__getitem__ / __setitem__ with integer
 * or boolean arrays (ndarray.py:874-891, 943-957, NumPy on the host) and
 * indexing.py (take, put, putmask, place, compress, extract, nonzero,
 * flatnonzero, argwhere: NumPy on the host, indexing.py:24-391). */

/* Gather rows: out row i (row_words words of `word` = 1, 2, 4, 8 or 16
 * bytes) = the row_words words starting at word offsets[i] * unit of src.
 * Words outside [0, src_bytes / word) read as 0.  wrap > 0 makes offsets
 * row indices of an axis of length wrap: negatives count from the end and
 * an index outside [-wrap, wrap) reads 0 and sets *flag (flag may be
 * NULL) -- NumPy's IndexError, checked by the caller after the call.
 * src and out must be aligned to `word`. */
int mmp_gather(int word, const void *src, int64_t src_bytes, const int64_t *offsets,
               int64_t unit, int64_t wrap, uint32_t *flag, int64_t n, int64_t row_words,
               void *out);

/* Scatter rows: the row_words words at word offsets[i] * unit of dst =
 * row i of src (src_rows = n), or its only row (src_rows = 1).  Targets
 * outside dst are skipped; when two offsets are equal, which row lands is
 * unspecified (as for NumPy's advanced assignment). */
int mmp_scatter(int word, void *dst, int64_t dst_bytes, const int64_t *offsets, int64_t unit,
                int64_t n, int64_t row_words, const void *src, int64_t src_rows);

/* Positions of the selected elements: incl is the inclusive int64 count
 * (cumsum) of a mask of n elements, count = incl[n - 1]; out[k] = the
 * position of the k-th selected element, k < count. */
int mmp_nonzero(int64_t n, const int64_t *incl, int64_t count, int64_t *out);

/* Boolean-mask compaction straight from the mask's bytes (any nonzero byte
 * selects), by tiles of 4096 elements.  Replaces the same NumPy nonzero the
 * reference's mask indexing and nonzero / flatnonzero / argwhere run on the
 * host (ndarray.py:874-891, indexing.py:370-391).
 * mmp_mask_tile_counts: tile_incl[t] = number of selected elements in tiles
 * 0..t (ceil(n / 4096) entries); the last entry is the total.
 * mmp_mask_positions: out[k] = position of the k-th selected element, given
 * tile_incl from the first call on the same mask (out holds the total). */
int mmp_mask_tile_counts(int64_t n, const void *mask, uint64_t *tile_incl);
int mmp_mask_positions(int64_t n, const void *mask, const uint64_t *tile_incl, int64_t *out);
/* The selected elements (word = 1, 2, 4 or 8 bytes each) of src, a
 * contiguous array of the mask's n elements, packed in order into out:
 * a[mask] for a mask of a's shape (reference ndarray.py:874-891). */
int mmp_mask_compact(int word, int64_t n, const void *mask, const uint64_t *tile_incl,
                     const void *src, void *out);

/* Integer counts (replace the NumPy host calls behind bincount / histogram,
 * math_ext.py).  counts (int64) are zeroed first, then:
 * mmp_bincount: counts[v] = number of integer elements equal to v, for v in
 * [0, nbins) (dtype MMP_BOOL .. MMP_U64; other values are not counted).
 * mmp_histogram: counts[b] = number of elements with edges[b] <= x <
 * edges[b+1] (the last bin also takes x == edges[nedges-1]), compared in
 * double; NaN and out-of-range values are not counted (dtype MMP_I16,
 * MMP_U16, MMP_I32, MMP_U32, MMP_F16, MMP_F32, MMP_F64; nedges >= 2). */
int mmp_bincount(int dtype, int64_t n, const void *x, int64_t nbins, int64_t *counts);
int mmp_histogram(int dtype, int64_t n, const void *x, int64_t nedges, const double *edges,
                  int64_t *counts);

/* ======================================================================== */
/* Dense factorizations: replace the reference's NumPy / LAPACK calls in    */
/* linalg.py (solve, inv, det, slogdet :37-61, 149-159; cholesky :83-88;    */
/* qr :97-105; eigh, eigvalsh :63-69, 122-127; svd, svdvals, pinv,          */
/* matrix_rank, cond, lstsq :71-81, 129-183, 269-274).  Batches of          */
/* contiguous row-major matrices, dtype MMP_F32 or MMP_F64, one workgroup   */
/* per matrix, batch <= 2^31 - 1.                                           */
/* ======================================================================== */

/* In-place LU with partial pivoting of `batch` n x n matrices (n <= 32768):
 * unit-lower L below the diagonal, U on and above it; piv[b*n + k] = the
 * row swapped with row k at step k (0-based); info[b] = 1-based index of
 * the first exactly-zero pivot, 0 if none. */
int mmp_lu(int dtype, void *a, int64_t batch, int64_t n, int32_t *piv, int32_t *info);

/* Solves A X = B in place of b (n x nrhs per matrix) from mmp_lu's output. */
int mmp_lu_solve(int dtype, const void *lu, const int32_t *piv, void *b, int64_t batch, int64_t n,
                 int64_t nrhs);

/* In-place lower Cholesky factor (upper triangle zeroed) of symmetric
 * positive-definite matrices read from their lower triangle; info[b] =
 * 1-based index of the first non-positive pivot, 0 if none. */
int mmp_cholesky(int dtype, void *a, int64_t batch, int64_t n, int32_t *info);

/* Householder QR of m x n matrices in place: R on and above the diagonal,
 * reflector vectors (implicit leading 1) below it, tau[b*min(m,n) + k]
 * (LAPACK geqrf's convention). */
int mmp_qr(int dtype, void *a, void *tau, int64_t batch, int64_t m, int64_t n);

/* The first qcols (min(m,n) <= qcols <= m) columns of Q = H_0 ... H_{k-1}
 * from mmp_qr's output, into q (m x qcols per matrix). */
int mmp_qr_q(int dtype, const void *a, const void *tau, int64_t batch, int64_t m, int64_t n,
             int64_t qcols, void *q);

/* Cyclic Jacobi eigen-decomposition of symmetric n x n matrices (n <= 2048):
 * a is overwritten with a nearly diagonal matrix holding the eigenvalues
 * (unsorted) on its diagonal, v (n x n) receives the eigenvectors as
 * columns; sweeps[b] = Jacobi sweeps used (at most 60). */
int mmp_eigh(int dtype, void *a, void *v, int64_t batch, int64_t n, int32_t *sweeps);

/* One-sided Jacobi: rotates the rows of w (rows x len, rows <= len,
 * rows <= 8192) until they are mutually orthogonal, applying the same
 * rotations to vt (rows x rows, set to I first); the row norms of w are
 * then the singular values.  sweeps[b] = sweeps used (at most 60). */
int mmp_svd(int dtype, void *w, void *vt, int64_t batch, int64_t rows, int64_t len, int32_t *sweeps);

/* ======================================================================== */
/* Matmul: replaces ndarray.__matmul__ + matmul_shader (ndarray.py:1398-1450,*/
/* _kernels.py:740-759); batched form replaces linalg_top.matmul's CPU path */
/* (linalg_top.py:105-106)                                                  */
/* ======================================================================== */

/* C[b] = A[b] @ B[b] for b < batch; A (M,K) row stride lda, B (K,N) row
 * stride ldb, C (M,N) row stride ldc; batch strides sA/sB/sC in elements
 * (0 broadcasts an operand).  dtype: MMP_F32, MMP_F16, MMP_BF16, MMP_F64
 * (float accumulation in fp32 for 16-bit inputs, fp64 for f64) or an
 * integer dtype (exact, wrapping). */
int mmp_matmul(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K,
               const void *A, int64_t lda, int64_t sA, const void *B,
               int64_t ldb, int64_t sB, void *C, int64_t ldc, int64_t sC);

/* ======================================================================== */
/* Runtime compilation: replaces createLibraryFromString + setFunction +    */
/* runFunction (_metal_backend.py:237-257, 313-357) for the fusion engine  */
/* (_fusion.py:443-486) and RawKernel (raw_kernel.py:32-62)                 */
/* ======================================================================== */

/* Compile HIP C++ `src` with hiprtc for the current device's arch (gfx950)
 * and return a kernel handle for `name`.  Cached by (src, name, options). */
int mmp_rtc_compile(const char *src, const char *name, const char *options,
                    void **kernel);

/* Compile only (no device needed): writes the code object size to
 * *code_size and copies it to `code` when code_cap is large enough. */
int mmp_rtc_build(const char *src, const char *options, const char *arch,
                  void *code, size_t code_cap, size_t *code_size);

/* Launch with a grid given in BLOCKS (HIP convention). args: kernel
 * parameter pointers, one per kernel argument.  The reference's RawKernel
 * gives a grid in threads (Metal dispatchThreads, raw_kernel.py:46-59); the
 * Python RawKernel turns that into uniform workgroups that divide it. */
int mmp_rtc_launch(void *kernel, const uint32_t *grid3, const uint32_t *block3,
                   uint32_t shared_bytes, void **args);

/* Launch exactly threads3 work-items (Metal's dispatchThreads, as the
 * reference's RawKernel and MetalBackend.execute_kernel dispatch:
 * raw_kernel.py:46-59, _metal_backend.py:313-357) in workgroups of block3;
 * a dimension that block3 does not divide gets a partial last workgroup
 * whose missing work-items do not run.  Kernels compiled by mmp_rtc_compile
 * assume uniform workgroups, so blockDim is the full block3 extent in every
 * workgroup and blockIdx * blockDim + threadIdx is the global index.
 * block3's product must be 1..1024. */
int mmp_rtc_launch_threads(void *kernel, const uint32_t *threads3, const uint32_t *block3,
                           uint32_t shared_bytes, void **args);

/* ---- device-side wait status ------------------------------------------ */
/* Split reductions and scans combine results across workgroups with
 * bounded waits; a wait that runs out records a flag (pinned host memory,
 * written by the kernel) and lets the kernel finish instead of hanging.
 * Waits for the library stream, stores the flags raised since the last
 * check in *flags (bit 0: a scan row tail found no prefix, bit 1: reduction combine) and
 * clears them.  Non-zero means a result produced since the last check may
 * be wrong; mmp_sync and mmp_d2h report the same flags as MMP_E_WAIT.  No
 * counterpart in the reference (its Metal scan and reductions use
 * separate passes). */
int mmp_wait_status(uint32_t *flags);

/* ---- test hooks -------------------------------------------------------- */
/* Make the next `count`-th call of kind (1 = mmp_alloc, 2 = mmp_rtc_compile,
 * 3 = kernel launch) fail with MMP_E_INJECTED.  Kind 4: the `count`-th next
 * split reduction or scan waits for a tag that its writers never write,
 * with a spin limit of 64: a reduction's bounded wait runs out at once (the
 * kernel still finishes) and the next mmp_sync / mmp_d2h returns
 * MMP_E_WAIT; a scan's tiles find no predecessor descriptor and sum their
 * predecessors' inputs themselves (the result stays exact).  count 0
 * disables. */
int mmp_debug_fail_next(int kind, int count);

#ifdef __cplusplus
}
#endif

#endif /* MMP_HIP_H */
