/*
 * jlust_hip.h -- C ABI of libjlust_hip.so, the MI355X (gfx950) sparse hot path
 * of JLUST: CSR/COO SpMV, CSR SpMM, CSR SDDMM and BSR SpMM.
 *
 * This is the surface a JLUST `ext/HIPExt` package extension reaches through
 * `ccall` (or any FFI: Python ctypes in this repository's host mirror).
 * Each entry point replaces one `execute(::EmitterBackend, ::Op{...}, ...)`
 * method of the reference; the citation above each declaration names it.
 *
 * Conventions (all entry points):
 *  - Plain device pointers and sizes only.  Every array is owned by the caller
 *    and must stay alive until the stream work completes (the Julia side keeps
 *    it alive through the USTensor `owner` field, src/tensor.jl:42).
 *  - Index arrays are Int32 and carry the tensor's index origin
 *    (`origin` = 1 for OneBased, 0 for ZeroBased, src/tensor.jl:3-5); kernels
 *    subtract it at use, like `_origin_off` (ext/KernelAbstractionsExt/ops/
 *    _walker.jl:125-128).
 *  - Dense matrices are column-major (Julia arrays) with a leading dimension
 *    `ld*` >= their row count, so views (`SubArray` columns) work.
 *  - alpha and beta are given in the value type T (the reference casts them to
 *    T first, ext/KernelAbstractionsExt/ops/spmv.jl:377-378).  beta == 0 makes
 *    the output write-only: it is never read, so NaN/Inf in it do not
 *    propagate (the reference's Tiled/ColFirst SpMM and its SDDMM read it
 *    anyway, so a NaN there would reach the output; here it does not).
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and
 *    returns without synchronising.  Entry points are reentrant.  The library
 *    keeps one scratch buffer per (device, stream) for the SpMV/SpMM partial
 *    results, so concurrent calls must use different streams.  The buffer
 *    grows on demand and an outgrown one is kept, never freed, so work already
 *    queued and HIP graphs that captured a call stay valid.  Capturing a call
 *    in a graph: make one call of the same size on the capturing stream first
 *    (no allocation may happen inside a capture); prepared plans own their
 *    buffers and need no such warm-up.
 *  - Return value: a jlust_status code.  A message for the last failure on the
 *    calling thread is available from jlust_hip_last_error().
 *  - There is no CPU fallback: with no usable GPU every compute entry point
 *    returns JLUST_STATUS_NO_DEVICE.
 */
#ifndef JLUST_HIP_H
#define JLUST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JLUST_HIP_ABI_VERSION 2

typedef void *jlust_stream_t;                 /* hipStream_t */
typedef struct jlust_spmv_plan *jlust_spmv_plan_t;
typedef struct jlust_spmv_graph *jlust_spmv_graph_t;
typedef struct jlust_convert *jlust_convert_t;
typedef struct jlust_spmm_plan *jlust_spmm_plan_t;
typedef struct jlust_sddmm_plan *jlust_sddmm_plan_t;
typedef struct jlust_bsr_plan *jlust_bsr_plan_t;
typedef struct jlust_bsr_spmv_plan *jlust_bsr_spmv_plan_t;

/*
 * Status codes.  The Julia side maps them onto the reference's exception
 * types (src/errors.jl:1-9):
 *   INVALID_ARGUMENT       -> IncompatibleExtents / ArgumentError
 *   UNSUPPORTED_VALUE_TYPE -> UnsupportedValueType
 *   UNSUPPORTED_FORMAT     -> UnsupportedFormat
 *   NONCANONICAL_STORAGE   -> NonCanonicalStorage
 *   INDEX_ORIGIN           -> IndexOriginMismatch
 */
enum jlust_status {
    JLUST_STATUS_SUCCESS = 0,
    JLUST_STATUS_INVALID_ARGUMENT = 1,
    JLUST_STATUS_UNSUPPORTED_VALUE_TYPE = 2,
    JLUST_STATUS_UNSUPPORTED_FORMAT = 3,
    JLUST_STATUS_NONCANONICAL_STORAGE = 4,
    JLUST_STATUS_INDEX_ORIGIN = 5,
    JLUST_STATUS_HIP_ERROR = 6,
    JLUST_STATUS_NO_DEVICE = 7,
    JLUST_STATUS_OUT_OF_MEMORY = 8,
    JLUST_STATUS_STREAM_CAPTURING = 9,  /* graph launch onto a capturing stream */
    JLUST_STATUS_UNSUPPORTED_INDEX_TYPE = 10  /* an index beyond the Int32 kernels' range */
};

/* ---------------------------------------------------------------- library */

/* ABI version (JLUST_HIP_ABI_VERSION of the build).  Version 2: the
 * update_values entry points of the SpMV and SpMM plans take a stream and
 * are stream-ordered. */
int jlust_hip_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char *jlust_hip_last_error(void);

/*
 * Loads the library's device code on the current device now (no counterpart
 * in the reference; for callers that want the cost at start-up, such as
 * servers).  The runtime otherwise loads each translation unit's code object,
 * and each rocPRIM instantiation, at its first launch, which adds tens of
 * milliseconds to the first call that needs it (the first prepared SpMV plan
 * of a process: about 35 ms of its first build).  Runs a few tiny sorts and
 * scans on `stream` and synchronises it; idempotent.
 */
int jlust_hip_preload(jlust_stream_t stream);

/* Name of the current device's ISA, e.g. "gfx950", into buf. */
int jlust_hip_device_arch(char *buf, size_t len);

/*
 * Host-side structural check of a CSR pattern already copied to the host:
 * rowptr monotone from `origin` to nnz+origin, column indices within
 * [origin, n+origin), and (if require_sorted) strictly increasing per row.
 * Mirrors `validate_storage` (src/backends.jl:309-316), which the reference
 * limits to the value-buffer length; this opt-in deep check reports
 * JLUST_STATUS_NONCANONICAL_STORAGE.  No GPU needed.
 */
int jlust_hip_check_csr(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                        const int32_t *rowptr_host, const int32_t *colind_host,
                        int require_sorted);

/*
 * Device-side checks of index arrays already on the GPU (the same opt-in deep
 * checks beside validate_storage, src/backends.jl:309-316; no counterpart in
 * the reference's kernels).  check_pos: pos[nouter+1] starts at origin, ends
 * at nnz + origin and never decreases (a CSR rowptr, CSC colptr, DCSR or BSR
 * segment pointer).  check_crd: len coordinates within [origin, extent +
 * origin), strictly increasing when strictly_increasing != 0 (a DCSR's stored
 * rows).  Either returns JLUST_STATUS_NONCANONICAL_STORAGE on a violation.
 * Synchronises `stream` (one flag word read back).
 */
int jlust_hip_check_pos_i32(int64_t nouter, int64_t nnz, int32_t origin,
                            const int32_t *pos, jlust_stream_t stream);
/*
 * Int64 index buffers (the walker keeps the index type as stored,
 * ext/KernelAbstractionsExt/ops/_walker.jl:105-110) narrowed to the Int32
 * the kernels take: dst[i] = src[i] for n entries.  An index outside Int32's
 * range, or n >= 2^31, returns JLUST_STATUS_UNSUPPORTED_INDEX_TYPE (the
 * reference's UnsupportedIndexType, src/errors.jl:4).  Synchronises `stream`
 * (one flag word read back).
 */
int jlust_hip_narrow_index_i64(int64_t n, const int64_t *src, int32_t *dst,
                               jlust_stream_t stream);
int jlust_hip_check_crd_i32(int64_t len, int64_t extent, int32_t origin,
                            int strictly_increasing, const int32_t *crd,
                            jlust_stream_t stream);

/*
 * Index passes of the COO/CSC operators (no counterpart in the reference's
 * interface; the steps its scatter and atomic paths avoid by adding in place,
 * ext/KernelAbstractionsExt/ops/spmm.jl:412-416):
 *  - expand_pos: crd_out[p] = the outer coordinate of entry p --
 *    outer_crd[s] for the segment s of pos holding p, or s + origin when
 *    outer_crd is NULL (a CSC colptr into one column per entry).  pos is
 *    checked as by check_pos first (synchronises `stream`).
 *  - row_order: the row order of COO (format JLUST_FORMAT_COO, idx1 = rows,
 *    idx2 = cols) or CSC (JLUST_FORMAT_CSC, idx1 = colptr[n+1], idx2 =
 *    rowind) entries: rowptr[m+1] (origin-based) always; perm[q] = the source
 *    position of row-ordered entry q (a stable order: ties keep storage
 *    order) and cols[q] = its column, with *reordered = 1, unless the COO rows
 *    were already non-decreasing (*reordered = 0, perm and cols untouched).
 *    Caller-owned outputs: rowptr m+1, perm and cols nnz entries.
 *    Synchronises `stream`.
 *  - gather: dst[i] = src[perm[i]], i < n (values into a row order), on
 *    `stream`.
 */
int jlust_hip_expand_pos_i32(int64_t nouter, int64_t nnz, int32_t origin,
                             const int32_t *pos, const int32_t *outer_crd,
                             int32_t *crd_out, jlust_stream_t stream);
int jlust_hip_row_order_i32(int32_t format, int64_t m, int64_t n, int64_t nnz,
                            int32_t origin, const int32_t *idx1,
                            const int32_t *idx2, int32_t *rowptr,
                            int32_t *perm, int32_t *cols, int32_t *reordered,
                            jlust_stream_t stream);
int jlust_hip_gather_f64(int64_t n, const int32_t *perm, const double *src,
                         double *dst, jlust_stream_t stream);
int jlust_hip_gather_f32(int64_t n, const int32_t *perm, const float *src,
                         float *dst, jlust_stream_t stream);

/* ----------------------------------------------------------------- SpMV */

/*
 * y = alpha*A*x + beta*y, A m x n CSR (rowptr[m+1], colind[nnz], val[nnz]).
 * Replaces execute(::EmitterBackend, ::Op{:SpMV,Tuple{CSR,Dense,Dense}}, ...)
 * (ext/KernelAbstractionsExt/ops/spmv.jl:371-504, CSR branch :449-502).
 * nnz-balanced merge-path tiles, so any row-length distribution is balanced.
 */
int jlust_hip_csr_spmv_f64_i32(int64_t m, int64_t n, int64_t nnz,
                               int32_t origin, const int32_t *rowptr,
                               const int32_t *colind, const double *val,
                               double alpha, const double *x, double beta,
                               double *y, jlust_stream_t stream);
int jlust_hip_csr_spmv_f32_i32(int64_t m, int64_t n, int64_t nnz,
                               int32_t origin, const int32_t *rowptr,
                               const int32_t *colind, const float *val,
                               float alpha, const float *x, float beta,
                               float *y, jlust_stream_t stream);

/*
 * jlust_hip_csr_spmv_f64_i32 without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results (bit for bit) as the plain call; the
 * merge path's carry slots live in a static device array of the library
 * (64 KiB per device, 4096 slots, held until the process ends) instead of the
 * per-stream scratch buffer, so the call never calls hipMalloc, hipFree or an
 * allocating library routine.  Any matrix size is accepted: the grid needs
 * at most one slot per resident workgroup (2048 on MI355X); a device whose
 * grid would need more than 4096 slots gets INVALID_ARGUMENT.  Every call on
 * one device shares that array, so calls that overlap in time on one device
 * (two streams, two host threads) race; order them.
 */
int jlust_hip_csr_spmv_f64_i32_noalloc(int64_t m, int64_t n, int64_t nnz,
                                       int32_t origin, const int32_t *rowptr,
                                       const int32_t *colind, const double *val,
                                       double alpha, const double *x,
                                       double beta, double *y,
                                       jlust_stream_t stream);

/*
 * Prepared SpMV: analysis once (the merge-path partition of the pattern),
 * execute many times, refresh the value pointer without re-analysis.
 * Replaces prepare(::EmitterBackend, SpMVOp, u_A) / execute(h, ...)
 * (ext/KernelAbstractionsExt/ops/spmv.jl:518-544) and the cuSPARSE handle
 * contract prepare -> execute(h) -> update_values! (ext/CUDAExt/ops/
 * spmv.jl:7-83, src/ops.jl:179-188).  value_type: 0 = f64, 1 = f32.
 * The plan records the pointers given here; they must outlive the plan.
 */
int jlust_hip_csr_spmv_plan_create(int64_t m, int64_t n, int64_t nnz,
                                   int32_t origin, int value_type,
                                   const int32_t *rowptr,
                                   const int32_t *colind, const void *val,
                                   jlust_stream_t stream,
                                   jlust_spmv_plan_t *plan_out);
int jlust_hip_csr_spmv_plan_update_values(jlust_spmv_plan_t plan,
                                          const void *val,
                                          jlust_stream_t stream);
int jlust_hip_csr_spmv_plan_execute_f64(jlust_spmv_plan_t plan, double alpha,
                                        const double *x, double beta,
                                        double *y, jlust_stream_t stream);
int jlust_hip_csr_spmv_plan_execute_f32(jlust_spmv_plan_t plan, float alpha,
                                        const float *x, float beta, float *y,
                                        jlust_stream_t stream);
int jlust_hip_csr_spmv_plan_destroy(jlust_spmv_plan_t plan);

/*
 * Which values a plan reads.  Merge and vector plans read the value buffer
 * they were given (plan_create or the last update_values), so values stored
 * into it in place are seen by the next execute.  The sliced and binned
 * layouts, and COO plans whose entries were reordered, run on a permuted copy
 * of the values: execute then uses the values as of plan_create or the last
 * update_values / execute_values, the cuSPARSE handle contract where values
 * change through update_values! (ext/CUDAExt/ops/spmv.jl:40-43,63-78).
 *
 * execute_values is the form that takes A at every call,
 * execute(h::EmitterSpMVHandle, A, x, y) (ext/KernelAbstractionsExt/ops/
 * spmv.jl:531-544): it reads `val` (nnz values, the plan's pattern) as they
 * are when the call's work runs on `stream`, whatever the plan kind: a copy
 * is refreshed on `stream` before the product (one gather of the values
 * through the stored permutation), and `val` becomes the plan's values for
 * later executes.  update_values makes `val` the plan's values with the same
 * refresh enqueued on `stream` and no product, like the reference's
 * descriptor swap (ext/CUDAExt/ops/spmv.jl:40-43): nothing is waited for on
 * the host or on other streams, and executes ordered after it on `stream`
 * see the new values.  Executes and updates of one plan on different streams
 * must be ordered by the caller: they share the plan's partial sums and
 * value copy.
 */
int jlust_hip_csr_spmv_plan_execute_values_f64(jlust_spmv_plan_t plan,
                                               const double *val, double alpha,
                                               const double *x, double beta,
                                               double *y, jlust_stream_t stream);
int jlust_hip_csr_spmv_plan_execute_values_f32(jlust_spmv_plan_t plan,
                                               const float *val, float alpha,
                                               const float *x, float beta,
                                               float *y, jlust_stream_t stream);

/*
 * A plan execution recorded once as a HIP graph and replayed on any stream of
 * the plan's device: the reference's GPU block products capture their SpMV
 * with CUDA.capture/instantiate and replay it with CUDA.launch, one graph per
 * (pointer(y), pointer(x)) (ext/CUDAExt/ops/block_mul.jl:233-267, 751-786).
 * capture records y = alpha*A*x + beta*y with these pointers and coefficients
 * (on a private stream, thread-local capture mode; nothing runs).  A launch
 * reads the buffers the captured kernels were given as they are then: a merge
 * or vector plan's value buffer (values stored into it in place are seen), or
 * the value copy of a sliced, binned or reordered-COO plan (refreshed in place
 * by update_values / execute_values, which are then seen).  update_values or
 * execute_values with another value pointer on a merge or vector plan needs a
 * new capture.  launch onto a stream that is itself being
 * captured returns JLUST_STATUS_STREAM_CAPTURING without launching (execute
 * the plan instead, so the outer capture records its kernels, as the
 * reference does under CUDA.is_capturing()).  destroy drains the device
 * first.  The plan must outlive its graphs.
 */
int jlust_hip_csr_spmv_plan_capture_f64(jlust_spmv_plan_t plan, double alpha,
                                        const double *x, double beta, double *y,
                                        jlust_spmv_graph_t *graph_out);
int jlust_hip_csr_spmv_plan_capture_f32(jlust_spmv_plan_t plan, float alpha,
                                        const float *x, float beta, float *y,
                                        jlust_spmv_graph_t *graph_out);
int jlust_hip_spmv_graph_launch(jlust_spmv_graph_t graph, jlust_stream_t stream);
int jlust_hip_spmv_graph_destroy(jlust_spmv_graph_t graph);

/* The kernel a plan runs (no counterpart in the reference; for diagnostics
 * and benchmarks): merge-path tiles, the vector kernel for short even rows
 * (*lanes_per_row lanes per row), XCD column slices, or the LDS-binned
 * two-pass layout (x slices and y bins held in LDS); *device_bytes (may be
 * NULL) is the device memory the plan holds until it is destroyed.
 * The sliced and binned layouts copy the matrix; a plan whose layout cannot
 * be allocated (hipMalloc reports out of memory, or the layout with its
 * build temporaries would exceed the byte limit in the environment variable
 * JLUST_HIP_PLAN_MAX_BYTES, read at plan_create) uses the merge or vector
 * kernel on the caller's arrays instead, with no error. */
enum jlust_spmv_kernel {
    JLUST_SPMV_MERGE = 0,
    JLUST_SPMV_VECTOR = 1,
    JLUST_SPMV_SLICED = 2,
    JLUST_SPMV_BINNED = 3
};
int jlust_hip_csr_spmv_plan_info(jlust_spmv_plan_t plan, int32_t *kernel,
                                 int32_t *lanes_per_row,
                                 int64_t *device_bytes);

/*
 * Prepared COO SpMV (rows[nnz], cols[nnz] as coo_tensor stores them,
 * src/interop.jl:248-260): the entries are put in row order once (a stable
 * radix sort only when the rows are not already non-decreasing) and every
 * execute runs the CSR plan over them: y = alpha*A*x + beta*y with no
 * atomics and a run-to-run identical result.  Returns a plan used with the
 * jlust_hip_csr_spmv_plan_{execute,update_values,destroy} entry points;
 * update_values takes values in the caller's COO order.  The plan keeps
 * `cols` and `val` when the rows were already sorted (they must outlive it),
 * otherwise row-ordered copies.  A row index outside [origin, m + origin)
 * returns NONCANONICAL_STORAGE.  Replaces the COO branch of
 * execute(::EmitterBackend, ::Op{:SpMV}) (ext/KernelAbstractionsExt/ops/
 * spmv.jl:407-448) under the prepare/execute/update_values! handle contract
 * (ext/CUDAExt/ops/spmv.jl:7-83).  Synchronises `stream`.
 */
int jlust_hip_coo_spmv_plan_create(int64_t m, int64_t n, int64_t nnz,
                                   int32_t origin, int value_type,
                                   const int32_t *rows, const int32_t *cols,
                                   const void *val, jlust_stream_t stream,
                                   jlust_spmv_plan_t *plan_out);

/*
 * COO SpMV (rows[nnz], cols[nnz] as stored by coo_tensor, src/interop.jl:
 * 248-260): y = beta*y (zero-filled when beta == 0), then y += alpha*A*x.
 * Replaces the COO branch of execute(::EmitterBackend, ::Op{:SpMV}, ...)
 * (ext/KernelAbstractionsExt/ops/spmv.jl:407-448).  Rows need not be sorted;
 * sorted rows reduce atomic traffic (one add per row run per tile).
 */
int jlust_hip_coo_spmv_f64_i32(int64_t m, int64_t n, int64_t nnz,
                               int32_t origin, const int32_t *rows,
                               const int32_t *cols, const double *val,
                               double alpha, const double *x, double beta,
                               double *y, jlust_stream_t stream);
int jlust_hip_coo_spmv_f32_i32(int64_t m, int64_t n, int64_t nnz,
                               int32_t origin, const int32_t *rows,
                               const int32_t *cols, const float *val,
                               float alpha, const float *x, float beta,
                               float *y, jlust_stream_t stream);

/*
 * CSC SpMV (colptr[n+1], rowind[nnz], val[nnz], Formats.CSC): y = beta*y
 * (zero-filled when beta == 0), then y[row] += (alpha*val)*x[col] for every
 * stored entry, with atomics, in the reference's scatter mode for column-outer
 * formats (execute(::EmitterBackend, ::Op{:SpMV}), ext/KernelAbstractionsExt/
 * ops/spmv.jl:391-408).  The atomic order varies, so results vary in their
 * last bits run to run.  input_fn composes (apply it to x first); output_fn
 * does not, as in the reference (spmv.jl:396-399).
 */
int jlust_hip_csc_spmv_f64_i32(int64_t m, int64_t n, int64_t nnz,
                               int32_t origin, const int32_t *colptr,
                               const int32_t *rowind, const double *val,
                               double alpha, const double *x, double beta,
                               double *y, jlust_stream_t stream);
int jlust_hip_csc_spmv_f32_i32(int64_t m, int64_t n, int64_t nnz,
                               int32_t origin, const int32_t *colptr,
                               const int32_t *rowind, const float *val,
                               float alpha, const float *x, float beta,
                               float *y, jlust_stream_t stream);

/*
 * Elementwise transforms for SpMV's input_fn / output_fn
 * (execute(::EmitterBackend, ::Op{:SpMV}; input_fn, output_fn),
 * ext/KernelAbstractionsExt/ops/spmv.jl:371-374): f(v) of one kind.
 */
enum jlust_fn_kind {
    JLUST_FN_IDENTITY = 0,  /* v                        */
    JLUST_FN_AFFINE = 1,    /* a*v + b (not contracted) */
    JLUST_FN_ABS = 2,       /* |v|                      */
    JLUST_FN_SQUARE = 3,    /* v*v                      */
    JLUST_FN_SQRT = 4,      /* sqrt(v)                  */
    JLUST_FN_EXP = 5,       /* exp(v)                   */
    JLUST_FN_LOG = 6,       /* log(v)                   */
    JLUST_FN_RELU = 7       /* max(v, 0), NaN kept      */
};

/*
 * dst[i] = alpha*f(src[i]) + beta*dst[i] for i < n (beta == 0 writes dst
 * without reading it; dst == src allowed).  With alpha = 1, beta = 0 it is
 * in_fn.(x); after an SpMV into a row-sum vector t it is the row write
 * alpha*out_fn(t) + beta*y (spmv.jl:168-169).
 */
int jlust_hip_apply_fn_f64(int64_t n, int32_t kind, double a, double b,
                           const double *src, double alpha, double beta,
                           double *dst, jlust_stream_t stream);
int jlust_hip_apply_fn_f32(int64_t n, int32_t kind, float a, float b,
                           const float *src, float alpha, float beta,
                           float *dst, jlust_stream_t stream);

/*
 * Row gathers / scatters of DCSR products (src/named_formats.jl:27): a DCSR
 * SpMV or SpMM runs as the CSR product over its stored rows into a compact
 * result t, with t = y[rows] gathered first when beta != 0 and y[rows] = t
 * scattered after, so rows that are not stored stay untouched as in the
 * reference (ext/KernelAbstractionsExt/ops/spmv.jl:449-502, n_outer = stored
 * rows; spmm.jl:397-423).  gather: dst[s + c*ldd] = src[rows[s] - origin +
 * c*lds]; scatter: dst[rows[s] - origin + c*ldd] = src[s + c*lds], for
 * s < nrows, c < k; m = rows of the full operand; rows outside [0, m) are
 * skipped.
 */
int jlust_hip_gather_rows_f64(int64_t nrows, int64_t k, int32_t origin,
                              const int32_t *rows, int64_t m, const double *src,
                              int64_t lds, double *dst, int64_t ldd,
                              jlust_stream_t stream);
int jlust_hip_gather_rows_f32(int64_t nrows, int64_t k, int32_t origin,
                              const int32_t *rows, int64_t m, const float *src,
                              int64_t lds, float *dst, int64_t ldd,
                              jlust_stream_t stream);
int jlust_hip_scatter_rows_f64(int64_t nrows, int64_t k, int32_t origin,
                               const int32_t *rows, int64_t m, const double *src,
                               int64_t lds, double *dst, int64_t ldd,
                               jlust_stream_t stream);
int jlust_hip_scatter_rows_f32(int64_t nrows, int64_t k, int32_t origin,
                               const int32_t *rows, int64_t m, const float *src,
                               int64_t lds, float *dst, int64_t ldd,
                               jlust_stream_t stream);

/* ----------------------------------------------------------------- SpMM */

/*
 * C = alpha*A*B + beta*C, A m x n CSR, B n x k (ldb), C m x k (ldc), both
 * column-major.  skip_empty_rows leaves rows with no stored entry untouched
 * (the reference's guarded 2-D path, ext/KernelAbstractionsExt/ops/
 * spmm.jl:203,340).  Replaces execute(::EmitterBackend, ::Op{:SpMM}, ...)
 * (spmm.jl:397-423).
 */
int jlust_hip_csr_spmm_f64_i32(int64_t m, int64_t n, int64_t k, int64_t nnz,
                               int32_t origin, const int32_t *rowptr,
                               const int32_t *colind, const double *val,
                               double alpha, const double *B, int64_t ldb,
                               double beta, double *C, int64_t ldc,
                               int skip_empty_rows, jlust_stream_t stream);
int jlust_hip_csr_spmm_f32_i32(int64_t m, int64_t n, int64_t k, int64_t nnz,
                               int32_t origin, const int32_t *rowptr,
                               const int32_t *colind, const float *val,
                               float alpha, const float *B, int64_t ldb,
                               float beta, float *C, int64_t ldc,
                               int skip_empty_rows, jlust_stream_t stream);

/*
 * Prepared CSR SpMM for B and C of k columns: prepare(backend, SpMMOp, A;
 * n_cols = k) -> execute(h, B, C) -> update_values!(h, A), the cuSPARSE SpMM
 * handle contract (ext/CUDAExt/ops/spmm.jl:8-70, src/ops.jl:170-188).
 * Analysis once: the column chunk per pass for this k, and the rows longer
 * than 1024 entries, which are cut into segments of 256 entries computed in
 * parallel into partial rows and added back in segment order (one wave would
 * otherwise walk each such row alone).  Workspace owned by the plan: the
 * row-major copy of one column chunk of B and the partial rows, so an execute
 * allocates nothing.  Results equal jlust_hip_csr_spmm_* bit for bit on rows
 * that are not split, and are deterministic run to run.  The plan records
 * rowptr, colind and val (read in place at each execute: values stored into
 * val are seen); update_values points it at another value buffer (a plan of
 * jlust_hip_coo_spmm_plan_create whose entries were reordered gathers the
 * values into its row order on `stream` instead; executes ordered after it
 * on `stream` see them).  value_type: 0 = f64, 1 = f32.  Synchronises `stream` (the row analysis
 * reads rowptr on the host).  Executes of one plan must not overlap in time.
 */
int jlust_hip_csr_spmm_plan_create(int64_t m, int64_t n, int64_t k,
                                   int64_t nnz, int32_t origin, int value_type,
                                   const int32_t *rowptr,
                                   const int32_t *colind, const void *val,
                                   jlust_stream_t stream,
                                   jlust_spmm_plan_t *plan_out);
int jlust_hip_csr_spmm_plan_update_values(jlust_spmm_plan_t plan,
                                          const void *val,
                                          jlust_stream_t stream);
int jlust_hip_csr_spmm_plan_execute_f64(jlust_spmm_plan_t plan, double alpha,
                                        const double *B, int64_t ldb,
                                        double beta, double *C, int64_t ldc,
                                        int skip_empty_rows,
                                        jlust_stream_t stream);
int jlust_hip_csr_spmm_plan_execute_f32(jlust_spmm_plan_t plan, float alpha,
                                        const float *B, int64_t ldb,
                                        float beta, float *C, int64_t ldc,
                                        int skip_empty_rows,
                                        jlust_stream_t stream);
/* What the analysis found (no counterpart in the reference; diagnostics):
 * rows split into segments, segments, columns per pass, and whether the
 * entries of a COO/CSC plan were reordered (the plan then holds a copy of the
 * values in its row order). */
int jlust_hip_csr_spmm_plan_info(jlust_spmm_plan_t plan, int64_t *split_rows,
                                 int64_t *segments, int64_t *cols_per_pass,
                                 int32_t *reordered);
/* Drains the device, then frees the plan's workspace. */
int jlust_hip_csr_spmm_plan_destroy(jlust_spmm_plan_t plan);

/*
 * SpMM with a COO A (idx1 = rows[nnz], idx2 = cols[nnz], rows in any order)
 * or a CSC A (idx1 = colptr[n+1], idx2 = rowind[nnz]): C = alpha*A*B +
 * beta*C with B n x k (ldb), C m x k (ldc), column-major; beta == 0 makes C
 * write-only.  The reference runs COO as ColFirst and CSC in the walker's
 * scatter direction, pre-scaling C by beta and adding alpha*val*B[col, :]
 * into C[row, :] with atomics (execute(::EmitterBackend, ::Op{:SpMM}),
 * ext/KernelAbstractionsExt/ops/spmm.jl:331-335, 412-416).  Here the entries
 * are put in row order (a stable sort, only for COO rows that are not already
 * non-decreasing; always for CSC) into temporaries and the CSR SpMM runs on
 * them: each output is summed in one fixed order, so the result is the
 * same product, deterministic run to run.  A COO row outside [origin,
 * m + origin) or a CSC colptr that is not canonical is NONCANONICAL_STORAGE.
 * Synchronises `stream` (the analysis reads flags on the host and the
 * temporaries are freed on return).
 */
int jlust_hip_coo_spmm_f64_i32(int64_t m, int64_t n, int64_t k, int64_t nnz,
                               int32_t origin, const int32_t *rows,
                               const int32_t *cols, const double *val,
                               double alpha, const double *B, int64_t ldb,
                               double beta, double *C, int64_t ldc,
                               jlust_stream_t stream);
int jlust_hip_coo_spmm_f32_i32(int64_t m, int64_t n, int64_t k, int64_t nnz,
                               int32_t origin, const int32_t *rows,
                               const int32_t *cols, const float *val,
                               float alpha, const float *B, int64_t ldb,
                               float beta, float *C, int64_t ldc,
                               jlust_stream_t stream);
int jlust_hip_csc_spmm_f64_i32(int64_t m, int64_t n, int64_t k, int64_t nnz,
                               int32_t origin, const int32_t *colptr,
                               const int32_t *rowind, const double *val,
                               double alpha, const double *B, int64_t ldb,
                               double beta, double *C, int64_t ldc,
                               jlust_stream_t stream);
int jlust_hip_csc_spmm_f32_i32(int64_t m, int64_t n, int64_t k, int64_t nnz,
                               int32_t origin, const int32_t *colptr,
                               const int32_t *rowind, const float *val,
                               float alpha, const float *B, int64_t ldb,
                               float beta, float *C, int64_t ldc,
                               jlust_stream_t stream);

/*
 * Prepared COO or CSC SpMM (format JLUST_FORMAT_COO: idx1 = rows, idx2 =
 * cols; JLUST_FORMAT_CSC: idx1 = colptr, idx2 = rowind): the row order of the
 * entries once, into memory the plan owns, then a CSR SpMM plan over it --
 * the cuSPARSE SpMM handle contract (ext/CUDAExt/ops/spmm.jl:8-70) for the
 * formats the reference's SpMM takes (spmm.jl:412-416).  Returns a plan of
 * the jlust_hip_csr_spmm_plan_{execute,update_values,info,destroy} entry
 * points; update_values takes values in the caller's storage order and, when
 * the entries were reordered, gathers them into the plan's order on its
 * stream.  When COO rows were already non-decreasing the plan keeps `idx2`
 * and `val` by pointer (they must outlive it).  Synchronises `stream`.
 */
int jlust_hip_coo_spmm_plan_create(int32_t format, int64_t m, int64_t n,
                                   int64_t k, int64_t nnz, int32_t origin,
                                   int value_type, const int32_t *idx1,
                                   const int32_t *idx2, const void *val,
                                   jlust_stream_t stream,
                                   jlust_spmm_plan_t *plan_out);

/* ---------------------------------------------------------------- SDDMM */

/*
 * Cval[p] = alpha*dot(A[i,:], B[:,j]) + beta*Cval[p] for each stored (i, j)
 * of the CSR pattern C (m x n); A m x K (lda), B K x n (ldb), column-major.
 * When mask != NULL the dot term is multiplied by mask[p]:
 * Cval[p] = mask[p]*(alpha*dot) + beta*Cval[p]; mask may alias Cval.
 * Replaces execute(::EmitterBackend, ::Op{:SDDMM}, A, B, C; alpha, beta)
 * (ext/KernelAbstractionsExt/ops/sddmm.jl:49-65; body :23-30).
 */
int jlust_hip_csr_sddmm_f64_i32(int64_t m, int64_t n, int64_t K, int64_t nnz,
                                int32_t origin, const int32_t *rowptr,
                                const int32_t *colind, double alpha,
                                const double *A, int64_t lda, const double *B,
                                int64_t ldb, double beta, double *Cval,
                                const double *mask, jlust_stream_t stream);
int jlust_hip_csr_sddmm_f32_i32(int64_t m, int64_t n, int64_t K, int64_t nnz,
                                int32_t origin, const int32_t *rowptr,
                                const int32_t *colind, float alpha,
                                const float *A, int64_t lda, const float *B,
                                int64_t ldb, float beta, float *Cval,
                                const float *mask, jlust_stream_t stream);

/*
 * SDDMM with a COO mask (rows[nnz], cols[nnz] as coo_tensor stores them;
 * rows in any order): the same operator, outputs and mask values in the
 * mask's storage order.  Replaces the COO case of execute(::EmitterBackend,
 * ::Op{:SDDMM}) (ext/KernelAbstractionsExt/ops/sddmm.jl:49-65; reference
 * answer test/test_emitter.jl:289-307).  No analysis: a group of lanes per
 * entry reads A's row with stride lda; a prepared plan (below) puts the
 * entries in row order once and runs the CSR kernel instead.
 */
int jlust_hip_coo_sddmm_f64_i32(int64_t m, int64_t n, int64_t K, int64_t nnz,
                                int32_t origin, const int32_t *rows,
                                const int32_t *cols, double alpha,
                                const double *A, int64_t lda, const double *B,
                                int64_t ldb, double beta, double *Cval,
                                const double *mask, jlust_stream_t stream);
int jlust_hip_coo_sddmm_f32_i32(int64_t m, int64_t n, int64_t K, int64_t nnz,
                                int32_t origin, const int32_t *rows,
                                const int32_t *cols, float alpha,
                                const float *A, int64_t lda, const float *B,
                                int64_t ldb, float beta, float *Cval,
                                const float *mask, jlust_stream_t stream);

/*
 * SDDMM with a DCSR mask (rows[nout] stored rows, increasing; pos[nout+1];
 * cols[nnz]; src/named_formats.jl:27): the reference's walker with the
 * compressed outer level binding the stored row (execute(::EmitterBackend,
 * ::Op{:SDDMM}), ext/KernelAbstractionsExt/ops/sddmm.jl:49-65, outer walk
 * _walker.jl:323-392).  The CSR kernel runs over the stored rows, reading A's
 * row rows[r] for stored row r (clamped into [0, m)); outputs in the mask's
 * storage order.  Rows that are not stored have no outputs.
 */
int jlust_hip_dcsr_sddmm_f64_i32(int64_t m, int64_t n, int64_t K, int64_t nout,
                                 int64_t nnz, int32_t origin,
                                 const int32_t *rows, const int32_t *pos,
                                 const int32_t *cols, double alpha,
                                 const double *A, int64_t lda, const double *B,
                                 int64_t ldb, double beta, double *Cval,
                                 const double *mask, jlust_stream_t stream);
int jlust_hip_dcsr_sddmm_f32_i32(int64_t m, int64_t n, int64_t K, int64_t nout,
                                 int64_t nnz, int32_t origin,
                                 const int32_t *rows, const int32_t *pos,
                                 const int32_t *cols, float alpha,
                                 const float *A, int64_t lda, const float *B,
                                 int64_t ldb, float beta, float *Cval,
                                 const float *mask, jlust_stream_t stream);

/*
 * SDDMM with a CSC mask (colptr[n+1], rowind[nnz]): Cval[p] = alpha*dot(A[i,:],
 * B[:,j]) (*mask[p]) + beta*Cval[p] for the stored entry p at row i = rowind[p]
 * of column j, in the mask's storage order -- the operator's definition
 * (C <- alpha*(A*B) o sparsity(C) + beta*C, ext/KernelAbstractionsExt/ops/
 * sddmm.jl:1-6).  The reference's gather walker binds a CSC mask's outer
 * level (the column) as the row instead (sddmm.jl:23-30 with _walker.jl:
 * 271-314), computing dot(A[j,:], B[:,i]); that transposed reading is not
 * reproduced.  colptr is checked (NONCANONICAL_STORAGE) and expanded into one
 * column per entry, then the COO-mask kernel runs.  Synchronises `stream`.
 */
int jlust_hip_csc_sddmm_f64_i32(int64_t m, int64_t n, int64_t K, int64_t nnz,
                                int32_t origin, const int32_t *colptr,
                                const int32_t *rowind, double alpha,
                                const double *A, int64_t lda, const double *B,
                                int64_t ldb, double beta, double *Cval,
                                const double *mask, jlust_stream_t stream);
int jlust_hip_csc_sddmm_f32_i32(int64_t m, int64_t n, int64_t K, int64_t nnz,
                                int32_t origin, const int32_t *colptr,
                                const int32_t *rowind, float alpha,
                                const float *A, int64_t lda, const float *B,
                                int64_t ldb, float beta, float *Cval,
                                const float *mask, jlust_stream_t stream);

/*
 * Prepared SDDMM for a mask pattern C (m x n) and inner dimension K:
 * prepare(backend, SDDMMOp, A, B, C) -> execute(h, A, B, C) ->
 * update_values!(h, C), the cuSPARSE SDDMM handle contract (ext/CUDAExt/ops/
 * sddmm.jl:10-76).  mask_format is JLUST_FORMAT_CSR (idx1 = rowptr[m+1],
 * idx2 = colind[nnz]), JLUST_FORMAT_COO (idx1 = rows[nnz], idx2 =
 * cols[nnz]) or JLUST_FORMAT_CSC (idx1 = colptr[n+1], idx2 = rowind[nnz],
 * with the semantics of jlust_hip_csc_sddmm_*); DCSR masks take
 * jlust_hip_dcsr_sddmm_plan_create.  Analysis once: a COO or CSC mask is put
 * in row order (rowptr, the columns and the permutation back to storage
 * order, owned by the plan; a row outside [origin, m + origin) or a CSC
 * colptr that is not canonical is NONCANONICAL_STORAGE); the row blocks
 * that hold entries become work items of at most 4096 entries, so blocks
 * without entries cost nothing and a block holding a long row is shared by
 * several workgroups.  execute writes Cval (and reads mask) in the mask's
 * storage order, with the semantics of jlust_hip_csr_sddmm_*; the values of
 * C are not part of the plan, so update_values! needs no call here.  The
 * plan keeps the caller's rowptr/colind (CSR) or cols (COO whose rows were
 * already in order): they must outlive it.  Synchronises `stream`.
 */
int jlust_hip_sddmm_plan_create(int32_t mask_format, int64_t m, int64_t n,
                                int64_t K, int64_t nnz, int32_t origin,
                                int value_type, const int32_t *idx1,
                                const int32_t *idx2, jlust_stream_t stream,
                                jlust_sddmm_plan_t *plan_out);
/* Prepared SDDMM over a DCSR mask (the arrays of jlust_hip_dcsr_sddmm_*,
 * kept by pointer): work items over the stored rows, pos checked
 * (NONCANONICAL_STORAGE).  Used with the plan entry points above. */
int jlust_hip_dcsr_sddmm_plan_create(int64_t m, int64_t n, int64_t K,
                                     int64_t nout, int64_t nnz, int32_t origin,
                                     int value_type, const int32_t *rows,
                                     const int32_t *pos, const int32_t *cols,
                                     jlust_stream_t stream,
                                     jlust_sddmm_plan_t *plan_out);
int jlust_hip_sddmm_plan_execute_f64(jlust_sddmm_plan_t plan, double alpha,
                                     const double *A, int64_t lda,
                                     const double *B, int64_t ldb, double beta,
                                     double *Cval, const double *mask,
                                     jlust_stream_t stream);
int jlust_hip_sddmm_plan_execute_f32(jlust_sddmm_plan_t plan, float alpha,
                                     const float *A, int64_t lda,
                                     const float *B, int64_t ldb, float beta,
                                     float *Cval, const float *mask,
                                     jlust_stream_t stream);
/* Work items of the plan and whether a COO mask was reordered (diagnostics;
 * no counterpart in the reference). */
int jlust_hip_sddmm_plan_info(jlust_sddmm_plan_t plan, int64_t *work_items,
                              int32_t *reordered);
/* Drains the device, then frees the plan's tables. */
int jlust_hip_sddmm_plan_destroy(jlust_sddmm_plan_t plan);

/* ------------------------------------------------------------------ BSR */

/*
 * C = alpha*A*B + beta*C, A an mb x nb grid of bs x bs blocks in BSR
 * (browptr[mb+1], bcolind[nnzb], val[nnzb*bs*bs] block-major; row-major
 * inside a block when row_major_blocks != 0 = Formats.BSRRight, else
 * column-major = BSRLeft; src/named_formats.jl:106-128, storage as in
 * ext/CUDAExt/CUDAExt.jl:144-156).  B (nb*bs) x k (ldb), C (mb*bs) x k (ldc),
 * column-major.  bs == 16 runs on fp32 MFMA; other block sizes return
 * JLUST_STATUS_UNSUPPORTED_FORMAT (jlust_hip_bsr_expand_csr_i32 + the CSR
 * SpMM serve them).  The reference routes BSR SpMM through the
 * generic execute(::EmitterBackend, ::Op{:SpMM}) (KernelAbstractionsExt.jl:
 * 35-37), which does not compute it correctly; this entry point implements
 * the operator's definition.
 */
int jlust_hip_bsr_spmm_f32_i32(int64_t mb, int64_t nb, int64_t bs,
                               int64_t nnzb, int32_t origin,
                               const int32_t *browptr, const int32_t *bcolind,
                               const float *val, int row_major_blocks,
                               int64_t k, float alpha, const float *B,
                               int64_t ldb, float beta, float *C, int64_t ldc,
                               jlust_stream_t stream);
/* The same for Float64 values on the fp64 matrix cores (16 x 16 blocks; any
 * alignment, element access where values, B or C are not 32-byte aligned or
 * ldb, ldc are not multiples of 4).  Same reference operator as above. */
int jlust_hip_bsr_spmm_f64_i32(int64_t mb, int64_t nb, int64_t bs,
                               int64_t nnzb, int32_t origin,
                               const int32_t *browptr, const int32_t *bcolind,
                               const double *val, int row_major_blocks,
                               int64_t k, double alpha, const double *B,
                               int64_t ldb, double beta, double *C, int64_t ldc,
                               jlust_stream_t stream);

/*
 * y = alpha*A*x + beta*y for BSR of any b1 x b2 block shape (A (mb*b1) x
 * (nb*b2), storage as for jlust_hip_bsr_spmm_f32_i32 with bs = b1 x b2
 * blocks).  The reference's EmitterBackend claims SpMV for every sparse
 * format (KernelAbstractionsExt.jl:31-37).  Each scalar row sums its entries
 * in the order of its row in the CSR expansion below.  Block ranges and block
 * columns are clamped to the stored blocks and to [0, nb), so a malformed
 * browptr or bcolind gives wrong sums, never an out-of-bounds read; they are
 * not validated here (the expansion validates browptr's ends).
 */
int jlust_hip_bsr_spmv_f64_i32(int64_t mb, int64_t nb, int64_t b1, int64_t b2,
                               int64_t nnzb, int32_t origin,
                               const int32_t *browptr, const int32_t *bcolind,
                               const double *val, int row_major_blocks,
                               double alpha, const double *x, double beta,
                               double *y, jlust_stream_t stream);
int jlust_hip_bsr_spmv_f32_i32(int64_t mb, int64_t nb, int64_t b1, int64_t b2,
                               int64_t nnzb, int32_t origin,
                               const int32_t *browptr, const int32_t *bcolind,
                               const float *val, int row_major_blocks,
                               float alpha, const float *x, float beta,
                               float *y, jlust_stream_t stream);

/*
 * BSR of any b1 x b2 block shape and value type, expanded to CSR for the CSR
 * kernels: the route of BSR SpMM where the MFMA path above does not apply
 * (blocks other than 16 x 16).  The reference's
 * EmitterBackend claims SpMV and SpMM for every sparse format
 * (KernelAbstractionsExt.jl:31-37); its BSR layout is Formats.BSRRight /
 * BSRLeft((b1, b2)) (src/named_formats.jl:106-128).  Scalar row b1*R + r lists, for
 * each stored block q of block-row R in storage order, columns b2*bcol[q] + s,
 * s = 0..b2-1.  Every stored entry is kept, explicit zeros included, so the
 * product is the block definition's.  Outputs (caller's buffers, the input's
 * origin): rowptr[mb*b1 + 1], colind[nnzb*b1*b2], val_out[nnzb*b1*b2].
 * value_type: 0 = Float64, 1 = Float32.  A browptr that does not run from
 * origin to origin + nnzb is NONCANONICAL_STORAGE.  Reads two entries of browptr
 * back, so it synchronises `stream` (not capturable).
 */
int jlust_hip_bsr_expand_csr_i32(int64_t mb, int64_t b1, int64_t b2,
                                 int64_t nnzb, int32_t origin,
                                 const int32_t *browptr,
                                 const int32_t *bcolind, const void *val,
                                 int value_type, int row_major_blocks,
                                 int32_t *rowptr, int32_t *colind,
                                 void *val_out, jlust_stream_t stream);

/*
 * Prepared BSR SpMM, the BSR analyse handle (the cuSPARSE SpMM handle
 * contract, ext/CUDAExt/ops/spmm.jl:8-70: analysis and workspace once,
 * execute many times, update_values! for new values of the same pattern).
 * 16 x 16 blocks keep the MFMA kernels (fp32, with 16-byte aligned values
 * for BSRRight, or fp64) and read the caller's buffers in place.  Any other
 * b1 x b2 shape is expanded to CSR once (jlust_hip_bsr_expand_csr_i32's
 * layout; the plan owns it) and runs through a CSR SpMM plan over it for k
 * columns.  create synchronises `stream` (browptr's ends are read back and
 * the CSR plan analyses its rows); update_values re-expands only the values,
 * stream-ordered, on the expansion path, and is a pointer swap on the MFMA
 * path.  execute: B (nb*b2) x k (ldb), C (mb*b1) x k (ldc), column-major;
 * C = alpha*A*B + beta*C (beta == 0: C write-only).  info: path 0 = MFMA,
 * 1 = CSR expansion.  The plan keeps browptr, bcolind (and, on the MFMA path,
 * the values) by pointer: the caller keeps them alive.
 */
int jlust_hip_bsr_spmm_plan_create(int64_t mb, int64_t nb, int64_t b1,
                                   int64_t b2, int64_t nnzb, int32_t origin,
                                   int value_type, int row_major_blocks,
                                   const int32_t *browptr,
                                   const int32_t *bcolind, const void *val,
                                   int64_t k, jlust_stream_t stream,
                                   jlust_bsr_plan_t *plan_out);
int jlust_hip_bsr_spmm_plan_update_values(jlust_bsr_plan_t plan,
                                          const void *val,
                                          jlust_stream_t stream);
int jlust_hip_bsr_spmm_plan_execute_f32(jlust_bsr_plan_t plan, float alpha,
                                        const float *B, int64_t ldb,
                                        float beta, float *C, int64_t ldc,
                                        jlust_stream_t stream);
int jlust_hip_bsr_spmm_plan_execute_f64(jlust_bsr_plan_t plan, double alpha,
                                        const double *B, int64_t ldb,
                                        double beta, double *C, int64_t ldc,
                                        jlust_stream_t stream);
int jlust_hip_bsr_spmm_plan_info(jlust_bsr_plan_t plan, int32_t *path);
/* Drains the device, then frees the plan's expansion and CSR plan. */
int jlust_hip_bsr_spmm_plan_destroy(jlust_bsr_plan_t plan);

/*
 * Prepared BSR SpMV: prepare(EmitterBackend, SpMVOp, u_A) on a BSR matrix
 * (ext/KernelAbstractionsExt/ops/spmv.jl:518-544, the handle execute(h, x, y)
 * and update_values! run on; the reference analyses nothing for it).  Any
 * block shape, either block order, Float64 or Float32 (value_type 0 / 1).
 * create builds the segment table of jlust_hip_bsr_spmv_*_i32 once (block-
 * rows cut into segments of at most 32 blocks; the plan owns it and the
 * per-segment sums) and synchronises `stream`; it reads browptr's ends back
 * and returns JLUST_STATUS_NONCANONICAL_STORAGE unless they are origin and
 * nnzb + origin.  execute: y = alpha*A*x + beta*y (beta == 0: y write-only),
 * stream-ordered; one plan must not run on two streams at once (the partial
 * sums are the plan's).  update_values: new values of the same pattern, a
 * pointer swap.  The plan keeps browptr, bcolind and the values by pointer:
 * the caller keeps them alive.
 */
int jlust_hip_bsr_spmv_plan_create(int64_t mb, int64_t nb, int64_t b1,
                                   int64_t b2, int64_t nnzb, int32_t origin,
                                   int value_type, int row_major_blocks,
                                   const int32_t *browptr,
                                   const int32_t *bcolind, const void *val,
                                   jlust_stream_t stream,
                                   jlust_bsr_spmv_plan_t *plan_out);
int jlust_hip_bsr_spmv_plan_update_values(jlust_bsr_spmv_plan_t plan,
                                          const void *val,
                                          jlust_stream_t stream);
int jlust_hip_bsr_spmv_plan_execute_f64(jlust_bsr_spmv_plan_t plan,
                                        double alpha, const double *x,
                                        double beta, double *y,
                                        jlust_stream_t stream);
int jlust_hip_bsr_spmv_plan_execute_f32(jlust_bsr_spmv_plan_t plan,
                                        float alpha, const float *x,
                                        float beta, float *y,
                                        jlust_stream_t stream);
/* Drains the device, then frees the plan's segment table. */
int jlust_hip_bsr_spmv_plan_destroy(jlust_bsr_spmv_plan_t plan);

/* ----------------------------------------------------------- conversions */

/* Sparse matrix formats of the conversion entry points
 * (src/named_formats.jl:24-27,106-128). */
enum jlust_format {
    JLUST_FORMAT_CSR = 0,   /* (i : dense, j : compressed)                        */
    JLUST_FORMAT_CSC = 1,   /* (j : dense, i : compressed)                        */
    JLUST_FORMAT_COO = 2,   /* (i : compressed(nonunique), j : singleton)         */
    JLUST_FORMAT_DCSR = 3,  /* (i : compressed, j : compressed)                   */
    JLUST_FORMAT_BSR = 4    /* BSRRight/BSRLeft((b1, b2)): (i/b1 : dense, j/b2 :
                               compressed, then the in-block levels)            */
};

/*
 * A 2-D sparse matrix: the level buffers of a USTensor (src/tensor.jl:33-44)
 * as device pointers.  Index values are origin-based Int32 (origin 0 or 1).
 *   CSR : pos2 = rowptr[m+1], crd2 = colind[nnz]
 *   CSC : pos2 = colptr[n+1], crd2 = rowind[nnz]
 *   COO : pos1 = {origin, nnz+origin} (may be NULL on input), crd1 = rows, crd2 = cols
 *   DCSR: pos1 = {origin, nouter+origin}, crd1 = stored rows[nouter],
 *         pos2 = row segments[nouter+1], crd2 = cols[nnz]
 *   BSR : pos2 = browptr[m/b1+1], crd2 = bcolind[nouter] (nouter = nnzb),
 *         nnz = nouter*b1*b2 values, block-major, row-major inside a block
 *         when row_major_blocks != 0
 * val holds nnz Float64 or Float32 values (value_type 0 / 1).
 */
typedef struct jlust_sparse {
    int32_t format;
    int32_t origin;
    int64_t m, n;
    int32_t b1, b2, row_major_blocks;
    int64_t nnz;
    int64_t nouter;
    int32_t *pos1, *crd1, *pos2, *crd2;
    void *val;
} jlust_sparse;

/*
 * convert_format(u, fmt) (src/convert.jl:302-388) on the GPU, step 1 of 2:
 * decomposes src, drops explicit zeros, sorts stably by the target's level
 * coordinates (unless the target is the identity ordering and the source is
 * an ordered identity format, convert.jl:331-349) and merges adjacent equal
 * coordinates on unique levels keeping the first value (convert.jl:232-250).
 * Reports the target's sizes: *dst_nnz values and *dst_nouter (DCSR stored
 * rows, BSR blocks; 0 otherwise).  Synchronises `stream`.  The handle owns
 * the analysed entries (its analysis workspace, about 32 bytes of device
 * memory per stored source value) until jlust_hip_convert_destroy; src must
 * stay valid until jlust_hip_convert_fill.  dst_b1/dst_b2/dst_row_major_blocks describe
 * a BSR target.  Returns NONCANONICAL_STORAGE where the reference asserts
 * (a CSR target built from rows in decreasing order).
 */
int jlust_hip_convert_analyze(const jlust_sparse *src, int32_t dst_format,
                              int32_t dst_b1, int32_t dst_b2,
                              int32_t dst_row_major_blocks, int value_type,
                              jlust_stream_t stream, jlust_convert_t *out,
                              int64_t *dst_nnz, int64_t *dst_nouter);

/* Step 2: writes the target's buffers (caller-allocated with the sizes from
 * analyze; origin, extents and format equal to the source's and the analysed
 * target), stream-ordered. */
int jlust_hip_convert_fill(jlust_convert_t h, const jlust_sparse *dst,
                           jlust_stream_t stream);

/* Frees the handle's device memory (after the fills that use it). */
int jlust_hip_convert_destroy(jlust_convert_t h);

/*
 * sparse_to_dense (ext/KernelAbstractionsExt/ops/conversion.jl:47-65): the
 * m x n column-major `dense` (leading dimension ld) is zero-filled and every
 * stored entry written at its (row, col).  Synchronises `stream`.
 */
int jlust_hip_sparse_to_dense(const jlust_sparse *src, int value_type,
                              void *dense, int64_t ld, jlust_stream_t stream);

/* dst[i] = src[i] + delta (dst == src allowed): the index shift of
 * materialize's origin change (ext/CUDAExt/CUDAExt.jl:199-220). */
int jlust_hip_shift_index(int32_t *dst, const int32_t *src, int64_t len,
                          int32_t delta, jlust_stream_t stream);

/* ------------------------------------------------------- block assembly */

/*
 * One block of an assembled matrix: a CSR or DCSR matrix (`block`), or, when
 * block == NULL, a shifted scaled identity of extents diag_m x diag_n whose
 * row r holds diag_val at column r + diag_shift where that column exists
 * (Formats.ShiftedDiag, src/named_formats.jl:53-61), placed with its (0, 0)
 * at (row_off, col_off) of the result (0-based).  When slots != NULL it
 * receives, for each stored value k of a CSR/DCSR block, the position of
 * that value in the assembled colind/val.
 */
typedef struct jlust_placement {
    const jlust_sparse *block;
    int64_t row_off, col_off;
    int64_t diag_m, diag_n, diag_shift;
    double diag_val;
    int32_t *slots;
} jlust_placement;

/*
 * The m x n CSR (origin 0) of a block aggregate: row R holds, for each
 * placement covering R in the given order, that block row's stored entries
 * in storage order (explicit zeros included) with columns shifted by
 * col_off.  rowptr[m+1], colind[nnz], val[nnz] are caller-allocated; nnz
 * must equal the placements' stored values.  Synchronises `stream`.  Invalid
 * block storage returns NONCANONICAL_STORAGE.  Replaces the host assembly
 * of _compile_bsm (ext/CUDAExt/ops/block_mul.jl:128-224) and _compile_bbm
 * (:453-556).
 */
int jlust_hip_csr_assemble(int64_t m, int64_t n, int32_t nplacements,
                           const jlust_placement *placements, int value_type,
                           int32_t *rowptr, int32_t *colind, void *val,
                           int64_t nnz, jlust_stream_t stream);

/*
 * y = alpha*M*x + beta*y for a T-period block-banded matrix M of bandwidth 1
 * whose diagonal block D (n_diag_rows x n_cols) is shared by every period and
 * whose coupling pair (neg, pos) (n_off_rows x n_cols each) is shared by
 * every transition, without the T-fold matrix: the reference's periodic view
 * and fused kernel (ext/CUDAExt/ops/block_mul.jl:584-676,
 * ext/KernelAbstractionsExt/ops/block_periodic.jl:108-236).  Rows of period
 * t: D's rows against x[t*n_cols ...], then (t < T-1) the coupling rows,
 * neg's against x[t*n_cols ...] plus pos's against x[(t+1)*n_cols ...]
 * (block_banded.jl:5-14); M is (T*n_diag_rows + (T-1)*n_off_rows) x
 * T*n_cols.  Each block is a placement's CSR block (any origin) or its
 * shifted diagonal (block == NULL; diag_m x diag_n, entries
 * (i, i + diag_shift) = diag_val); row_off, col_off and slots are ignored.
 * Other block formats return UNSUPPORTED_FORMAT.  neg and pos are read only
 * when T > 1 and n_off_rows > 0.  Rows must fit in 32 bits.
 */
int jlust_hip_bbm_periodic_spmv_f64(int64_t T, int64_t n_diag_rows,
                                    int64_t n_off_rows, int64_t n_cols,
                                    const jlust_placement *diag,
                                    const jlust_placement *neg,
                                    const jlust_placement *pos, double alpha,
                                    const double *x, double beta, double *y,
                                    jlust_stream_t stream);
int jlust_hip_bbm_periodic_spmv_f32(int64_t T, int64_t n_diag_rows,
                                    int64_t n_off_rows, int64_t n_cols,
                                    const jlust_placement *diag,
                                    const jlust_placement *neg,
                                    const jlust_placement *pos, float alpha,
                                    const float *x, float beta, float *y,
                                    jlust_stream_t stream);

/*
 * dst[slots[k]] = src[k] for k < len (slots outside [0, dst_len) are
 * skipped): new values of one block into an assembled matrix, the compiled
 * view update of update_block_values! (ext/CUDAExt/ops/block_mul.jl:310-336).
 */
int jlust_hip_scatter_values(void *dst, int64_t dst_len, const int32_t *slots,
                             const void *src, int64_t len, int value_type,
                             jlust_stream_t stream);

/*
 * y = alpha*A*x + beta*y for the m x n shifted scaled identity A: row r holds
 * val at column r + shift where that column exists, and nothing else
 * (Formats.ShiftedDiag, src/named_formats.jl:53-61, whose level yields
 * (r + shift, val) per row, src/backends.jl:223-227).  beta == 0 writes y
 * without reading it.
 */
int jlust_hip_shifted_diag_spmv_f64(int64_t m, int64_t n, int64_t shift,
                                    double val, double alpha, const double *x,
                                    double beta, double *y,
                                    jlust_stream_t stream);
int jlust_hip_shifted_diag_spmv_f32(int64_t m, int64_t n, int64_t shift,
                                    float val, float alpha, const float *x,
                                    float beta, float *y,
                                    jlust_stream_t stream);

/*
 * C = alpha*A*B + beta*C for the same shifted scaled identity A (m x n), B
 * n x k (ldb), C m x k (ldc), column-major: the SpMM the reference's
 * EmitterBackend takes for every non-dense A (ext/KernelAbstractionsExt/
 * KernelAbstractionsExt.jl:35-37), with the nzval-less level's (r + shift,
 * val) per row (src/backends.jl:223-227).  Rows whose column r + shift does
 * not exist get alpha*0 + beta*C.  beta == 0 writes C without reading it.
 */
int jlust_hip_shifted_diag_spmm_f64(int64_t m, int64_t n, int64_t k,
                                    int64_t shift, double val, double alpha,
                                    const double *B, int64_t ldb, double beta,
                                    double *C, int64_t ldc,
                                    jlust_stream_t stream);
int jlust_hip_shifted_diag_spmm_f32(int64_t m, int64_t n, int64_t k,
                                    int64_t shift, float val, float alpha,
                                    const float *B, int64_t ldb, float beta,
                                    float *C, int64_t ldc,
                                    jlust_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* JLUST_HIP_H */
