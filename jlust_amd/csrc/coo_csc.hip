// coo_csc.hip -- SpMM with COO or CSC operands, SDDMM with CSC masks, and the
// index passes behind them: checks of position and coordinate arrays, the
// expansion of a position array into one coordinate per entry, the row order
// of COO/CSC entries and permuted value gathers.
//
// The reference's EmitterBackend takes SpMM for every non-dense A and SDDMM
// for every non-dense C (ext/KernelAbstractionsExt/KernelAbstractionsExt.jl:
// 35-37, ops/sddmm.jl:12-14).  For a COO A it pre-scales C by beta (zero fill
// when beta == 0) and adds alpha*val*B[col, :] into C[row, :] with atomics,
// one thread per stored entry (ColFirst, ops/spmm.jl:331-335, 412-416); a CSC
// A runs the same adds in the walker's scatter direction (columns outer).
// Atomics into a column-major C cost one cache line per column per entry, so
// here the entries are put in row order first -- a stable sort of (row,
// position) when COO rows are not already non-decreasing, and always for CSC,
// whose column per entry is expanded from colptr -- and the CSR SpMM kernels
// run on that order.  Every entry is added once and rows without entries are
// scaled by beta, so C = alpha*A*B + beta*C as in the reference, with each
// output summed in one fixed order (deterministic) instead of the atomics'
// arrival order.
//
// SDDMM writes one output per stored entry, so a mask's format decides only
// how an entry's (i, j) is found: a CSC mask expands colptr into one column
// per entry and runs the COO-mask kernel on (rowind, column), in storage
// order.  (DCSR masks run the CSR kernel over the stored rows with a row map,
// in sddmm.hip.)
#include <algorithm>

#include "common.hpp"

namespace jlust {
namespace {

constexpr int XB = 256;

unsigned xgrid(int64_t n) { return (unsigned)((n + XB - 1) / XB); }

size_t a256(size_t v) { return (v + 255) / 256 * 256; }

struct DevMem {
    void *p = nullptr;
    ~DevMem() { if (p) (void)hipFree(p); }
};

// Flag bits: 1 pos[0] != origin; 2 pos[nouter] - origin != nnz; 4 pos decreases.
__global__ void pos_check_kernel(int64_t nouter, int64_t nnz, int32_t origin, const int32_t *__restrict__ pos,
                                 int32_t *__restrict__ flag)
{
    const int64_t i = (int64_t)blockIdx.x * XB + threadIdx.x;
    if (i > nouter) return;
    const int64_t v = (int64_t)pos[i] - origin;
    int32_t f = 0;
    if (i == 0 && v != 0) f |= 1;
    if (i == nouter && v != nnz) f |= 2;
    if (i < nouter && (int64_t)pos[i + 1] - origin < v) f |= 4;
    if (f) atomicOr(flag, f);
}

// Flag bits: 8 a coordinate outside [origin, extent + origin); 16 not
// strictly increasing (checked only when `strict`).
__global__ void crd_check_kernel(int64_t len, int64_t extent, int32_t origin, int strict,
                                 const int32_t *__restrict__ crd, int32_t *__restrict__ flag)
{
    const int64_t i = (int64_t)blockIdx.x * XB + threadIdx.x;
    if (i >= len) return;
    const int64_t v = (int64_t)crd[i] - origin;
    int32_t f = 0;
    if (v < 0 || v >= extent) f |= 8;
    if (strict && i > 0 && crd[i] <= crd[i - 1]) f |= 16;
    if (f) atomicOr(flag, f);
}

// dst[i] = src[i] narrowed to Int32; a value outside Int32's range sets flag
// bit 32 (and leaves 0).
__global__ void narrow_index_kernel(int64_t n, const int64_t *__restrict__ src, int32_t *__restrict__ dst,
                                    int32_t *__restrict__ flag)
{
    const int64_t i = (int64_t)blockIdx.x * XB + threadIdx.x;
    if (i >= n) return;
    const int64_t v = src[i];
    const bool ok = v >= INT32_MIN && v <= INT32_MAX;
    dst[i] = ok ? (int32_t)v : 0;
    if (!ok) atomicOr(flag, 32);
}

// crd_out[p] = outer ? outer[s] : s + origin, for the segment s holding entry
// p: the last s < nouter with pos[s] - origin <= p (pos checked canonical, so
// empty segments before it are skipped).
__global__ void expand_pos_kernel(int64_t nouter, int64_t nnz, int32_t origin, const int32_t *__restrict__ pos,
                                  const int32_t *__restrict__ outer, int32_t *__restrict__ crd_out)
{
    const int64_t p = (int64_t)blockIdx.x * XB + threadIdx.x;
    if (p >= nnz) return;
    int64_t lo = 0, hi = nouter - 1;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if ((int64_t)pos[mid] - origin <= p) lo = mid;
        else hi = mid - 1;
    }
    crd_out[p] = outer ? outer[lo] : (int32_t)(lo + origin);
}

__global__ void iota_kernel(int64_t n, int32_t *__restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * XB + threadIdx.x;
    if (i < n) out[i] = (int32_t)i;
}

template <typename T>
__global__ void perm_gather_kernel(int64_t n, const int32_t *__restrict__ perm, const T *__restrict__ src,
                                   T *__restrict__ dst)
{
    const int64_t i = (int64_t)blockIdx.x * XB + threadIdx.x;
    if (i < n) dst[i] = src[perm[i]];
}

// Runs the check kernels queued by `enqueue` against one flag word of the
// stream's scratch buffer and reads the flag back (synchronises s).
template <typename F>
int run_checks(hipStream_t s, int32_t *flags_out, F &&enqueue)
{
    void *w = nullptr;
    if (int st = scratch((jlust_stream_t)s, 256, &w)) return st;
    int32_t *flag = (int32_t *)w;
    JLUST_HIP_TRY(hipMemsetAsync(flag, 0, sizeof(int32_t), s));
    if (int st = enqueue(flag)) return st;
    int32_t h = 0;
    JLUST_HIP_TRY(hipMemcpyAsync(&h, flag, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    JLUST_HIP_TRY(hipStreamSynchronize(s));
    *flags_out = h;
    return JLUST_STATUS_SUCCESS;
}

int pos_status(const char *who, int32_t f)
{
    if (f & 1) return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "%s: the position array does not start at the origin", who);
    if (f & 2) return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "%s: the position array does not end at nnz + origin", who);
    if (f & 4) return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "%s: the position array decreases", who);
    if (f & 8) return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "%s: a coordinate is out of range", who);
    if (f & 16) return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "%s: coordinates are not strictly increasing", who);
    return JLUST_STATUS_SUCCESS;
}

int enqueue_pos_check(int64_t nouter, int64_t nnz, int32_t origin, const int32_t *pos, int32_t *flag, hipStream_t s)
{
    hipLaunchKernelGGL(pos_check_kernel, dim3(xgrid(nouter + 1)), dim3(XB), 0, s, nouter, nnz, origin, pos, flag);
    return check_launch("pos_check_kernel");
}

}  // namespace

int check_pos(const char *who, int64_t nouter, int64_t nnz, int32_t origin, const int32_t *pos, hipStream_t s)
{
    int32_t f = 0;
    if (int st = run_checks(s, &f, [&](int32_t *flag) { return enqueue_pos_check(nouter, nnz, origin, pos, flag, s); }))
        return st;
    return pos_status(who, f);
}

int expand_pos(int64_t nouter, int64_t nnz, int32_t origin, const int32_t *pos, const int32_t *outer,
               int32_t *crd_out, hipStream_t s)
{
    if (int st = check_pos("expand_pos", nouter, nnz, origin, pos, s)) return st;
    if (nnz == 0) return JLUST_STATUS_SUCCESS;
    hipLaunchKernelGGL(expand_pos_kernel, dim3(xgrid(nnz)), dim3(XB), 0, s, nouter, nnz, origin, pos, outer,
                       crd_out);
    return check_launch("expand_pos_kernel");
}

// Row order of COO (idx1 = rows, idx2 = cols) or CSC (idx1 = colptr[n+1],
// idx2 = rowind) entries: rowptr[m+1] always; for CSC, and for COO rows that
// are not non-decreasing, perm[q] (source position of row-ordered entry q)
// and cols[q] (its column) with *reordered = 1; otherwise *reordered = 0 and
// perm/cols are untouched (the source order is the row order).  Synchronises s.
int row_order(int32_t format, int64_t m, int64_t n, int64_t nnz, int32_t origin, const int32_t *idx1,
              const int32_t *idx2, int32_t *rowptr, int32_t *perm, int32_t *cols, int32_t *reordered, hipStream_t s)
{
    *reordered = 0;
    if (format == JLUST_FORMAT_COO) {
        bool sorted = true;
        if (int st = coo_row_order(m, nnz, origin, idx1, idx2, rowptr, perm, cols, &sorted, s)) return st;
        *reordered = !sorted;
        return JLUST_STATUS_SUCCESS;
    }
    // CSC: the column of every entry, then the COO row order of (rowind, column).
    DevMem colexp;
    JLUST_HIP_TRY(hipMalloc(&colexp.p, a256(4 * (size_t)(nnz > 0 ? nnz : 1))));
    int32_t *ce = (int32_t *)colexp.p;
    if (int st = expand_pos(n, nnz, origin, idx1, nullptr, ce, s)) return st;
    bool sorted = true;
    if (int st = coo_row_order(m, nnz, origin, idx2, ce, rowptr, perm, cols, &sorted, s)) return st;
    if (sorted && nnz > 0) {
        // Rows already non-decreasing in storage order: the identity order.
        hipLaunchKernelGGL(iota_kernel, dim3(xgrid(nnz)), dim3(XB), 0, s, nnz, perm);
        if (int st = check_launch("iota_kernel")) return st;
        JLUST_HIP_TRY(hipMemcpyAsync(cols, ce, 4 * (size_t)nnz, hipMemcpyDeviceToDevice, s));
    }
    JLUST_HIP_TRY(hipStreamSynchronize(s));      // colexp is freed on return
    *reordered = 1;
    return JLUST_STATUS_SUCCESS;
}

int perm_gather(int value_type, int64_t nnz, const int32_t *perm, const void *src, void *dst, hipStream_t s)
{
    if (nnz == 0) return JLUST_STATUS_SUCCESS;
    if (value_type == 0)
        hipLaunchKernelGGL((perm_gather_kernel<double>), dim3(xgrid(nnz)), dim3(XB), 0, s, nnz, perm,
                           (const double *)src, (double *)dst);
    else
        hipLaunchKernelGGL((perm_gather_kernel<float>), dim3(xgrid(nnz)), dim3(XB), 0, s, nnz, perm,
                           (const float *)src, (float *)dst);
    return check_launch("perm_gather_kernel");
}

namespace {

int check_reorder_args(const char *who, int32_t format, int64_t m, int64_t n, int64_t nnz, int32_t origin,
                       const int32_t *idx1, const int32_t *idx2)
{
    if (format != JLUST_FORMAT_COO && format != JLUST_FORMAT_CSC)
        return fail(JLUST_STATUS_UNSUPPORTED_FORMAT, "%s: format %d (COO = %d, CSC = %d)", who, format,
                    JLUST_FORMAT_COO, JLUST_FORMAT_CSC);
    if (m < 0 || n < 0 || nnz < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: negative extent", who);
    if (m > INT32_MAX - 1 || n > INT32_MAX - 1 || nnz > INT32_MAX - 1)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: extents exceed the Int32 index range", who);
    if (int st = check_origin(origin)) return st;
    const bool csc = format == JLUST_FORMAT_CSC;
    if ((csc ? !idx1 : bad_ptr(idx1, nnz)) || bad_ptr(idx2, nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: null device pointer", who);
    if (nnz > 0 && (m == 0 || n == 0))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: entries in an empty matrix", who);
    return JLUST_STATUS_SUCCESS;
}

// The plain COO/CSC SpMM: row order and values into temporaries, then the
// CSR SpMM call on them; the temporaries are freed after the stream drains.
template <typename T>
int reordered_spmm(const char *who, int32_t format, int64_t m, int64_t n, int64_t k, int64_t nnz, int32_t origin,
                   const int32_t *idx1, const int32_t *idx2, const T *val, T alpha, const T *B, int64_t ldb, T beta,
                   T *C, int64_t ldc, jlust_stream_t stream)
{
    clear_error();
    if (int st = check_reorder_args(who, format, m, n, nnz, origin, idx1, idx2)) return st;
    if (k < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: negative column count", who);
    if (bad_ptr(val, nnz) || bad_ptr(B, (nnz > 0 && k > 0) ? n : 0) || bad_ptr(C, m * k))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: null device pointer", who);
    if (k > 1 && (ldb < std::max<int64_t>(n, 1) || ldc < std::max<int64_t>(m, 1)))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: leading dimensions too small (ldb=%lld, ldc=%lld)", who,
                    (long long)ldb, (long long)ldc);
    if (int st = require_device(nullptr)) return st;
    if (m == 0 || k == 0) return JLUST_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;
    const size_t nz = (size_t)(nnz > 0 ? nnz : 1);
    const size_t sz_rp = a256(4 * (size_t)(m + 1)), sz_i = a256(4 * nz), sz_v = a256(sizeof(T) * nz);
    DevMem mem;
    JLUST_HIP_TRY(hipMalloc(&mem.p, sz_rp + 2 * sz_i + sz_v));
    char *b = (char *)mem.p;
    int32_t *rowptr = (int32_t *)b;
    int32_t *perm = (int32_t *)(b + sz_rp);
    int32_t *cols = (int32_t *)(b + sz_rp + sz_i);
    T *vals = (T *)(b + sz_rp + 2 * sz_i);
    int32_t reordered = 0;
    if (int st = row_order(format, m, n, nnz, origin, idx1, idx2, rowptr, perm, cols, &reordered, s)) return st;
    const int32_t *csr_cols = idx2;
    const T *csr_val = val;
    if (reordered) {
        if (int st = perm_gather(sizeof(T) == 8 ? 0 : 1, nnz, perm, val, vals, s)) return st;
        csr_cols = cols;
        csr_val = vals;
    }
    int st;
    if constexpr (sizeof(T) == 8)
        st = jlust_hip_csr_spmm_f64_i32(m, n, k, nnz, origin, rowptr, csr_cols, csr_val, alpha, B, ldb, beta, C,
                                        ldc, 0, stream);
    else
        st = jlust_hip_csr_spmm_f32_i32(m, n, k, nnz, origin, rowptr, csr_cols, csr_val, alpha, B, ldb, beta, C,
                                        ldc, 0, stream);
    const hipError_t e = hipStreamSynchronize(s);     // the temporaries are freed on return
    if (st) return st;
    if (e != hipSuccess) return hip_fail(e, who);
    return JLUST_STATUS_SUCCESS;
}

// The plain CSC-mask SDDMM: the column of every entry, then the COO-mask call.
template <typename T>
int csc_sddmm(int64_t m, int64_t n, int64_t K, int64_t nnz, int32_t origin, const int32_t *colptr,
              const int32_t *rowind, T alpha, const T *A, int64_t lda, const T *B, int64_t ldb, T beta, T *Cval,
              const T *mask, jlust_stream_t stream)
{
    clear_error();
    if (int st = check_reorder_args("csc_sddmm", JLUST_FORMAT_CSC, m, n, nnz, origin, colptr, rowind)) return st;
    if (int st = require_device(nullptr)) return st;
    if (nnz == 0) return JLUST_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;
    DevMem colexp;
    JLUST_HIP_TRY(hipMalloc(&colexp.p, a256(4 * (size_t)nnz)));
    int32_t *ce = (int32_t *)colexp.p;
    if (int st = expand_pos(n, nnz, origin, colptr, nullptr, ce, s)) return st;
    int st;
    if constexpr (sizeof(T) == 8)
        st = jlust_hip_coo_sddmm_f64_i32(m, n, K, nnz, origin, rowind, ce, alpha, A, lda, B, ldb, beta, Cval, mask,
                                         stream);
    else
        st = jlust_hip_coo_sddmm_f32_i32(m, n, K, nnz, origin, rowind, ce, alpha, A, lda, B, ldb, beta, Cval, mask,
                                         stream);
    const hipError_t e = hipStreamSynchronize(s);     // colexp is freed on return
    if (st) return st;
    if (e != hipSuccess) return hip_fail(e, "csc_sddmm");
    return JLUST_STATUS_SUCCESS;
}

}  // namespace
}  // namespace jlust

using namespace jlust;

extern "C" int jlust_hip_check_pos_i32(int64_t nouter, int64_t nnz, int32_t origin, const int32_t *pos,
                                       jlust_stream_t stream)
{
    clear_error();
    if (nouter < 0 || nnz < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "check_pos: negative extent");
    if (int st = check_origin(origin)) return st;
    if (!pos) return fail(JLUST_STATUS_INVALID_ARGUMENT, "check_pos: null device pointer");
    if (int st = require_device(nullptr)) return st;
    return check_pos("check_pos", nouter, nnz, origin, pos, (hipStream_t)stream);
}

extern "C" int jlust_hip_check_crd_i32(int64_t len, int64_t extent, int32_t origin, int strictly_increasing,
                                       const int32_t *crd, jlust_stream_t stream)
{
    clear_error();
    if (len < 0 || extent < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "check_crd: negative extent");
    if (int st = check_origin(origin)) return st;
    if (bad_ptr(crd, len)) return fail(JLUST_STATUS_INVALID_ARGUMENT, "check_crd: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (len == 0) return JLUST_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;
    int32_t f = 0;
    if (int st = run_checks(s, &f, [&](int32_t *flag) {
            hipLaunchKernelGGL(crd_check_kernel, dim3(xgrid(len)), dim3(XB), 0, s, len, extent, origin,
                               strictly_increasing, crd, flag);
            return check_launch("crd_check_kernel");
        }))
        return st;
    return pos_status("check_crd", f);
}

extern "C" int jlust_hip_narrow_index_i64(int64_t n, const int64_t *src, int32_t *dst, jlust_stream_t stream)
{
    clear_error();
    if (n < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "narrow_index: negative length");
    if (n >= (int64_t)1 << 31)
        return fail(JLUST_STATUS_UNSUPPORTED_INDEX_TYPE, "narrow_index: %lld entries exceed the Int32 index range",
                    (long long)n);
    if (bad_ptr(src, n) || bad_ptr(dst, n)) return fail(JLUST_STATUS_INVALID_ARGUMENT, "narrow_index: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (n == 0) return JLUST_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;
    int32_t f = 0;
    if (int st = run_checks(s, &f, [&](int32_t *flag) {
            hipLaunchKernelGGL(narrow_index_kernel, dim3(xgrid(n)), dim3(XB), 0, s, n, src, dst, flag);
            return check_launch("narrow_index_kernel");
        }))
        return st;
    if (f & 32)
        return fail(JLUST_STATUS_UNSUPPORTED_INDEX_TYPE, "narrow_index: an index is outside the Int32 range");
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_expand_pos_i32(int64_t nouter, int64_t nnz, int32_t origin, const int32_t *pos,
                                        const int32_t *outer_crd, int32_t *crd_out, jlust_stream_t stream)
{
    clear_error();
    if (nouter < 0 || nnz < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "expand_pos: negative extent");
    if (int st = check_origin(origin)) return st;
    if (!pos || bad_ptr(crd_out, nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "expand_pos: null device pointer");
    if (int st = require_device(nullptr)) return st;
    return expand_pos(nouter, nnz, origin, pos, outer_crd, crd_out, (hipStream_t)stream);
}

extern "C" int jlust_hip_row_order_i32(int32_t format, int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                       const int32_t *idx1, const int32_t *idx2, int32_t *rowptr, int32_t *perm,
                                       int32_t *cols, int32_t *reordered, jlust_stream_t stream)
{
    clear_error();
    if (int st = check_reorder_args("row_order", format, m, n, nnz, origin, idx1, idx2)) return st;
    if (!rowptr || bad_ptr(perm, nnz) || bad_ptr(cols, nnz) || !reordered)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "row_order: null output pointer");
    if (int st = require_device(nullptr)) return st;
    return host_guard("row_order", [&] {
        return row_order(format, m, n, nnz, origin, idx1, idx2, rowptr, perm, cols, reordered,
                         (hipStream_t)stream);
    });
}

extern "C" int jlust_hip_gather_f64(int64_t n, const int32_t *perm, const double *src, double *dst,
                                    jlust_stream_t stream)
{
    clear_error();
    if (n < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "gather: negative length");
    if (bad_ptr(perm, n) || bad_ptr(src, n) || bad_ptr(dst, n))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "gather: null device pointer");
    if (int st = require_device(nullptr)) return st;
    return perm_gather(0, n, perm, src, dst, (hipStream_t)stream);
}

extern "C" int jlust_hip_gather_f32(int64_t n, const int32_t *perm, const float *src, float *dst,
                                    jlust_stream_t stream)
{
    clear_error();
    if (n < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "gather: negative length");
    if (bad_ptr(perm, n) || bad_ptr(src, n) || bad_ptr(dst, n))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "gather: null device pointer");
    if (int st = require_device(nullptr)) return st;
    return perm_gather(1, n, perm, src, dst, (hipStream_t)stream);
}

#define JLUST_REORDERED_SPMM(NAME, FMT, T)                                                                     \
    extern "C" int NAME(int64_t m, int64_t n, int64_t k, int64_t nnz, int32_t origin, const int32_t *idx1,    \
                        const int32_t *idx2, const T *val, T alpha, const T *B, int64_t ldb, T beta, T *C,     \
                        int64_t ldc, jlust_stream_t stream)                                                    \
    {                                                                                                          \
        return host_guard(#NAME, [&] {                                                                         \
            return reordered_spmm<T>(#NAME, FMT, m, n, k, nnz, origin, idx1, idx2, val, alpha, B, ldb, beta, C, \
                                     ldc, stream);                                                             \
        });                                                                                                    \
    }
JLUST_REORDERED_SPMM(jlust_hip_coo_spmm_f64_i32, JLUST_FORMAT_COO, double)
JLUST_REORDERED_SPMM(jlust_hip_coo_spmm_f32_i32, JLUST_FORMAT_COO, float)
JLUST_REORDERED_SPMM(jlust_hip_csc_spmm_f64_i32, JLUST_FORMAT_CSC, double)
JLUST_REORDERED_SPMM(jlust_hip_csc_spmm_f32_i32, JLUST_FORMAT_CSC, float)
#undef JLUST_REORDERED_SPMM

extern "C" int jlust_hip_csc_sddmm_f64_i32(int64_t m, int64_t n, int64_t K, int64_t nnz, int32_t origin,
                                           const int32_t *colptr, const int32_t *rowind, double alpha,
                                           const double *A, int64_t lda, const double *B, int64_t ldb,
                                           double beta, double *Cval, const double *mask, jlust_stream_t stream)
{
    return csc_sddmm<double>(m, n, K, nnz, origin, colptr, rowind, alpha, A, lda, B, ldb, beta, Cval, mask,
                             stream);
}

extern "C" int jlust_hip_csc_sddmm_f32_i32(int64_t m, int64_t n, int64_t K, int64_t nnz, int32_t origin,
                                           const int32_t *colptr, const int32_t *rowind, float alpha,
                                           const float *A, int64_t lda, const float *B, int64_t ldb,
                                           float beta, float *Cval, const float *mask, jlust_stream_t stream)
{
    return csc_sddmm<float>(m, n, K, nnz, origin, colptr, rowind, alpha, A, lda, B, ldb, beta, Cval, mask,
                            stream);
}

// A prepared COO/CSC SpMM: the row order once, into memory the plan owns,
// then a CSR SpMM plan over it (spmm.hip), which keeps the permutation for
// update_values.
static int coo_spmm_plan_create_body(int32_t format, int64_t m, int64_t n, int64_t k, int64_t nnz, int32_t origin,
                                     int value_type, const int32_t *idx1, const int32_t *idx2, const void *val,
                                     jlust_stream_t stream, jlust_spmm_plan_t *plan_out)
{
    clear_error();
    if (!plan_out) return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmm_plan_create: null plan_out");
    *plan_out = nullptr;
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE,
                    "coo_spmm_plan_create: value_type %d (0 = Float64, 1 = Float32)", value_type);
    if (int st = check_reorder_args("coo_spmm_plan_create", format, m, n, nnz, origin, idx1, idx2)) return st;
    if (k < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmm_plan_create: negative column count");
    if (bad_ptr(val, nnz)) return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmm_plan_create: null values");
    if (int st = require_device(nullptr)) return st;
    hipStream_t s = (hipStream_t)stream;
    const size_t tsz = value_type == 0 ? 8 : 4;
    const size_t nz = (size_t)(nnz > 0 ? nnz : 1);
    const size_t sz_rp = a256(4 * (size_t)(m + 1)), sz_i = a256(4 * nz), sz_v = a256(tsz * nz);
    DevMem own;
    JLUST_HIP_TRY(hipMalloc(&own.p, sz_rp + 2 * sz_i + sz_v));
    char *b = (char *)own.p;
    int32_t *rowptr = (int32_t *)b;
    int32_t *perm = (int32_t *)(b + sz_rp);
    int32_t *cols = (int32_t *)(b + sz_rp + sz_i);
    void *vals = b + sz_rp + 2 * sz_i;
    int32_t reordered = 0;
    if (int st = row_order(format, m, n, nnz, origin, idx1, idx2, rowptr, perm, cols, &reordered, s)) return st;
    if (reordered)
        if (int st = perm_gather(value_type, nnz, perm, val, vals, s)) return st;
    jlust_spmm_plan_t plan = nullptr;
    if (int st = jlust_hip_csr_spmm_plan_create(m, n, k, nnz, origin, value_type, rowptr, reordered ? cols : idx2,
                                                reordered ? vals : val, stream, &plan))
        return st;
    spmm_plan_adopt_reorder(plan, own.p, reordered ? perm : nullptr, reordered ? vals : nullptr);
    own.p = nullptr;
    *plan_out = plan;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_coo_spmm_plan_create(int32_t format, int64_t m, int64_t n, int64_t k, int64_t nnz,
                                              int32_t origin, int value_type, const int32_t *idx1,
                                              const int32_t *idx2, const void *val, jlust_stream_t stream,
                                              jlust_spmm_plan_t *plan_out)
{
    return host_guard("coo_spmm_plan_create", [&] {
        return coo_spmm_plan_create_body(format, m, n, k, nnz, origin, value_type, idx1, idx2, val, stream,
                                         plan_out);
    });
}

namespace jlust {
int preload_coo_csc()
{
    JLUST_PRELOAD_KERNEL(pos_check_kernel);
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
