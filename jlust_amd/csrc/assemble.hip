// assemble.hip -- one CSR matrix from placed blocks, on the device.
//
// The block aggregates (BlockSparseMatrix, BlockBandedMatrix) multiply through
// a single CSR built once from their blocks: every block is a CSR or DCSR
// matrix, or a shifted scaled identity, placed at a (row, column) offset.
// Row R of the result holds, for each placement covering R in the order the
// placements are given, that block row's stored entries in storage order with
// their columns shifted.  This is the host assembly of the reference
// (_compile_bsm, ext/CUDAExt/ops/block_mul.jl:128-224; _compile_bbm,
// :453-556) done with three passes over device memory instead of a host copy:
//
//   1. row lengths: per placement, add each block row's length to counts[R]
//      (placements run one after another, so no atomics);
//   2. rowptr = exclusive scan of the counts;
//   3. per placement, every stored entry finds its block row by binary search
//      over the block's row pointer and lands at cursor[R] + (k - pos[r]); the
//      cursors then advance by the row lengths (pass 1 again, onto cursor).
//
// Each stored entry's slot is optionally written back (slots[k]) so that new
// values of one block can be scattered into the assembled values later
// (update_block_values!, block_mul.jl:310-336).
#include "common.hpp"

#include <climits>
#include <vector>

namespace jlust {
namespace {

constexpr int AS_BLOCK = 256;

unsigned as_grid(int64_t n) { return (unsigned)((n + AS_BLOCK - 1) / AS_BLOCK); }

// A placement as the kernels see it (0-based, validated on the host).
struct Piece {
    int kind;                 // 0 CSR, 1 DCSR, 2 shifted diagonal
    int32_t origin;
    int64_t m, n;             // block extents
    int64_t nseg;             // CSR: m; DCSR: stored rows
    int64_t nnz;              // stored values (shifted diagonal: rows with a column in range)
    const int32_t *pos;       // nseg + 1 segment pointers
    const int32_t *outer;     // DCSR stored rows
    const int32_t *crd;       // columns
    const void *val;
    int64_t row_off, col_off;
    int64_t shift;            // shifted diagonal: row r -> column r + shift
    double dval;
    int32_t *slots;
};

enum Bad : int32_t {
    BAD_PTR = 1,       // pos[0] != origin or pos[nseg] - pos[0] != nnz
    BAD_LEN = 2,       // a negative segment length
    BAD_ROW = 4,       // a DCSR stored row outside [0, m) or not increasing
    BAD_COL = 8,       // a column outside [0, n)
};

__device__ __forceinline__ void flag(int32_t *bad, int32_t what) { atomicOr(bad, what); }

// Rows of a shifted diagonal that hold an entry: r in [0, m) with r + shift in [0, n).
__host__ __device__ inline void diag_rows(int64_t m, int64_t n, int64_t shift, int64_t &lo, int64_t &hi)
{
    lo = shift < 0 ? -shift : 0;
    hi = n - shift < m ? n - shift : m;
    if (hi < lo) hi = lo;
}

// acc[row_off + row] += length of each block row (pass 1, and the cursor advance).
__global__ __launch_bounds__(AS_BLOCK) void row_len_kernel(Piece p, int32_t *__restrict__ acc,
                                                           int32_t *__restrict__ bad)
{
    const int64_t s = (int64_t)blockIdx.x * AS_BLOCK + threadIdx.x;
    if (p.kind == 2) {
        int64_t lo, hi;
        diag_rows(p.m, p.n, p.shift, lo, hi);
        if (s >= lo && s < hi) acc[p.row_off + s] += 1;
        return;
    }
    if (s >= p.nseg) return;
    const int32_t a = p.pos[s], b = p.pos[s + 1];
    if (s == 0 && (a != p.origin || (int64_t)p.pos[p.nseg] - a != p.nnz)) flag(bad, BAD_PTR);
    if (b < a) {
        flag(bad, BAD_LEN);
        return;
    }
    int64_t row = s;
    if (p.kind == 1) {
        row = (int64_t)p.outer[s] - p.origin;
        if (row < 0 || row >= p.m || (s > 0 && p.outer[s] <= p.outer[s - 1])) {
            flag(bad, BAD_ROW);
            return;
        }
    }
    acc[p.row_off + row] += b - a;
}

// Pass 3: every stored entry to its slot.
template <typename T>
__global__ __launch_bounds__(AS_BLOCK) void place_kernel(Piece p, const int32_t *__restrict__ cursor,
                                                         int32_t *__restrict__ colind, T *__restrict__ val,
                                                         int64_t nnz_out, int32_t *__restrict__ bad)
{
    const int64_t k = (int64_t)blockIdx.x * AS_BLOCK + threadIdx.x;
    if (p.kind == 2) {
        int64_t lo, hi;
        diag_rows(p.m, p.n, p.shift, lo, hi);
        const int64_t r = lo + k;
        if (r >= hi) return;
        const int64_t slot = cursor[p.row_off + r];
        if (slot < 0 || slot >= nnz_out) {
            flag(bad, BAD_PTR);
            return;
        }
        colind[slot] = (int32_t)(r + p.shift + p.col_off);
        val[slot] = (T)p.dval;
        return;
    }
    if (k >= p.nnz) return;
    // Last segment s with pos[s] - origin <= k (empty segments are skipped
    // because the next non-empty one starts at the same position).
    const int64_t kk = k + p.origin;
    int64_t lo = 0, hi = p.nseg;              // invariant: pos[lo] <= kk < pos[hi]
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (p.pos[mid] <= kk) lo = mid;
        else hi = mid;
    }
    const int64_t row = p.kind == 1 ? (int64_t)p.outer[lo] - p.origin : lo;
    const int64_t slot = (int64_t)cursor[p.row_off + row] + (kk - p.pos[lo]);
    if (slot < 0 || slot >= nnz_out) {
        flag(bad, BAD_PTR);
        return;
    }
    const int64_t c = (int64_t)p.crd[k] - p.origin;
    if (c < 0 || c >= p.n) flag(bad, BAD_COL);
    colind[slot] = (int32_t)(c + p.col_off);
    val[slot] = static_cast<const T *>(p.val)[k];
    if (p.slots) p.slots[k] = (int32_t)slot;
}

template <typename T>
__global__ __launch_bounds__(AS_BLOCK) void scatter_kernel(T *__restrict__ dst, int64_t dst_len,
                                                           const int32_t *__restrict__ slots,
                                                           const T *__restrict__ src, int64_t len)
{
    const int64_t k = (int64_t)blockIdx.x * AS_BLOCK + threadIdx.x;
    if (k >= len) return;
    const int32_t s = slots[k];
    if (s >= 0 && s < dst_len) dst[s] = src[k];
}

// y = alpha*(val*x[r + shift]) + beta*y over the m rows of a shifted scaled
// identity; rows whose column falls outside [0, n) hold no entry.
template <typename T>
__global__ __launch_bounds__(AS_BLOCK) void shifted_diag_spmv_kernel(int64_t m, int64_t n, int64_t shift, T v,
                                                                     T alpha, const T *__restrict__ x, T beta,
                                                                     T *__restrict__ y)
{
    const int64_t r = (int64_t)blockIdx.x * AS_BLOCK + threadIdx.x;
    if (r >= m) return;
    const int64_t c = r + shift;
    const T acc = (c >= 0 && c < n) ? v * x[c] : T(0);
    y[r] = beta == T(0) ? alpha * acc : alpha * acc + beta * y[r];
}

template <typename T>
int shifted_diag_spmv(int64_t m, int64_t n, int64_t shift, T v, T alpha, const T *x, T beta, T *y,
                      jlust_stream_t stream)
{
    clear_error();
    if (m < 0 || n < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "shifted_diag_spmv: negative extents");
    if (bad_ptr(x, n) || bad_ptr(y, m))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "shifted_diag_spmv: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (m == 0) return JLUST_STATUS_SUCCESS;
    hipLaunchKernelGGL((shifted_diag_spmv_kernel<T>), dim3(as_grid(m)), dim3(AS_BLOCK), 0, (hipStream_t)stream,
                       m, n, shift, v, alpha, x, beta, y);
    return check_launch("shifted_diag_spmv_kernel");
}

// C = alpha*A*B + beta*C for the shifted diagonal A (m x n, A[r, r + shift] =
// v where 0 <= r + shift < n), B n x k (ldb), C m x k (ldc): one thread per
// (row, column) of C, rows fastest, so each column is read and written
// contiguously.
template <typename T>
__global__ __launch_bounds__(AS_BLOCK) void shifted_diag_spmm_kernel(int64_t m, int64_t n, int64_t k,
                                                                     int64_t shift, T v, T alpha,
                                                                     const T *__restrict__ B, int64_t ldb, T beta,
                                                                     T *__restrict__ C, int64_t ldc)
{
    const int64_t t = (int64_t)blockIdx.x * AS_BLOCK + threadIdx.x;
    if (t >= m * k) return;
    const int64_t r = t % m, col = t / m;
    const int64_t c = r + shift;
    const T acc = (c >= 0 && c < n) ? v * B[c + col * ldb] : T(0);
    T *out = C + r + col * ldc;
    *out = beta == T(0) ? alpha * acc : alpha * acc + beta * *out;
}

template <typename T>
int shifted_diag_spmm(int64_t m, int64_t n, int64_t k, int64_t shift, T v, T alpha, const T *B, int64_t ldb,
                      T beta, T *C, int64_t ldc, jlust_stream_t stream)
{
    clear_error();
    if (m < 0 || n < 0 || k < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "shifted_diag_spmm: negative extents");
    if (k > 1 && (ldb < (n > 0 ? n : 1) || ldc < (m > 0 ? m : 1)))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "shifted_diag_spmm: leading dimensions too small");
    if (bad_ptr(B, k > 0 ? n : 0) || bad_ptr(C, m * k))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "shifted_diag_spmm: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (m == 0 || k == 0) return JLUST_STATUS_SUCCESS;
    hipLaunchKernelGGL((shifted_diag_spmm_kernel<T>), dim3(as_grid(m * k)), dim3(AS_BLOCK), 0,
                       (hipStream_t)stream, m, n, k, shift, v, alpha, B, ldb, beta, C, ldc);
    return check_launch("shifted_diag_spmm_kernel");
}

struct DevMem {
    void *p = nullptr;
    ~DevMem() { if (p) (void)hipFree(p); }
};

int to_piece(const jlust_placement &pl, int64_t m, int64_t n, int i, Piece &p)
{
    p = Piece{};
    p.row_off = pl.row_off;
    p.col_off = pl.col_off;
    p.slots = pl.slots;
    const jlust_sparse *b = pl.block;
    if (!b) {
        p.kind = 2;
        p.m = pl.diag_m;
        p.n = pl.diag_n;
        p.shift = pl.diag_shift;
        p.dval = pl.diag_val;
        if (p.m < 0 || p.n < 0 || p.shift > INT32_MAX || p.shift < -(int64_t)INT32_MAX)
            return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_assemble: placement %d: bad shifted diagonal", i);
        int64_t lo, hi;
        diag_rows(p.m, p.n, p.shift, lo, hi);
        p.nnz = hi - lo;
    } else {
        if (b->format != JLUST_FORMAT_CSR && b->format != JLUST_FORMAT_DCSR)
            return fail(JLUST_STATUS_UNSUPPORTED_FORMAT,
                        "csr_assemble: placement %d: blocks must be CSR, DCSR or a shifted diagonal (format %d)",
                        i, b->format);
        if (int st = check_origin(b->origin)) return st;
        p.kind = b->format == JLUST_FORMAT_CSR ? 0 : 1;
        p.origin = b->origin;
        p.m = b->m;
        p.n = b->n;
        p.nnz = b->nnz;
        p.nseg = p.kind == 0 ? b->m : b->nouter;
        p.pos = b->pos2;
        p.outer = b->crd1;
        p.crd = b->crd2;
        p.val = b->val;
        if (p.m < 0 || p.n < 0 || p.nnz < 0 || p.nseg < 0 || p.nnz > INT32_MAX ||
            (p.kind == 1 && p.nseg > p.m))
            return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_assemble: placement %d: bad extents", i);
        if ((p.nseg > 0 && !p.pos) || (p.kind == 1 && bad_ptr(p.outer, p.nseg)) || bad_ptr(p.crd, p.nnz) ||
            bad_ptr(p.val, p.nnz) || (p.kind == 0 && !p.pos))
            return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_assemble: placement %d: null device pointer", i);
    }
    if (p.row_off < 0 || p.col_off < 0 || p.row_off + p.m > m || p.col_off + p.n > n)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "csr_assemble: placement %d (%lld x %lld at %lld, %lld) outside the %lld x %lld result", i,
                    (long long)p.m, (long long)p.n, (long long)p.row_off, (long long)p.col_off, (long long)m,
                    (long long)n);
    return JLUST_STATUS_SUCCESS;
}

template <typename T>
int assemble(int64_t m, const std::vector<Piece> &ps, int32_t *rowptr, int32_t *colind, T *val, int64_t nnz,
             hipStream_t st)
{
    DevMem ws;
    JLUST_HIP_TRY(hipMalloc(&ws.p, 4 * (size_t)(m + 1) + 64));
    int32_t *cursor = (int32_t *)ws.p;
    int32_t *bad = cursor + (m + 1);
    JLUST_HIP_TRY(hipMemsetAsync(bad, 0, 4, st));
    JLUST_HIP_TRY(hipMemsetAsync(rowptr, 0, 4 * (size_t)(m + 1), st));
    for (const Piece &p : ps) {
        const int64_t n_threads = p.kind == 2 ? p.m : p.nseg;
        if (n_threads == 0) continue;
        hipLaunchKernelGGL(row_len_kernel, dim3(as_grid(n_threads)), dim3(AS_BLOCK), 0, st, p, rowptr, bad);
        if (int e = check_launch("row_len_kernel")) return e;
    }
    if (int e = exclusive_scan_i32(rowptr, rowptr, m + 1, st)) return e;
    int32_t h[2] = {0, 0};
    JLUST_HIP_TRY(hipMemcpyAsync(&h[0], bad, 4, hipMemcpyDeviceToHost, st));
    JLUST_HIP_TRY(hipMemcpyAsync(&h[1], rowptr + m, 4, hipMemcpyDeviceToHost, st));
    JLUST_HIP_TRY(hipStreamSynchronize(st));
    if (h[0] & BAD_PTR)
        return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                    "csr_assemble: a block's row pointer does not start at its origin or span its values");
    if (h[0] & BAD_LEN)
        return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "csr_assemble: a block's row pointer decreases");
    if (h[0] & BAD_ROW)
        return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                    "csr_assemble: a DCSR block's stored rows are out of range or not increasing");
    if (h[1] != nnz)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_assemble: blocks hold %d entries, nnz says %lld", h[1],
                    (long long)nnz);
    if (m > 0) JLUST_HIP_TRY(hipMemcpyAsync(cursor, rowptr, 4 * (size_t)m, hipMemcpyDeviceToDevice, st));
    for (const Piece &p : ps) {
        if (p.nnz == 0) continue;
        hipLaunchKernelGGL((place_kernel<T>), dim3(as_grid(p.nnz)), dim3(AS_BLOCK), 0, st, p, cursor, colind, val,
                           nnz, bad);
        if (int e = check_launch("place_kernel")) return e;
        hipLaunchKernelGGL(row_len_kernel, dim3(as_grid(p.kind == 2 ? p.m : p.nseg)), dim3(AS_BLOCK), 0, st, p,
                           cursor, bad);
        if (int e = check_launch("row_len_kernel")) return e;
    }
    JLUST_HIP_TRY(hipMemcpyAsync(&h[0], bad, 4, hipMemcpyDeviceToHost, st));
    JLUST_HIP_TRY(hipStreamSynchronize(st));
    if (h[0] & BAD_COL)
        return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "csr_assemble: a block column index is out of range");
    if (h[0])
        return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "csr_assemble: inconsistent block storage (code %d)", h[0]);
    return JLUST_STATUS_SUCCESS;
}

}  // namespace
}  // namespace jlust

using namespace jlust;

static int csr_assemble_body(int64_t m, int64_t n, int32_t nplacements, const jlust_placement *placements,
                             int value_type, int32_t *rowptr, int32_t *colind, void *val, int64_t nnz,
                             jlust_stream_t stream)
{
    clear_error();
    if (m < 0 || n < 0 || m >= INT32_MAX || n > INT32_MAX || nnz < 0 || nnz > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_assemble: extents outside the Int32 range");
    if (nplacements < 0 || (nplacements > 0 && !placements))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_assemble: bad placement list");
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "csr_assemble: value_type %d", value_type);
    if (!rowptr || bad_ptr(colind, nnz) || bad_ptr(val, nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_assemble: null output pointer");
    std::vector<Piece> ps((size_t)nplacements);
    int64_t total = 0;
    for (int i = 0; i < nplacements; ++i) {
        if (int st = to_piece(placements[i], m, n, i, ps[(size_t)i])) return st;
        total += ps[(size_t)i].nnz;
    }
    if (total != nnz)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_assemble: placements hold %lld values, nnz is %lld",
                    (long long)total, (long long)nnz);
    if (int st = require_device(nullptr)) return st;
    hipStream_t s = (hipStream_t)stream;
    return value_type == 0 ? assemble<double>(m, ps, rowptr, colind, (double *)val, nnz, s)
                           : assemble<float>(m, ps, rowptr, colind, (float *)val, nnz, s);
}

extern "C" int jlust_hip_csr_assemble(int64_t m, int64_t n, int32_t nplacements, const jlust_placement *placements,
                                      int value_type, int32_t *rowptr, int32_t *colind, void *val, int64_t nnz,
                                      jlust_stream_t stream)
{
    return jlust::host_guard("csr_assemble", [&] {
        return csr_assemble_body(m, n, nplacements, placements, value_type, rowptr, colind, val, nnz, stream);
    });
}

extern "C" int jlust_hip_scatter_values(void *dst, int64_t dst_len, const int32_t *slots, const void *src,
                                        int64_t len, int value_type, jlust_stream_t stream)
{
    clear_error();
    if (len < 0 || dst_len < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "scatter_values: negative length");
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "scatter_values: value_type %d", value_type);
    if (bad_ptr(dst, dst_len) || bad_ptr(slots, len) || bad_ptr(src, len))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "scatter_values: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (len == 0) return JLUST_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;
    if (value_type == 0)
        hipLaunchKernelGGL(scatter_kernel<double>, dim3(as_grid(len)), dim3(AS_BLOCK), 0, s, (double *)dst, dst_len,
                           slots, (const double *)src, len);
    else
        hipLaunchKernelGGL(scatter_kernel<float>, dim3(as_grid(len)), dim3(AS_BLOCK), 0, s, (float *)dst, dst_len,
                           slots, (const float *)src, len);
    return check_launch("scatter_kernel");
}

extern "C" int jlust_hip_shifted_diag_spmv_f64(int64_t m, int64_t n, int64_t shift, double val, double alpha,
                                               const double *x, double beta, double *y, jlust_stream_t stream)
{
    return shifted_diag_spmv<double>(m, n, shift, val, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_shifted_diag_spmv_f32(int64_t m, int64_t n, int64_t shift, float val, float alpha,
                                               const float *x, float beta, float *y, jlust_stream_t stream)
{
    return shifted_diag_spmv<float>(m, n, shift, val, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_shifted_diag_spmm_f64(int64_t m, int64_t n, int64_t k, int64_t shift, double val,
                                               double alpha, const double *B, int64_t ldb, double beta, double *C,
                                               int64_t ldc, jlust_stream_t stream)
{
    return shifted_diag_spmm<double>(m, n, k, shift, val, alpha, B, ldb, beta, C, ldc, stream);
}

extern "C" int jlust_hip_shifted_diag_spmm_f32(int64_t m, int64_t n, int64_t k, int64_t shift, float val,
                                               float alpha, const float *B, int64_t ldb, float beta, float *C,
                                               int64_t ldc, jlust_stream_t stream)
{
    return shifted_diag_spmm<float>(m, n, k, shift, val, alpha, B, ldb, beta, C, ldc, stream);
}

namespace jlust {
int preload_assemble()
{
    JLUST_PRELOAD_KERNEL(row_len_kernel);
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
