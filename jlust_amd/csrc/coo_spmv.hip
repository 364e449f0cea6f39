// coo_spmv.hip -- COO SpMV for gfx950: y = beta*y (zero-filled when beta == 0),
// then y += alpha*A*x.
//
// Replaces the COO branch of execute(::EmitterBackend, ::Op{:SpMV}, ...)
// (ext/KernelAbstractionsExt/ops/spmv.jl:407-448): the reference pre-scales y
// by beta and then adds products with atomics, either one per row change over
// 8-nonzero chunks (`_coo_spmv_chunked!`, spmv.jl:217-243) or after a
// warp-segmented reduction (_walker.jl:343-375).
//
// Here a block stages a tile of BLOCK*IPT nonzeros (row keys and products
// val*x[col]) in LDS with coalesced loads; each thread then walks IPT
// consecutive entries and issues one atomic add per run of equal rows in its
// slice.  Rows need not be sorted; sorted input keeps runs long.
#include "common.hpp"

namespace jlust {
namespace {

constexpr int COO_BLOCK = 256;
constexpr int COO_IPT = 8;

template <typename T>
__global__ void scale_kernel(int64_t m, T beta, int beta_zero, T *__restrict__ y)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < m) y[i] = beta_zero ? T(0) : beta * y[i];
}

template <typename T>
__global__ __launch_bounds__(COO_BLOCK) void coo_spmv_kernel(
    int64_t nnz, int32_t origin, const int32_t *__restrict__ rows,
    const int32_t *__restrict__ cols, const T *__restrict__ val, const T *__restrict__ x,
    T *__restrict__ y, T alpha)
{
    constexpr int TILE = COO_BLOCK * COO_IPT;
    __shared__ T s_prod[TILE];
    __shared__ int32_t s_key[TILE];
    const int tid = threadIdx.x;
    const int64_t base = (int64_t)blockIdx.x * TILE;
    const int n = (int)min((int64_t)TILE, nnz - base);

    int32_t c[COO_IPT], rk[COO_IPT];
    T v[COO_IPT], xv[COO_IPT];
#pragma unroll
    for (int u = 0; u < COO_IPT; ++u) {
        const int q = tid + u * COO_BLOCK;
        if (q < n) {
            c[u] = cols[base + q];
            rk[u] = rows[base + q];
            v[u] = val[base + q];
        }
    }
#pragma unroll
    for (int u = 0; u < COO_IPT; ++u) {
        const int q = tid + u * COO_BLOCK;
        if (q < n) xv[u] = x[c[u] - origin];
    }
#pragma unroll
    for (int u = 0; u < COO_IPT; ++u) {
        const int q = tid + u * COO_BLOCK;
        if (q < n) {
            s_prod[q] = v[u] * xv[u];
            s_key[q] = rk[u] - origin;
        }
    }
    __syncthreads();

    const int lo = tid * COO_IPT;
    const int hi = min(lo + COO_IPT, n);
    if (lo >= hi) return;
    int cur = s_key[lo];
    T acc = s_prod[lo];
    for (int q = lo + 1; q < hi; ++q) {
        const int r = s_key[q];
        if (r != cur) {
            atomicAdd(&y[cur], alpha * acc);
            cur = r;
            acc = s_prod[q];
        } else {
            acc += s_prod[q];
        }
    }
    atomicAdd(&y[cur], alpha * acc);
}

template <typename T>
int coo_spmv(int64_t m, int64_t n, int64_t nnz, int32_t origin, const int32_t *rows,
             const int32_t *cols, const T *val, T alpha, const T *x, T beta, T *y,
             jlust_stream_t stream)
{
    clear_error();
    if (m < 0 || n < 0 || nnz < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmv: negative extent");
    if (m > INT32_MAX || n > INT32_MAX || nnz > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmv: extents exceed the Int32 index range");
    if (int st = check_origin(origin)) return st;
    if (bad_ptr(rows, nnz) || bad_ptr(cols, nnz) || bad_ptr(val, nnz) || bad_ptr(x, nnz > 0 ? n : 0) ||
        bad_ptr(y, m))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmv: null device pointer");
    if (nnz > 0 && (m == 0 || n == 0))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmv: nnz > 0 with an empty dimension");
    if (int st = require_device(nullptr)) return st;
    hipStream_t s = (hipStream_t)stream;
    if (m > 0) {
        hipLaunchKernelGGL((scale_kernel<T>), dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, m,
                           beta, (int)(beta == T(0)), y);
        if (int st = check_launch("scale_kernel")) return st;
    }
    if (nnz > 0) {
        const int64_t tile = COO_BLOCK * COO_IPT;
        hipLaunchKernelGGL((coo_spmv_kernel<T>), dim3((unsigned)((nnz + tile - 1) / tile)),
                           dim3(COO_BLOCK), 0, s, nnz, origin, rows, cols, val, x, y, alpha);
        if (int st = check_launch("coo_spmv_kernel")) return st;
    }
    return JLUST_STATUS_SUCCESS;
}

// CSC SpMV in scatter mode (the reference's walk of a column-outer format,
// ext/KernelAbstractionsExt/ops/spmv.jl:391-408, leaf spmv.jl:140-141): y is
// pre-scaled by beta, then every stored (row, col) adds (alpha*val)*x[col]
// into y[row] with an atomic.  A thread takes COO_IPT consecutive entries; the
// column of its first one is found by binary search of colptr, later ones by
// moving on (binary search again past empty columns).  Atomic order varies,
// so the sums vary in their last bits run to run, as the reference's do.
__device__ __forceinline__ int64_t csc_col_of(const int32_t *__restrict__ colptr, int32_t origin, int64_t a,
                                             int64_t b, int64_t p)
{
    // colptr[a] - origin <= p < colptr[b] - origin; returns c with p in column c.
    while (b - a > 1) {
        const int64_t mid = (a + b) >> 1;
        if ((int64_t)colptr[mid] - origin <= p) a = mid;
        else b = mid;
    }
    return a;
}

// Memory-safe on a malformed colptr or rowind: the column search stays in
// [0, n), entries past the end of the last column (colptr[n] - origin < nnz)
// end the thread, and a row outside [0, m) is skipped.
template <typename T>
__global__ __launch_bounds__(COO_BLOCK) void csc_spmv_kernel(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                                             const int32_t *__restrict__ colptr,
                                                             const int32_t *__restrict__ rowind,
                                                             const T *__restrict__ val, const T *__restrict__ x,
                                                             T *__restrict__ y, T alpha)
{
    const int64_t lo = ((int64_t)blockIdx.x * COO_BLOCK + threadIdx.x) * COO_IPT;
    if (lo >= nnz) return;
    const int64_t hi = min(lo + (int64_t)COO_IPT, nnz);
    int64_t c = csc_col_of(colptr, origin, 0, n, lo);
    int64_t cend = (int64_t)colptr[c + 1] - origin;
    T xc = x[c];
    for (int64_t p = lo; p < hi; ++p) {
        if (p >= cend) {
            while (p >= cend) {
                if (c + 1 >= n) return;
                c = csc_col_of(colptr, origin, c + 1, n, p);
                cend = (int64_t)colptr[c + 1] - origin;
            }
            xc = x[c];
        }
        const int64_t r = (int64_t)rowind[p] - origin;
        if (r >= 0 && r < m) atomicAdd(&y[r], (alpha * val[p]) * xc);
    }
}

template <typename T>
int csc_spmv(int64_t m, int64_t n, int64_t nnz, int32_t origin, const int32_t *colptr, const int32_t *rowind,
             const T *val, T alpha, const T *x, T beta, T *y, jlust_stream_t stream)
{
    clear_error();
    if (m < 0 || n < 0 || nnz < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csc_spmv: negative extent");
    if (m > INT32_MAX || n > INT32_MAX - 1 || nnz > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csc_spmv: extents exceed the Int32 index range");
    if (int st = check_origin(origin)) return st;
    if ((n > 0 && !colptr) || bad_ptr(rowind, nnz) || bad_ptr(val, nnz) || bad_ptr(x, nnz > 0 ? n : 0) ||
        bad_ptr(y, m))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csc_spmv: null device pointer");
    if (nnz > 0 && (m == 0 || n == 0))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csc_spmv: nnz > 0 with an empty dimension");
    if (int st = require_device(nullptr)) return st;
    hipStream_t s = (hipStream_t)stream;
    if (m > 0) {
        hipLaunchKernelGGL((scale_kernel<T>), dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, m, beta,
                           (int)(beta == T(0)), y);
        if (int st = check_launch("scale_kernel")) return st;
    }
    if (nnz > 0) {
        const int64_t per_block = (int64_t)COO_BLOCK * COO_IPT;
        hipLaunchKernelGGL((csc_spmv_kernel<T>), dim3((unsigned)((nnz + per_block - 1) / per_block)),
                           dim3(COO_BLOCK), 0, s, m, n, nnz, origin, colptr, rowind, val, x, y, alpha);
        if (int st = check_launch("csc_spmv_kernel")) return st;
    }
    return JLUST_STATUS_SUCCESS;
}

}  // namespace
}  // namespace jlust

using namespace jlust;

extern "C" int jlust_hip_coo_spmv_f64_i32(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                          const int32_t *rows, const int32_t *cols,
                                          const double *val, double alpha, const double *x,
                                          double beta, double *y, jlust_stream_t stream)
{
    return coo_spmv<double>(m, n, nnz, origin, rows, cols, val, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_coo_spmv_f32_i32(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                          const int32_t *rows, const int32_t *cols,
                                          const float *val, float alpha, const float *x,
                                          float beta, float *y, jlust_stream_t stream)
{
    return coo_spmv<float>(m, n, nnz, origin, rows, cols, val, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_csc_spmv_f64_i32(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                          const int32_t *colptr, const int32_t *rowind, const double *val,
                                          double alpha, const double *x, double beta, double *y,
                                          jlust_stream_t stream)
{
    return csc_spmv<double>(m, n, nnz, origin, colptr, rowind, val, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_csc_spmv_f32_i32(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                          const int32_t *colptr, const int32_t *rowind, const float *val,
                                          float alpha, const float *x, float beta, float *y,
                                          jlust_stream_t stream)
{
    return csc_spmv<float>(m, n, nnz, origin, colptr, rowind, val, alpha, x, beta, y, stream);
}

namespace jlust {
int preload_coo_spmv()
{
    JLUST_PRELOAD_KERNEL(scale_kernel<double>);
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
