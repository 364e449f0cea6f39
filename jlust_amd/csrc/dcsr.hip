// dcsr.hip -- row gathers and scatters for DCSR products.
//
// A DCSR matrix (i : compressed, j : compressed; src/named_formats.jl:27)
// stores only its non-empty rows: crd1 = their row indices, pos2/crd2/val a
// CSR over those rows.  The reference walks the stored rows and writes y (or
// C) there only: rows not stored stay untouched whatever beta is
// (ext/KernelAbstractionsExt/ops/spmv.jl:449-502 with n_outer = stored rows).
// Here the product runs in the CSR kernels over the compact row set:
//
//   t = y[rows]            (only when beta != 0)
//   t = alpha*A_compact*x + beta*t
//   y[rows] = t
//
// so the product keeps the CSR kernels' load balance and plans; the two row
// passes move O(stored rows * k) values next to the product's O(nnz).
// Row indices outside [0, m) are skipped (memory-safe; canonical DCSR has
// increasing stored rows).
#include "common.hpp"

namespace jlust {
namespace {

constexpr int RW_BLOCK = 256;

// dst[s + c*ldd] = src[rows[s] + c*lds] (GATHER) or dst[rows[s] + c*ldd] =
// src[s + c*lds] (scatter) for s < nrows, c < k.
template <typename T, bool GATHER>
__global__ __launch_bounds__(RW_BLOCK) void rows_kernel(int64_t nrows, int64_t k, int32_t origin,
                                                        const int32_t *__restrict__ rows, int64_t m,
                                                        const T *__restrict__ src, int64_t lds,
                                                        T *__restrict__ dst, int64_t ldd)
{
    const int64_t i = (int64_t)blockIdx.x * RW_BLOCK + threadIdx.x;
    if (i >= nrows * k) return;
    const int64_t s = i % nrows, c = i / nrows;
    const int64_t r = (int64_t)rows[s] - origin;
    if (r < 0 || r >= m) return;
    if (GATHER) dst[s + c * ldd] = src[r + c * lds];
    else dst[r + c * ldd] = src[s + c * lds];
}

template <typename T, bool GATHER>
int rows_copy(int64_t nrows, int64_t k, int32_t origin, const int32_t *rows, int64_t m, const T *src,
              int64_t lds, T *dst, int64_t ldd, jlust_stream_t stream)
{
    clear_error();
    if (nrows < 0 || k < 0 || m < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "dcsr rows: negative extent");
    if (int st = check_origin(origin)) return st;
    const int64_t src_rows = GATHER ? m : nrows, dst_rows = GATHER ? nrows : m;
    if (k > 1 && (lds < src_rows || ldd < dst_rows))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "dcsr rows: leading dimension below the row count");
    if (bad_ptr(rows, nrows) || bad_ptr(src, nrows * k) || bad_ptr(dst, nrows * k))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "dcsr rows: null device pointer");
    if (int st = require_device(nullptr)) return st;
    const int64_t n = nrows * k;
    if (n == 0) return JLUST_STATUS_SUCCESS;
    hipLaunchKernelGGL((rows_kernel<T, GATHER>), dim3((unsigned)((n + RW_BLOCK - 1) / RW_BLOCK)), dim3(RW_BLOCK),
                       0, (hipStream_t)stream, nrows, k, origin, rows, m, src, lds, dst, ldd);
    return check_launch("rows_kernel");
}

}  // namespace
}  // namespace jlust

#define JLUST_ROWS(NAME, T, G)                                                                         \
    extern "C" int NAME(int64_t nrows, int64_t k, int32_t origin, const int32_t *rows, int64_t m,       \
                        const T *src, int64_t lds, T *dst, int64_t ldd, jlust_stream_t stream)          \
    {                                                                                                  \
        return jlust::rows_copy<T, G>(nrows, k, origin, rows, m, src, lds, dst, ldd, stream);          \
    }
JLUST_ROWS(jlust_hip_gather_rows_f64, double, true)
JLUST_ROWS(jlust_hip_gather_rows_f32, float, true)
JLUST_ROWS(jlust_hip_scatter_rows_f64, double, false)
JLUST_ROWS(jlust_hip_scatter_rows_f32, float, false)
#undef JLUST_ROWS

namespace jlust {
int preload_dcsr()
{
    JLUST_PRELOAD_KERNEL((rows_kernel<double, true>));
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
