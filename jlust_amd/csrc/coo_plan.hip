// coo_plan.hip -- prepared COO SpMV: the entries put in row order once, then
// every product runs in the CSR SpMV plan (merge-path tiles, no atomics,
// deterministic).
//
// The reference's COO SpMV pre-scales y by beta and adds alpha*val*x[col]
// into y[row] with atomics (ext/KernelAbstractionsExt/ops/spmv.jl:407-448;
// CUDAExt.jl:91-104); the cuSPARSE handles it offers are analysed once and
// refreshed with update_values! (ext/CUDAExt/ops/spmv.jl:7-83).  A CSR over
// the same entries gives y = alpha*A*x + beta*y with every entry summed once
// (duplicates included) and rows without entries scaled by beta, i.e. the
// same matrix product.  Analysis: a check of the row indices (in range; in
// non-decreasing order or not), then, only for unsorted rows, a stable radix
// sort of (row, position) pairs (rocPRIM) and gathers of the columns and
// values into row order; row pointers by binary search of the sorted rows.
#include <cstring>

#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>

#include "common.hpp"

namespace jlust {
namespace {

constexpr int CP_BLOCK = 256;

unsigned cp_grid(int64_t n) { return (unsigned)((n + CP_BLOCK - 1) / CP_BLOCK); }

// flags[0] |= 1: a row outside [origin, m + origin); flags[0] |= 2: rows decrease somewhere.
__global__ void coo_rows_check_kernel(int64_t nnz, const int32_t *__restrict__ rows, int32_t origin, int64_t m,
                                      uint32_t *__restrict__ keys, int32_t *__restrict__ iota,
                                      int32_t *__restrict__ flags)
{
    const int64_t i = (int64_t)blockIdx.x * CP_BLOCK + threadIdx.x;
    if (i >= nnz) return;
    const int64_t r = (int64_t)rows[i] - origin;
    int32_t f = 0;
    if (r < 0 || r >= m) f |= 1;
    if (i > 0 && rows[i] < rows[i - 1]) f |= 2;
    // One atomic per wave, and none once the flags hold the wave's bits: the
    // rows of a shuffled COO set bit 2 in about half of the entries.
    const int32_t wf = (__ballot(f & 1) ? 1 : 0) | (__ballot(f & 2) ? 2 : 0);
    if (wf && __lane_id() == (int)__builtin_ctzll(__ballot(1)) &&
        (__hip_atomic_load(flags, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & wf) != wf)
        atomicOr(flags, wf);
    keys[i] = (uint32_t)(r < 0 ? 0 : (r >= m ? m - 1 : r));
    iota[i] = (int32_t)i;
}

// rowptr[i] = origin + (entries with row < i), i in [0, m]; keys sorted, 0-based.
__global__ void coo_rowptr_kernel(int64_t nnz, const uint32_t *__restrict__ keys, int64_t m, int32_t origin,
                                  int32_t *__restrict__ rowptr)
{
    const int64_t i = (int64_t)blockIdx.x * CP_BLOCK + threadIdx.x;
    if (i > m) return;
    int64_t lo = 0, hi = nnz;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((int64_t)keys[mid] < i) lo = mid + 1;
        else hi = mid;
    }
    rowptr[i] = (int32_t)(lo + origin);
}

__global__ void coo_gather_cols_kernel(int64_t nnz, const int32_t *__restrict__ perm,
                                       const int32_t *__restrict__ cols, int32_t *__restrict__ cols_out)
{
    const int64_t i = (int64_t)blockIdx.x * CP_BLOCK + threadIdx.x;
    if (i >= nnz) return;
    cols_out[i] = cols[perm[i]];
}

template <typename T>
__global__ void coo_gather_kernel(int64_t nnz, const int32_t *__restrict__ perm, const T *__restrict__ val,
                                  T *__restrict__ val_out)
{
    const int64_t i = (int64_t)blockIdx.x * CP_BLOCK + threadIdx.x;
    if (i >= nnz) return;
    val_out[i] = val[perm[i]];
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

int bits_for(int64_t n)
{
    int b = 1;
    while (b < 32 && ((int64_t)1 << b) < n) ++b;
    return b;
}

struct Mem {
    void *p = nullptr;
    ~Mem() { if (p) (void)hipFree(p); }
};

}  // namespace
}  // namespace jlust

namespace jlust {

int coo_row_order(int64_t m, int64_t nnz, int32_t origin, const int32_t *rows, const int32_t *cols,
                  int32_t *rowptr, int32_t *perm, int32_t *cols_out, bool *sorted, hipStream_t s)
{
    const size_t nz = (size_t)(nnz > 0 ? nnz : 1);
    const size_t sz_i = align256(4 * nz);
    // Scratch: keys x2, iota, flags, sort temporary.
    size_t sort_bytes = 0;
    JLUST_HIP_TRY(rocprim::radix_sort_pairs(nullptr, sort_bytes, (uint32_t *)nullptr, (uint32_t *)nullptr,
                                            (int32_t *)nullptr, (int32_t *)nullptr, nz, 0, bits_for(m), s));
    Mem work;
    JLUST_HIP_TRY(hipMalloc(&work.p, 3 * sz_i + 256 + align256(sort_bytes)));
    char *w = (char *)work.p;
    uint32_t *keys = (uint32_t *)w;
    uint32_t *keys_s = (uint32_t *)(w + sz_i);
    int32_t *iota = (int32_t *)(w + 2 * sz_i);
    int32_t *flags = (int32_t *)(w + 3 * sz_i);
    void *sort_tmp = w + 3 * sz_i + 256;
    JLUST_HIP_TRY(hipMemsetAsync(flags, 0, 4, s));
    if (nnz > 0) {
        hipLaunchKernelGGL(coo_rows_check_kernel, dim3(cp_grid(nnz)), dim3(CP_BLOCK), 0, s, nnz, rows, origin, m,
                           keys, iota, flags);
        if (int st = check_launch("coo_rows_check_kernel")) return st;
    }
    int32_t fh = 0;
    JLUST_HIP_TRY(hipMemcpyAsync(&fh, flags, 4, hipMemcpyDeviceToHost, s));
    JLUST_HIP_TRY(hipStreamSynchronize(s));
    if (fh & 1) return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "COO analysis: a row index is out of range");
    *sorted = !(fh & 2);
    const uint32_t *sorted_keys = keys;
    if (!*sorted) {
        JLUST_HIP_TRY(rocprim::radix_sort_pairs(sort_tmp, sort_bytes, keys, keys_s, iota, perm, (size_t)nnz, 0,
                                                bits_for(m), s));
        hipLaunchKernelGGL(coo_gather_cols_kernel, dim3(cp_grid(nnz)), dim3(CP_BLOCK), 0, s, nnz, perm, cols,
                           cols_out);
        if (int st = check_launch("coo_gather_cols_kernel")) return st;
        sorted_keys = keys_s;
    }
    hipLaunchKernelGGL(coo_rowptr_kernel, dim3(cp_grid(m + 1)), dim3(CP_BLOCK), 0, s, nnz, sorted_keys, m, origin,
                       rowptr);
    if (int st = check_launch("coo_rowptr_kernel")) return st;
    JLUST_HIP_TRY(hipStreamSynchronize(s));       // the scratch is freed on return
    return JLUST_STATUS_SUCCESS;
}

}  // namespace jlust

using namespace jlust;

static int coo_spmv_plan_create_body(int64_t m, int64_t n, int64_t nnz, int32_t origin, int value_type,
                                     const int32_t *rows, const int32_t *cols, const void *val,
                                     jlust_stream_t stream, jlust_spmv_plan_t *plan_out)
{
    clear_error();
    if (!plan_out) return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmv_plan_create: null plan_out");
    *plan_out = nullptr;
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "coo_spmv_plan_create: value_type %d", value_type);
    if (m < 0 || n < 0 || nnz < 0 || m > INT32_MAX - 1 || n > INT32_MAX || nnz > INT32_MAX - 1)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmv_plan_create: extents outside the Int32 range");
    if (int st = check_origin(origin)) return st;
    if (bad_ptr(rows, nnz) || bad_ptr(cols, nnz) || bad_ptr(val, nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmv_plan_create: null device pointer");
    if (nnz > 0 && (m == 0 || n == 0))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_spmv_plan_create: entries in an empty matrix");
    if (int st = require_device(nullptr)) return st;
    hipStream_t s = (hipStream_t)stream;
    const size_t tsz = value_type == 0 ? 8 : 4;
    const size_t nz = (size_t)(nnz > 0 ? nnz : 1);
    // Owned for the plan's life: rowptr [, perm, columns and values in row order].
    const size_t sz_rp = align256(4 * (size_t)(m + 1));
    const size_t sz_i = align256(4 * nz);
    const size_t sz_v = align256(tsz * nz);
    Mem own;
    JLUST_HIP_TRY(hipMalloc(&own.p, sz_rp + 2 * sz_i + sz_v));
    char *b = (char *)own.p;
    int32_t *rowptr = (int32_t *)b;
    int32_t *perm = (int32_t *)(b + sz_rp);
    int32_t *cols_s = (int32_t *)(b + sz_rp + sz_i);
    void *val_s = b + sz_rp + 2 * sz_i;
    bool sorted = true;
    if (int st = coo_row_order(m, nnz, origin, rows, cols, rowptr, perm, cols_s, &sorted, s)) return st;
    const int32_t *csr_cols = cols;
    const void *csr_val = val;
    if (!sorted) {
        if (value_type == 0)
            hipLaunchKernelGGL(coo_gather_kernel<double>, dim3(cp_grid(nnz)), dim3(CP_BLOCK), 0, s, nnz, perm,
                               (const double *)val, (double *)val_s);
        else
            hipLaunchKernelGGL(coo_gather_kernel<float>, dim3(cp_grid(nnz)), dim3(CP_BLOCK), 0, s, nnz, perm,
                               (const float *)val, (float *)val_s);
        if (int st = check_launch("coo_gather_kernel")) return st;
        csr_cols = cols_s;
        csr_val = val_s;
    }
    jlust_spmv_plan_t plan = nullptr;
    if (int st = jlust_hip_csr_spmv_plan_create(m, n, nnz, origin, value_type, rowptr, csr_cols, csr_val, stream,
                                                &plan))
        return st;
    JLUST_HIP_TRY(hipStreamSynchronize(s));
    spmv_plan_adopt_coo(plan, own.p, sorted ? nullptr : perm, sorted ? nullptr : val_s, sz_rp + 2 * sz_i + sz_v);
    own.p = nullptr;
    *plan_out = plan;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_coo_spmv_plan_create(int64_t m, int64_t n, int64_t nnz, int32_t origin, int value_type,
                                             const int32_t *rows, const int32_t *cols, const void *val,
                                             jlust_stream_t stream, jlust_spmv_plan_t *plan_out)
{
    return jlust::host_guard("coo_spmv_plan_create", [&] {
        return coo_spmv_plan_create_body(m, n, nnz, origin, value_type, rows, cols, val, stream, plan_out);
    });
}

namespace jlust {
// A tiny sort of `n` (key, value) pairs through the instantiation `Sort`
// uses, into a temporary that is freed after the stream drains.
template <typename K, typename V>
static int preload_radix_sort(hipStream_t s, int bits)
{
    constexpr size_t n = 64;
    size_t need = 0;
    JLUST_HIP_TRY(rocprim::radix_sort_pairs(nullptr, need, (K *)nullptr, (K *)nullptr, (V *)nullptr, (V *)nullptr,
                                            n, 0, bits, s));
    void *buf = nullptr;
    const size_t sz = 4 * n * 8 + (need + 255) / 256 * 256;
    JLUST_HIP_TRY(hipMalloc(&buf, sz));
    char *b = (char *)buf;
    K *k0 = (K *)b, *k1 = (K *)(b + n * 8);
    V *v0 = (V *)(b + 2 * n * 8), *v1 = (V *)(b + 3 * n * 8);
    hipError_t e = hipMemsetAsync(buf, 0, 4 * n * 8, s);
    if (e == hipSuccess) e = rocprim::radix_sort_pairs(b + 4 * n * 8, need, k0, k1, v0, v1, n, 0, bits, s);
    const hipError_t e2 = hipStreamSynchronize(s);
    (void)hipFree(buf);
    if (e != hipSuccess) return hip_fail(e, "preload sort");
    if (e2 != hipSuccess) return hip_fail(e2, "preload sort");
    return JLUST_STATUS_SUCCESS;
}

int preload_coo_plan(hipStream_t s)
{
    JLUST_PRELOAD_KERNEL(coo_rowptr_kernel);
    return preload_radix_sort<uint32_t, int32_t>(s, 20);
}
}  // namespace jlust
