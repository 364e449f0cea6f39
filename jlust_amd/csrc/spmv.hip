// spmv.hip -- CSR SpMV y = alpha*A*x + beta*y for gfx950 (wave64).
//
// Replaces the CSR branch of execute(::EmitterBackend, ::Op{:SpMV}, ...)
// (ext/KernelAbstractionsExt/ops/spmv.jl:449-502), whose per-row arithmetic is
// `acc = 0; for k in row: acc += val[k]*x[col[k]]; y = alpha*acc (+beta*y)`
// (spmv.jl:154-169, _walker.jl:123-132).
//
// Work split: the merge path of (m row ends, nnz nonzeros) is cut into tiles
// of TILE = BLOCK*IPT items, so every tile costs the same whatever the row
// lengths (a 10^5-nonzero row spans ~50 tiles; 10^4 empty rows share one).
// Each block owns `tiles_per_block` consecutive tiles and finds only its first
// coordinate in global memory (a 64-ary wave-parallel search of rowptr); the
// next tile starts where the previous one ended, found from the row ends the
// tile already staged in LDS.  Per tile:
//   1. the row ends of rows i0..i0+TILE are staged in LDS (coalesced);
//   2. every thread locates its IPT-item slice of the tile by binary search in
//      LDS, and the tile end by the same search;
//   3. products val[k]*x[col[k]] of the tile's nonzeros are staged in LDS:
//      col/val stream coalesced, x is gathered (the only random traffic);
//   4. each thread walks its slice sequentially, closing rows as it meets
//      their ends; partial sums of rows cut by slice borders are combined by
//      a wave64 segmented scan (shuffles) plus a 4-wave LDS step;
//   5. finished rows are written to y coalesced, as alpha*sum (+beta*y).
// A row still open at the end of a block leaves (row, partial) in a carry
// slot; a small second kernel adds each run of equal-row carries into y in
// block order, so the result is deterministic run to run.
#include "common.hpp"

namespace jlust {
namespace {

constexpr int SPMV_BLOCK = 256;
template <typename T> struct SpmvIpt;
template <> struct SpmvIpt<double> { static constexpr int value = 8; };
template <> struct SpmvIpt<float> { static constexpr int value = 8; };

// Smallest i in [max(0, d-nnz), min(d, m)] with (rowptr[i+1]-origin) + i >= d,
// taking i == m as true: the number of rows finished after the first d items
// of the merge path.  Called by a whole wave; every lane returns the answer.
__device__ int64_t wave_merge_search(const int32_t *__restrict__ rowptr, int32_t origin,
                                     int64_t m, int64_t nnz, int64_t d)
{
    const int lane = __lane_id();
    int64_t lo = d - nnz > 0 ? d - nnz : 0;
    int64_t hi = d < m ? d : m;
    while (lo < hi) {
        const int64_t n = hi - lo;
        const int64_t p = lo + (n * lane) / 64;
        const bool pred = (p >= m) || ((int64_t)rowptr[p + 1] - origin + p >= d);
        const uint64_t mask = __ballot(pred);
        if (mask & 1ull) return lo;
        const int f = mask ? __builtin_ctzll(mask) : 64;
        const int64_t new_hi = f < 64 ? lo + (n * f) / 64 : hi;
        lo = lo + (n * (f - 1)) / 64 + 1;
        hi = new_hi;
    }
    return lo;
}

template <typename T, int BLOCK, int IPT>
__global__ __launch_bounds__(BLOCK) void csr_spmv_merge_kernel(
    int64_t m, int64_t nnz, int32_t origin, const int32_t *__restrict__ rowptr,
    const int32_t *__restrict__ colind, const T *__restrict__ val, const T *__restrict__ x,
    T *__restrict__ y, T alpha, T beta, int beta_zero, int64_t tiles_per_block,
    const int64_t *__restrict__ start_rows, int64_t *__restrict__ carry_row,
    T *__restrict__ carry_val)
{
    constexpr int TILE = BLOCK * IPT;
    constexpr int NW = BLOCK / 64;
    __shared__ T s_prod[TILE];
    __shared__ T s_ysum[TILE];
    __shared__ int32_t s_rowend[TILE + 1];
    __shared__ int64_t s_i0;
    __shared__ int32_t s_wkey[NW];
    __shared__ T s_wval[NW];
    __shared__ T s_bs[NW];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t total = m + nnz;
    const int64_t dbeg = (int64_t)blockIdx.x * tiles_per_block * TILE;
    if (dbeg >= total) return;
    const int64_t dend = min(total, dbeg + tiles_per_block * (int64_t)TILE);

    if (start_rows) {
        if (tid == 0) s_i0 = start_rows[blockIdx.x];
    } else if (wave == 0) {
        const int64_t r = wave_merge_search(rowptr, origin, m, nnz, dbeg);
        if (lane == 0) s_i0 = r;
    }
    __syncthreads();
    int64_t i0 = s_i0;
    int64_t j0 = dbeg - i0;
    T carry = T(0);
    bool carry_has = false;

    for (int64_t d = dbeg; d < dend; d += TILE) {
        const int tlen = (int)min((int64_t)TILE, dend - d);
        // (1) row ends (0-based nonzero index) of rows i0 .. i0+tlen.
        for (int r = tid; r <= tlen; r += BLOCK) {
            const int64_t row = i0 + r;
            s_rowend[r] = row < m ? rowptr[row + 1] - origin : INT32_MAX;
        }
        __syncthreads();

        // (2) smallest local row r in [0, dl] whose end lies at or past diagonal dl.
        auto search = [&](int dl) {
            int lo = 0, hi = dl;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if ((int64_t)s_rowend[mid] - j0 + mid >= dl) hi = mid;
                else lo = mid + 1;
            }
            return lo;
        };
        const int dl = min(tid * IPT, tlen);
        const int dl_next = min(dl + IPT, tlen);
        const int rend = search(tlen);
        int r = search(dl);
        int jl = dl - r;
        const int r_first = r;
        const int64_t j1 = d + tlen - (i0 + rend);
        // j1 <= nnz whenever rowptr[m] - origin == nnz; the clamp keeps a
        // malformed rowptr from reading past the nonzero arrays.
        const int nloc = (int)(min(j1, nnz) - j0);

        // (3) products of the tile's nonzeros into LDS.
        {
            int32_t c[IPT];
            T v[IPT];
            T xv[IPT];
#pragma unroll
            for (int u = 0; u < IPT; ++u) {
                const int q = tid + u * BLOCK;
                if (q < nloc) {
                    c[u] = colind[j0 + q];
                    v[u] = val[j0 + q];
                }
            }
#pragma unroll
            for (int u = 0; u < IPT; ++u) {
                const int q = tid + u * BLOCK;
                if (q < nloc) xv[u] = x[c[u] - origin];
            }
#pragma unroll
            for (int u = 0; u < IPT; ++u) {
                const int q = tid + u * BLOCK;
                if (q < nloc) s_prod[q] = v[u] * xv[u];
            }
        }
        __syncthreads();

        // (4) sequential walk of this thread's slice of the merge path.
        T acc = T(0);
        for (int s = dl; s < dl_next; ++s) {
            if ((int64_t)jl < (int64_t)s_rowend[r] - j0) {
                acc += s_prod[jl];
                ++jl;
            } else {
                s_ysum[r] = acc;
                acc = T(0);
                ++r;
            }
        }
        if (tid == 0) {          // partial sum of row i0 left by the previous tile
            if (r > 0) s_ysum[0] += carry;
            else acc += carry;
        }

        // Segmented inclusive scan of (row, partial) over the block, in thread order.
        int key = r;
        T sv = acc;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int k2 = __shfl_up(key, off, 64);
            const T v2 = __shfl_up(sv, off, 64);
            if (lane >= off && k2 == key) sv += v2;
        }
        if (lane == 63) {
            s_wkey[wave] = key;
            s_wval[wave] = sv;
        }
        __syncthreads();
        if (tid == 0) {
            T run = s_wval[0];
            s_bs[0] = run;
            for (int w = 1; w < NW; ++w) {
                T b = s_wval[w];
                if (s_wkey[w] == s_wkey[w - 1]) b += run;
                s_bs[w] = b;
                run = b;
            }
        }
        __syncthreads();
        if (wave > 0 && key == s_wkey[wave - 1]) sv += s_bs[wave - 1];
        T prev = __shfl_up(sv, 1, 64);
        if (lane == 0) prev = wave > 0 ? s_bs[wave - 1] : T(0);
        if (tid > 0 && r > r_first) s_ysum[r_first] += prev;
        __syncthreads();

        // (5) finished rows i0 .. i0+rend-1.
        for (int q = tid; q < rend; q += BLOCK) {
            const int64_t row = i0 + q;
            const T s = alpha * s_ysum[q];
            y[row] = beta_zero ? s : s + beta * y[row];
        }
        if (rend > 0) carry_has = j1 > (int64_t)s_rowend[rend - 1];
        else carry_has = carry_has || (j1 > j0);
        carry = s_bs[NW - 1];
        i0 += rend;
        j0 = j1;
        __syncthreads();
    }
    if (tid == 0) {
        carry_row[blockIdx.x] = (i0 < m && carry_has) ? i0 : -1;
        carry_val[blockIdx.x] = carry;
    }
}

// Adds each run of equal-row carries (in block order) into y.
template <typename T>
__global__ void spmv_carry_fixup_kernel(int64_t nblocks, const int64_t *__restrict__ carry_row,
                                        const T *__restrict__ carry_val, T *__restrict__ y, T alpha)
{
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const int64_t r = carry_row[b];
    if (r < 0) return;
    if (b > 0 && carry_row[b - 1] == r) return;
    T s = carry_val[b];
    for (int64_t u = b + 1; u < nblocks && carry_row[u] == r; ++u) s += carry_val[u];
    atomicAdd(&y[r], alpha * s);
}

__global__ void merge_start_kernel(int64_t m, int64_t nnz, int32_t origin,
                                   const int32_t *__restrict__ rowptr, int64_t items_per_block,
                                   int64_t nblocks, int64_t *__restrict__ start_rows)
{
    const int64_t b = blockIdx.x;
    if (b >= nblocks) return;
    const int64_t r = wave_merge_search(rowptr, origin, m, nnz, b * items_per_block);
    if (__lane_id() == 0) start_rows[b] = r;
}

struct SpmvGrid {
    int64_t tiles_per_block = 1;
    int64_t nblocks = 0;
};

template <typename T>
int spmv_grid(int64_t m, int64_t nnz, SpmvGrid *g)
{
    constexpr int TILE = SPMV_BLOCK * SpmvIpt<T>::value;
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    static int occ_cache[2][64] = {};
    int &occ = occ_cache[sizeof(T) == 8 ? 0 : 1][dev & 63];
    if (occ == 0) {
        int nb = 0;
        JLUST_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &nb, csr_spmv_merge_kernel<T, SPMV_BLOCK, SpmvIpt<T>::value>, SPMV_BLOCK, 0));
        occ = nb > 0 ? nb : 1;
    }
    const int64_t target = (int64_t)occ * device_info(dev).cu_count;
    const int64_t ntiles = (m + nnz + TILE - 1) / TILE;
    g->tiles_per_block = ntiles / (target > 0 ? target : 1);
    if (g->tiles_per_block < 1) g->tiles_per_block = 1;
    g->nblocks = (ntiles + g->tiles_per_block - 1) / g->tiles_per_block;
    return JLUST_STATUS_SUCCESS;
}

int check_spmv_args(int64_t m, int64_t n, int64_t nnz, int32_t origin, const void *rowptr,
                    const void *colind, const void *val, const void *x, const void *y)
{
    if (m < 0 || n < 0 || nnz < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_spmv: negative extent (m=%lld n=%lld nnz=%lld)",
                    (long long)m, (long long)n, (long long)nnz);
    if (m > INT32_MAX || n > INT32_MAX || nnz > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "csr_spmv: extents exceed the Int32 index range (m=%lld n=%lld nnz=%lld)",
                    (long long)m, (long long)n, (long long)nnz);
    if (int st = check_origin(origin)) return st;
    if ((m > 0 && !rowptr) || bad_ptr(colind, nnz) || bad_ptr(val, nnz) ||
        (nnz > 0 && n > 0 && !x) || bad_ptr(y, m))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_spmv: null device pointer");
    if (nnz > 0 && n == 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_spmv: nnz > 0 with n == 0");
    return JLUST_STATUS_SUCCESS;
}

template <typename T>
int spmv_launch(int64_t m, int64_t nnz, int32_t origin, const int32_t *rowptr,
                const int32_t *colind, const T *val, T alpha, const T *x, T beta, T *y,
                const SpmvGrid &g, const int64_t *start_rows, int64_t *carry_row, T *carry_val,
                hipStream_t stream)
{
    constexpr int IPT = SpmvIpt<T>::value;
    hipLaunchKernelGGL((csr_spmv_merge_kernel<T, SPMV_BLOCK, IPT>), dim3((unsigned)g.nblocks),
                       dim3(SPMV_BLOCK), 0, stream, m, nnz, origin, rowptr, colind, val, x, y,
                       alpha, beta, (int)(beta == T(0)), g.tiles_per_block, start_rows,
                       carry_row, carry_val);
    if (int st = check_launch("csr_spmv_merge_kernel")) return st;
    // A single block ends on the last row end, so it never leaves a carry.
    if (g.nblocks > 1) {
        hipLaunchKernelGGL((spmv_carry_fixup_kernel<T>), dim3((unsigned)((g.nblocks + 255) / 256)),
                           dim3(256), 0, stream, g.nblocks, carry_row, carry_val, y, alpha);
        if (int st = check_launch("spmv_carry_fixup_kernel")) return st;
    }
    return JLUST_STATUS_SUCCESS;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

template <typename T>
int csr_spmv(int64_t m, int64_t n, int64_t nnz, int32_t origin, const int32_t *rowptr,
             const int32_t *colind, const T *val, T alpha, const T *x, T beta, T *y,
             jlust_stream_t stream)
{
    clear_error();
    if (int st = check_spmv_args(m, n, nnz, origin, rowptr, colind, val, x, y)) return st;
    if (int st = require_device(nullptr)) return st;
    if (m == 0) return JLUST_STATUS_SUCCESS;
    SpmvGrid g;
    if (int st = spmv_grid<T>(m, nnz, &g)) return st;
    void *ws = nullptr;
    const size_t rows_bytes = align_up(sizeof(int64_t) * (size_t)g.nblocks, 256);
    if (int st = scratch(stream, rows_bytes + sizeof(T) * (size_t)g.nblocks, &ws)) return st;
    int64_t *carry_row = (int64_t *)ws;
    T *carry_val = (T *)((char *)ws + rows_bytes);
    return spmv_launch<T>(m, nnz, origin, rowptr, colind, val, alpha, x, beta, y, g, nullptr,
                          carry_row, carry_val, (hipStream_t)stream);
}

}  // namespace
}  // namespace jlust

// ------------------------------------------------------------------- plans

struct jlust_spmv_plan {
    int64_t m, n, nnz;
    int32_t origin;
    int value_type;  // 0 f64, 1 f32
    const int32_t *rowptr;
    const int32_t *colind;
    const void *val;
    jlust::SpmvGrid grid;
    int device;
    void *mem;        // start rows | carry rows | carry values
    int64_t *start_rows;
    int64_t *carry_row;
    void *carry_val;
};

using namespace jlust;

extern "C" int jlust_hip_csr_spmv_f64_i32(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                          const int32_t *rowptr, const int32_t *colind,
                                          const double *val, double alpha, const double *x,
                                          double beta, double *y, jlust_stream_t stream)
{
    return csr_spmv<double>(m, n, nnz, origin, rowptr, colind, val, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_csr_spmv_f32_i32(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                          const int32_t *rowptr, const int32_t *colind,
                                          const float *val, float alpha, const float *x,
                                          float beta, float *y, jlust_stream_t stream)
{
    return csr_spmv<float>(m, n, nnz, origin, rowptr, colind, val, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_csr_spmv_plan_create(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                              int value_type, const int32_t *rowptr,
                                              const int32_t *colind, const void *val,
                                              jlust_stream_t stream, jlust_spmv_plan_t *plan_out)
{
    clear_error();
    if (!plan_out) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_create: null plan_out");
    *plan_out = nullptr;
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE,
                    "spmv_plan_create: value_type %d (0 = Float64, 1 = Float32)", value_type);
    if (int st = check_spmv_args(m, n, nnz, origin, rowptr, colind, val, (const void *)1,
                                 (const void *)1))
        return st;
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    SpmvGrid g;
    if (m > 0) {
        int st = value_type == 0 ? spmv_grid<double>(m, nnz, &g) : spmv_grid<float>(m, nnz, &g);
        if (st) return st;
    }
    const size_t tsz = value_type == 0 ? sizeof(double) : sizeof(float);
    const size_t nb = (size_t)(g.nblocks > 0 ? g.nblocks : 1);
    const size_t sz_rows = align_up(sizeof(int64_t) * nb, 256);
    void *mem = nullptr;
    JLUST_HIP_TRY(hipMalloc(&mem, 2 * sz_rows + tsz * nb));
    auto *p = new jlust_spmv_plan{m, n, nnz, origin, value_type, rowptr, colind, val, g, dev, mem,
                                  (int64_t *)mem, (int64_t *)((char *)mem + sz_rows),
                                  (char *)mem + 2 * sz_rows};
    if (m > 0) {
        const int tile = SPMV_BLOCK * (value_type == 0 ? SpmvIpt<double>::value : SpmvIpt<float>::value);
        hipLaunchKernelGGL(merge_start_kernel, dim3((unsigned)g.nblocks), dim3(64), 0,
                           (hipStream_t)stream, m, nnz, origin, rowptr,
                           g.tiles_per_block * (int64_t)tile, g.nblocks, p->start_rows);
        if (int st = check_launch("merge_start_kernel")) {
            (void)hipFree(mem);
            delete p;
            return st;
        }
    }
    *plan_out = p;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_csr_spmv_plan_update_values(jlust_spmv_plan_t plan, const void *val)
{
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_update_values: null plan");
    if (bad_ptr(val, plan->nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_update_values: null values");
    plan->val = val;
    return JLUST_STATUS_SUCCESS;
}

template <typename T>
static int plan_execute(jlust_spmv_plan_t plan, int want_type, T alpha, const T *x, T beta, T *y,
                        jlust_stream_t stream)
{
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_execute: null plan");
    if (plan->value_type != want_type)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE,
                    "spmv_plan_execute: plan was created for %s values",
                    plan->value_type == 0 ? "Float64" : "Float32");
    if ((plan->nnz > 0 && !x) || bad_ptr(y, plan->m))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_execute: null vector");
    if (plan->m == 0) return JLUST_STATUS_SUCCESS;
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    if (dev != plan->device)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "spmv_plan_execute: plan belongs to device %d, current device is %d",
                    plan->device, dev);
    return spmv_launch<T>(plan->m, plan->nnz, plan->origin, plan->rowptr, plan->colind,
                          (const T *)plan->val, alpha, x, beta, y, plan->grid, plan->start_rows,
                          plan->carry_row, (T *)plan->carry_val, (hipStream_t)stream);
}

extern "C" int jlust_hip_csr_spmv_plan_execute_f64(jlust_spmv_plan_t plan, double alpha,
                                                   const double *x, double beta, double *y,
                                                   jlust_stream_t stream)
{
    return plan_execute<double>(plan, 0, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_csr_spmv_plan_execute_f32(jlust_spmv_plan_t plan, float alpha,
                                                   const float *x, float beta, float *y,
                                                   jlust_stream_t stream)
{
    return plan_execute<float>(plan, 1, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_csr_spmv_plan_destroy(jlust_spmv_plan_t plan)
{
    clear_error();
    if (!plan) return JLUST_STATUS_SUCCESS;
    hipError_t e = hipFree(plan->mem);
    delete plan;
    if (e != hipSuccess) return hip_fail(e, "hipFree(plan)");
    return JLUST_STATUS_SUCCESS;
}
