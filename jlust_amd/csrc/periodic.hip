// SpMV of a T-period block-banded matrix with one diagonal block shared by
// every period and one (neg, pos) coupling pair shared by every transition,
// without materialising the T-fold matrix: the reference's periodic view
// (ext/CUDAExt/ops/block_mul.jl:584-676, fused kernel
// ext/KernelAbstractionsExt/ops/block_periodic.jl:108-236).
//
// Row layout (block_banded.jl:5-14, bandwidth 1): period t (0-based) owns
// rows [t*P, t*P + n_diag) of the diagonal block and, for t < T-1, rows
// [t*P + n_diag, (t+1)*P) of coupling, P = n_diag + n_off.  A diagonal row i
// of period t is row i of D against x[t*n_cols ...]; a coupling row i is row
// i of neg against x[t*n_cols ...] plus row i of pos against
// x[(t+1)*n_cols ...].
//
// A block row is the same in every period, so LPR lanes take a row for PT
// consecutive periods: the row's pointers, columns and values are loaded
// once and its PT gathers of x per entry are independent.  The blocks (a few
// MB for the DCOPF operators) are read T/PT times, mostly from L2, instead of
// as a T-fold matrix from HBM; the x gathers themselves (one per entry and
// period) remain, and they set the time.

#include "common.hpp"

#include <climits>
#include <cstdlib>

namespace jlust {
namespace {

constexpr int PV_U = 4;   // entries per lane per step

// A block as the kernel reads it: CSR (kind 0) or a shifted diagonal
// (kind 1: entry (i, i + shift) = dval for every i with 0 <= i + shift < n).
struct PBlk {
    const int32_t *rowptr;
    const int32_t *colind;
    const void *val;
    int32_t origin;
    int32_t kind;
    int64_t n;
    int64_t shift;
    double dval;
};

// acc[q] += row i of b against period q of x (x[xo[q] + column], q < PT):
// the row's pointers, columns and values are loaded once for all PT
// periods, whose gathers are independent.
template <typename T, int LPR, int PT>
__device__ __forceinline__ void row_walk(const PBlk &b, int32_t i, const T *__restrict__ x,
                                         const int64_t (&xo)[PT], int sub, T (&acc)[PT])
{
    if (b.kind == 1) {
        const int64_t c = (int64_t)i + b.shift;
        if (sub == 0 && c >= 0 && c < b.n) {
#pragma unroll
            for (int q = 0; q < PT; ++q) acc[q] += (T)b.dval * x[xo[q] + c];
        }
        return;
    }
    int32_t rp0 = b.rowptr[i], rp1 = b.rowptr[i + 1];
    __asm__ volatile("" : "+v"(rp0), "+v"(rp1));     // both loads before the first wait
    const int64_t lo = (int64_t)rp0 - b.origin;
    const int64_t hi = (int64_t)rp1 - b.origin;
    const int32_t *__restrict__ colind = b.colind;
    const T *__restrict__ val = (const T *)b.val;
    const int32_t org = b.origin;
    for (int64_t p0 = lo + sub; p0 < hi; p0 += PV_U * LPR) {
        int32_t c[PV_U];
        T v[PV_U], xv[PV_U][PT];
#pragma unroll
        for (int u = 0; u < PV_U; ++u) {
            const int64_t p = min(p0 + u * LPR, hi - 1);
            c[u] = colind[p] - org;
            v[u] = val[p];
        }
#pragma unroll
        for (int u = 0; u < PV_U; ++u)
#pragma unroll
            for (int q = 0; q < PT; ++q) xv[u][q] = x[xo[q] + c[u]];
#pragma unroll
        for (int u = 0; u < PV_U; ++u) {
            const bool ok = p0 + u * LPR < hi;
#pragma unroll
            for (int q = 0; q < PT; ++q) {
                const T a = acc[q] + v[u] * xv[u][q];
                acc[q] = ok ? a : acc[q];
            }
        }
    }
}

// Item = (row i of a period, group of PT consecutive periods), LPR lanes per
// item, items ordered row-fastest within a group so that a wave's stores of
// one period are contiguous.
template <typename T, int LPR, int PT, bool BZ>
__global__ __launch_bounds__(256) void bbm_periodic_spmv_kernel(int32_t nT, int32_t n_diag, int32_t period,
                                                                int64_t items, int64_t n_cols, PBlk D, PBlk N,
                                                                PBlk Pb, T alpha, const T *__restrict__ x, T beta,
                                                                T *__restrict__ y)
{
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t item = g / LPR;
    const int sub = (int)(g % LPR);
    const bool live = item < items;
    const uint32_t it = live ? (uint32_t)item : (uint32_t)(items - 1);   // clamped: loads stay in bounds
    const uint32_t grp = it / (uint32_t)period;
    const int32_t i = (int32_t)(it - grp * (uint32_t)period);
    const int32_t t0 = (int32_t)grp * PT;
    const bool diag = i < n_diag;
    // Periods this item writes: every period for a diagonal row, those with
    // a successor for a coupling row.
    const int32_t nper = min(PT, (diag ? nT : nT - 1) - t0);
    int64_t xo[PT];
    T acc[PT];
#pragma unroll
    for (int q = 0; q < PT; ++q) {
        xo[q] = (int64_t)min(t0 + q, nT - 1) * n_cols;
        acc[q] = T(0);
    }
    if (diag) {
        row_walk<T, LPR, PT>(D, i, x, xo, sub, acc);
    } else {
        row_walk<T, LPR, PT>(N, i - n_diag, x, xo, sub, acc);
#pragma unroll
        for (int q = 0; q < PT; ++q) xo[q] = (int64_t)min(t0 + q + 1, nT - 1) * n_cols;
        row_walk<T, LPR, PT>(Pb, i - n_diag, x, xo, sub, acc);
    }
#pragma unroll
    for (int q = 0; q < PT; ++q)
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) acc[q] += __shfl_xor(acc[q], off, LPR);
    if (sub == 0 && live) {
#pragma unroll
        for (int q = 0; q < PT; ++q) {
            if (q < nper) {
                T *yr = y + (int64_t)(t0 + q) * period + i;
                *yr = BZ ? alpha * acc[q] : alpha * acc[q] + beta * *yr;
            }
        }
    }
}

// Block descriptor from a placement (its block, or its shifted diagonal);
// expects an m x n block.
int to_blk(const jlust_placement *pl, const char *which, int64_t m, int64_t n, PBlk &b)
{
    b = PBlk{};
    if (!pl) return fail(JLUST_STATUS_INVALID_ARGUMENT, "bbm_periodic_spmv: null %s block", which);
    const jlust_sparse *s = pl->block;
    int64_t bm, bn;
    if (!s) {
        bm = pl->diag_m;
        bn = pl->diag_n;
        b.kind = 1;
        b.shift = pl->diag_shift;
        b.dval = pl->diag_val;
        if (b.shift > INT32_MAX || b.shift < -(int64_t)INT32_MAX)
            return fail(JLUST_STATUS_INVALID_ARGUMENT, "bbm_periodic_spmv: %s shift out of range", which);
    } else {
        if (s->format != JLUST_FORMAT_CSR)
            return fail(JLUST_STATUS_UNSUPPORTED_FORMAT,
                        "bbm_periodic_spmv: the %s block must be CSR or a shifted diagonal (format %d)", which,
                        s->format);
        if (int st = check_origin(s->origin)) return st;
        bm = s->m;
        bn = s->n;
        if (s->nnz < 0 || s->nnz > INT32_MAX)
            return fail(JLUST_STATUS_INVALID_ARGUMENT, "bbm_periodic_spmv: %s block nnz out of range", which);
        if (!s->pos2 || bad_ptr(s->crd2, s->nnz) || bad_ptr(s->val, s->nnz))
            return fail(JLUST_STATUS_INVALID_ARGUMENT, "bbm_periodic_spmv: null %s block buffer", which);
        b.kind = 0;
        b.rowptr = s->pos2;
        b.colind = s->crd2;
        b.val = s->val;
        b.origin = s->origin;
    }
    if (bm != m || bn != n)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bbm_periodic_spmv: %s block is %lld x %lld, expected %lld x %lld",
                    which, (long long)bm, (long long)bn, (long long)m, (long long)n);
    b.n = bn;
    return JLUST_STATUS_SUCCESS;
}

template <typename T>
int bbm_periodic(int64_t T_, int64_t nd, int64_t no, int64_t nc, const jlust_placement *diag,
                 const jlust_placement *neg, const jlust_placement *pos, T alpha, const T *x, T beta, T *y,
                 hipStream_t s)
{
    clear_error();
    if (T_ < 1 || nd < 0 || no < 0 || nc < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bbm_periodic_spmv: T=%lld, n_diag_rows=%lld, n_off_rows=%lld, "
                    "n_cols=%lld", (long long)T_, (long long)nd, (long long)no, (long long)nc);
    if (T_ == 1) no = 0;                     // no transitions, no coupling rows
    // Row indices, and the period and row within it, are 32-bit in the kernel.
    if (T_ > INT32_MAX || nd > INT32_MAX || no > INT32_MAX || nc > INT32_MAX ||
        T_ * nd + (T_ - 1) * no > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bbm_periodic_spmv: matrix too large for 32-bit rows");
    const int64_t period = nd + no;
    const int64_t rows = T_ * nd + (T_ - 1) * no;
    PBlk D, N{}, P{};
    if (int st = to_blk(diag, "diagonal", nd, nc, D)) return st;
    if (no > 0) {
        if (int st = to_blk(neg, "neg", no, nc, N)) return st;
        if (int st = to_blk(pos, "pos", no, nc, P)) return st;
    } else {
        N = D;                               // never read: every row is a diagonal row
        P = D;
    }
    if (bad_ptr(x, T_ * nc) || bad_ptr(y, rows))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bbm_periodic_spmv: null vector");
    if (rows == 0) return JLUST_STATUS_SUCCESS;
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    // Lanes per row: about 4 entries per lane of the diagonal block's mean
    // row, at least 2.  Periods per item: the most of 4 and 2 that still gives
    // about 4 waves per SIMD (more periods per lane measured slower).
    const double avg = D.kind == 1 || nd == 0 ? 1.0 : (double)diag->block->nnz / (double)nd;
    int lpr = 2;
    while (lpr < 64 && 4 * lpr < avg) lpr <<= 1;
    int pt = 4;
    while (pt > 1 && ((T_ + pt - 1) / pt) * period * lpr < ((int64_t)256 * 4 * 64 * 4)) pt >>= 1;
    if (const char *e = getenv("JLUST_HIP_BBM_LANES")) {
        const int f = atoi(e);
        if (f >= 1 && f <= 64 && (f & (f - 1)) == 0) lpr = f;
    }
    if (const char *e = getenv("JLUST_HIP_BBM_PERIODS")) {
        const int f = atoi(e);
        if (f == 1 || f == 2 || f == 4 || f == 8) pt = f;
    }
    const int64_t items = ((T_ + pt - 1) / pt) * period;
    const int64_t threads = items * lpr;
    const dim3 grid((unsigned)((threads + 255) / 256));
#define K(LP, PTV)                                                                                       \
    do {                                                                                                 \
        if (beta == T(0))                                                                                \
            hipLaunchKernelGGL((bbm_periodic_spmv_kernel<T, LP, PTV, true>), grid, dim3(256), 0, s,      \
                               (int32_t)T_, (int32_t)nd, (int32_t)period, items, nc, D, N, P, alpha, x,  \
                               beta, y);                                                                 \
        else                                                                                             \
            hipLaunchKernelGGL((bbm_periodic_spmv_kernel<T, LP, PTV, false>), grid, dim3(256), 0, s,     \
                               (int32_t)T_, (int32_t)nd, (int32_t)period, items, nc, D, N, P, alpha, x,  \
                               beta, y);                                                                 \
    } while (0)
#define L(LP)                                                                                            \
    do {                                                                                                 \
        switch (pt) {                                                                                    \
        case 8: K(LP, 8); break;                                                                         \
        case 4: K(LP, 4); break;                                                                         \
        case 2: K(LP, 2); break;                                                                         \
        default: K(LP, 1); break;                                                                        \
        }                                                                                                \
    } while (0)
    switch (lpr) {
    case 1: L(1); break;
    case 2: L(2); break;
    case 4: L(4); break;
    case 8: L(8); break;
    case 16: L(16); break;
    case 32: L(32); break;
    default: L(64); break;
    }
#undef L
#undef K
    return check_launch("bbm_periodic_spmv_kernel");
}

}  // namespace
}  // namespace jlust

using namespace jlust;

extern "C" int jlust_hip_bbm_periodic_spmv_f64(int64_t T, int64_t n_diag_rows, int64_t n_off_rows, int64_t n_cols,
                                               const jlust_placement *diag, const jlust_placement *neg,
                                               const jlust_placement *pos, double alpha, const double *x,
                                               double beta, double *y, jlust_stream_t stream)
{
    return bbm_periodic<double>(T, n_diag_rows, n_off_rows, n_cols, diag, neg, pos, alpha, x, beta, y,
                                (hipStream_t)stream);
}

extern "C" int jlust_hip_bbm_periodic_spmv_f32(int64_t T, int64_t n_diag_rows, int64_t n_off_rows, int64_t n_cols,
                                               const jlust_placement *diag, const jlust_placement *neg,
                                               const jlust_placement *pos, float alpha, const float *x,
                                               float beta, float *y, jlust_stream_t stream)
{
    return bbm_periodic<float>(T, n_diag_rows, n_off_rows, n_cols, diag, neg, pos, alpha, x, beta, y,
                               (hipStream_t)stream);
}

namespace jlust {
int preload_periodic()
{
    JLUST_PRELOAD_KERNEL((bbm_periodic_spmv_kernel<double, 2, 4, true>));
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
