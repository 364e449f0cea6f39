// spmm.hip -- CSR SpMM C = alpha*A*B + beta*C for gfx950 (wave64).
//
// Replaces execute(::EmitterBackend, ::Op{:SpMM}, ...)
// (ext/KernelAbstractionsExt/ops/spmm.jl:397-423).  Per output the reference
// sums val[k]*B[col[k], c] sequentially over the row and writes
// alpha*acc + beta*C (spmm.jl:272-279 for the Tiled strategy used at k > 32).
//
// B and C are column-major (Julia layout).  Gathering a row B[j, :] straight
// from column-major B touches k cache lines 4*ldb bytes apart for k useful
// values, so the kernel first re-lays B out row-major (Bt, n x ldt) in the
// library's scratch buffer with an LDS-tiled transpose: one coalesced read
// and one coalesced write of B.  Then:
//   - a block owns SPMM_ROWS consecutive rows; each wave walks one row at a
//     time, its 64 lanes covering a 64*VEC-column chunk (VEC consecutive
//     columns per lane, one vector load per lane per nonzero, so one nonzero
//     reads a contiguous 64*VEC*sizeof(T)-byte slice of Bt);
//   - the row's col/val are read 64 at a time with one coalesced load and
//     broadcast lane by lane (v_readlane), several B slices in flight;
//   - results are staged in LDS and written to column-major C column by
//     column (SPMM_ROWS consecutive values per column), so C writes are
//     coalesced too.
#include "common.hpp"

#include <cstdlib>
#include <memory>
#include <vector>

namespace jlust {
namespace {

constexpr int SPMM_BLOCK = 256;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
constexpr int SPMM_ROWS = 32;
constexpr int SPMM_UNROLL = 8;

template <typename T>
__device__ __forceinline__ T bcast(T v, int lane);
template <>
__device__ __forceinline__ float bcast<float>(float v, int lane)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
template <>
__device__ __forceinline__ double bcast<double>(double v, int lane)
{
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), lane);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ __forceinline__ int bcast_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

template <typename T, int VEC> struct Vec;
template <typename T> struct Vec<T, 1> { T v[1]; };
template <typename T> struct alignas(2 * sizeof(T)) Vec<T, 2> { T v[2]; };
template <typename T> struct alignas(4 * sizeof(T)) Vec<T, 4> { T v[4]; };

// Bt[j*ldt + c] = B[j + c*ldb] for j < n, c < k (64 x 64 tiles through LDS).
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(int64_t n, int64_t k,
                                                        const T *__restrict__ B, int64_t ldb,
                                                        T *__restrict__ Bt, int64_t ldt)
{
    __shared__ T tile[64][65];
    const int tx = threadIdx.x & 63;
    const int ty = threadIdx.x >> 6;
    const int64_t j0 = (int64_t)blockIdx.x * 64;
    const int64_t c0 = (int64_t)blockIdx.y * 64;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const int cc = ty + 4 * s;
        const int64_t j = j0 + tx, c = c0 + cc;
        if (j < n && c < k) tile[cc][tx] = B[j + c * ldb];
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const int jj = ty + 4 * s;
        const int64_t j = j0 + jj, c = c0 + tx;
        if (j < n && c < k) Bt[j * ldt + c] = tile[tx][jj];
    }
}

// Chunks of at most 32 columns: groups of KV lanes (KV the smallest power of
// two >= the chunk's columns), one nonzero per group per step, so a wave
// takes 64/KV nonzeros per step (64 at k = 1, where the kernel is a
// wave-per-row SpMV).  Each lane loads its group's col/val itself (the
// group's lanes read one address), gathers its column of the nonzero's Bt
// row, and keeps its group's sum in nonzero order; the groups' sums are added
// with xor-shuffles at the row's end.  U steps are loaded at once (indices
// clamped into the row, products of the clamped copies dropped by a select;
// U is chosen per call from the mean row length, so a short row issues no
// clamped copies), and the next row's pointers are loaded before the current
// row's nonzeros, so a wave's rows do not wait on each other's pointer loads.
template <typename T, int KV, int U>
__global__ __launch_bounds__(SPMM_BLOCK) void csr_spmm_group_kernel(
    int64_t m, int64_t k, int32_t origin, const int32_t *__restrict__ rowptr,
    const int32_t *__restrict__ colind, const T *__restrict__ val, const T *__restrict__ Bt,
    int64_t ldt, T alpha, T beta, int beta_zero, T *__restrict__ C, int64_t ldc,
    int skip_empty_rows, const int32_t *__restrict__ rowend, const uint8_t *__restrict__ row_skip)
{
    constexpr int G = 64 / KV;                 // nonzeros per step
    constexpr int NW = SPMM_BLOCK / 64;
    __shared__ T s_c[SPMM_ROWS][KV + 1];
    __shared__ int s_empty[SPMM_ROWS];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int grp = lane / KV;
    const int col = lane % KV;
    const int64_t row0 = (int64_t)blockIdx.x * SPMM_ROWS;
    const int nrows = (int)min((int64_t)SPMM_ROWS, m - row0);
    const int64_t cl = col < k ? col : 0;      // clamped, in-bounds column

    int32_t lo_n = 0, hi_n = 0;
    if (wave < nrows) {
        lo_n = rowptr[row0 + wave];
        hi_n = rowend ? rowend[row0 + wave] : rowptr[row0 + wave + 1];
    }
    for (int rr = wave; rr < nrows; rr += NW) {
        const int64_t lo = (int64_t)lo_n - origin;
        int64_t hi = (int64_t)hi_n - origin;
        if (rr + NW < nrows) {                 // the wave's next row
            lo_n = rowptr[row0 + rr + NW];
            hi_n = rowend ? rowend[row0 + rr + NW] : rowptr[row0 + rr + NW + 1];
        }
        const bool skip = row_skip && row_skip[row0 + rr];
        if (skip) hi = lo;                     // a split row: its segments compute it
        if (lane == 0) s_empty[rr] = skip ? 2 : hi <= lo;
        T acc = T(0);
        for (int64_t p0 = lo + grp; p0 < hi; p0 += (int64_t)G * U) {
            int32_t c[U];
            T a[U], b[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t p = min(p0 + (int64_t)u * G, hi - 1);
                c[u] = colind[p];
                a[u] = val[p];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) b[u] = Bt[(int64_t)(c[u] - origin) * ldt + cl];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const T s = acc + a[u] * b[u];
                acc = p0 + (int64_t)u * G < hi ? s : acc;
            }
        }
#pragma unroll
        for (int off = KV; off < 64; off <<= 1) acc += __shfl_xor(acc, off, 64);
        if (lane < KV) s_c[rr][col] = acc;
    }
    __syncthreads();
    const int ncols = (int)k;                  // k <= KV here
    for (int idx = tid; idx < SPMM_ROWS * ncols; idx += SPMM_BLOCK) {
        const int rr = idx % SPMM_ROWS;
        const int cc = idx / SPMM_ROWS;
        if (rr >= nrows) continue;
        if (s_empty[rr] == 2 || (skip_empty_rows && s_empty[rr])) continue;
        T *dst = C + (row0 + rr) + cc * ldc;
        const T s = alpha * s_c[rr][cc];
        *dst = beta_zero ? s : s + beta * *dst;
    }
}

template <typename T, int VEC>
__global__ __launch_bounds__(SPMM_BLOCK) void csr_spmm_kernel(
    int64_t m, int64_t k, int32_t origin, const int32_t *__restrict__ rowptr,
    const int32_t *__restrict__ colind, const T *__restrict__ val, const T *__restrict__ Bt,
    int64_t ldt, T alpha, T beta, int beta_zero, T *__restrict__ C, int64_t ldc,
    int skip_empty_rows, const int32_t *__restrict__ rowend, const uint8_t *__restrict__ row_skip)
{
    constexpr int KC = 64 * VEC;              // columns per chunk
    constexpr int NW = SPMM_BLOCK / 64;
    __shared__ T s_c[SPMM_ROWS][KC + 1];
    __shared__ int s_empty[SPMM_ROWS];
    using V = Vec<T, VEC>;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t row0 = (int64_t)blockIdx.x * SPMM_ROWS;
    const int nrows = (int)min((int64_t)SPMM_ROWS, m - row0);

    for (int64_t c0 = 0; c0 < k; c0 += KC) {
        const int64_t cl = c0 + (int64_t)lane * VEC;     // first column of this lane
        const bool full = cl + VEC <= k;
        for (int rr = wave; rr < nrows; rr += NW) {
            const int64_t row = row0 + rr;
            const int64_t lo = (int64_t)rowptr[row] - origin;
            int64_t hi = (int64_t)(rowend ? rowend[row] : rowptr[row + 1]) - origin;
            const bool skip = row_skip && row_skip[row];
            if (skip) hi = lo;                 // a split row: its segments compute it
            if (lane == 0 && c0 == 0) s_empty[rr] = skip ? 2 : hi <= lo;
            T acc[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[e] = T(0);
            for (int64_t p0 = lo; p0 < hi; p0 += 64) {
                const int cnt = (int)min((int64_t)64, hi - p0);
                int cidx = 0;
                T cv = T(0);
                if (lane < cnt) {
                    cidx = colind[p0 + lane] - origin;
                    cv = val[p0 + lane];
                }
                int q = 0;
                for (; q + SPMM_UNROLL <= cnt; q += SPMM_UNROLL) {
                    V b[SPMM_UNROLL];
                    T a[SPMM_UNROLL];
#pragma unroll
                    for (int u = 0; u < SPMM_UNROLL; ++u) {
                        const int64_t j = bcast_i(cidx, q + u);
                        a[u] = bcast(cv, q + u);
                        if (full) {
                            b[u] = *reinterpret_cast<const V *>(Bt + j * ldt + cl);
                        } else {
#pragma unroll
                            for (int e = 0; e < VEC; ++e)
                                b[u].v[e] = cl + e < k ? Bt[j * ldt + cl + e] : T(0);
                        }
                    }
#pragma unroll
                    for (int u = 0; u < SPMM_UNROLL; ++u)
#pragma unroll
                        for (int e = 0; e < VEC; ++e) acc[e] += a[u] * b[u].v[e];
                }
                for (; q < cnt; ++q) {
                    const int64_t j = bcast_i(cidx, q);
                    const T a = bcast(cv, q);
#pragma unroll
                    for (int e = 0; e < VEC; ++e)
                        if (cl + e < k) acc[e] += a * Bt[j * ldt + cl + e];
                }
            }
#pragma unroll
            for (int e = 0; e < VEC; ++e) s_c[rr][lane * VEC + e] = acc[e];
        }
        __syncthreads();
        // Column-major write-out: SPMM_ROWS consecutive rows per column.
        const int ncols = (int)min((int64_t)KC, k - c0);
        for (int idx = tid; idx < SPMM_ROWS * ncols; idx += SPMM_BLOCK) {
            const int rr = idx % SPMM_ROWS;
            const int cc = idx / SPMM_ROWS;
            if (rr >= nrows) continue;
            if (s_empty[rr] == 2 || (skip_empty_rows && s_empty[rr])) continue;
            T *dst = C + (row0 + rr) + (c0 + cc) * ldc;
            const T s = alpha * s_c[rr][cc];
            *dst = beta_zero ? s : s + beta * *dst;
        }
        __syncthreads();
    }
}

// Columns per pass: all of k while the row-major copy of B fits a budget of
// the 256 MB MALL, else the widest multiple of 16 columns that does (at least
// 16).  JLUST_HIP_SPMM_KCHUNK=c forces c columns per pass.
constexpr size_t SPMM_MALL_BUDGET = (size_t)256 << 20;

bool spmm_group()
{
    static const bool on = [] {
        const char *e = getenv("JLUST_HIP_SPMM_GROUP");
        return !(e && e[0] == '0');
    }();
    return on;
}

int64_t spmm_kchunk(int64_t n, int64_t k, size_t tsz)
{
    static const int64_t forced = [] {
        const char *e = getenv("JLUST_HIP_SPMM_KCHUNK");
        return e ? (int64_t)atoll(e) : (int64_t)0;
    }();
    if (forced > 0) return forced < k ? forced : k;
    const size_t row = (size_t)(n > 0 ? n : 1) * tsz;
    if ((size_t)k * row <= SPMM_MALL_BUDGET) return k;
    int64_t kc = (int64_t)(SPMM_MALL_BUDGET / row) / 16 * 16;
    if (kc < 16) kc = 16;
    return kc < k ? kc : k;
}

// Long rows of a prepared plan: a row with more than SPMM_LONG_ROW entries
// is cut into segments of SPMM_SEG entries, each a wave's work in the same
// kernels (rowptr = segment starts, rowend = segment ends) writing one partial
// row into the plan's workspace; spmm_long_reduce_kernel adds a row's
// partials in segment order.  A wave otherwise walks a whole row alone, so a
// 10^5-entry row of a power-law matrix would keep one wave busy for the whole
// product.
constexpr int64_t SPMM_LONG_ROW = 1024;
constexpr int64_t SPMM_SEG = 256;

// C[r, c] = alpha * sum_s part[s, c] + beta * C[r, c] for the long rows:
// one thread per (long row, column), partials of the row's segments
// [seg_first[l], seg_first[l+1]) added in segment order.
template <typename T>
__global__ void spmm_long_reduce_kernel(int64_t nlong, int64_t kk, const int32_t *__restrict__ long_rows,
                                        const int32_t *__restrict__ seg_first, const T *__restrict__ part,
                                        int64_t ldp, T alpha, T beta, int beta_zero, T *__restrict__ C,
                                        int64_t ldc)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nlong * kk) return;
    const int64_t l = t % nlong, c = t / nlong;
    const int32_t s0 = seg_first[l], s1 = seg_first[l + 1];
    T acc = part[s0 + c * ldp];
    for (int32_t q = s0 + 1; q < s1; ++q) acc += part[q + c * ldp];
    T *dst = C + long_rows[l] + c * ldc;
    const T v = alpha * acc;
    *dst = beta_zero ? v : v + beta * *dst;
}

// How one column chunk of kk columns is computed: the group kernel (kk <= 32)
// or the wide kernel; the group kernel's B copy is unpadded, the wide one's
// rows padded to 16 bytes; one column gathers from B's own column.
struct SpmmChunk {
    bool group;
    bool direct;
    int64_t ldt;
};

SpmmChunk spmm_chunk_kind(int64_t kk)
{
    SpmmChunk c;
    c.group = kk <= 32 && spmm_group();
    c.direct = c.group && kk == 1;
    c.ldt = c.group ? kk : (kk + 3) / 4 * 4;
    return c;
}

// Row-major copy of columns [c0, c0+kk) of B into Bt (skipped when direct).
template <typename T>
int spmm_copy_chunk(int64_t n, int64_t kk, const T *B, int64_t ldb, const SpmmChunk &ck, T *Bt, hipStream_t s)
{
    if (n == 0 || ck.direct) return JLUST_STATUS_SUCCESS;
    dim3 tgrid((unsigned)((n + 63) / 64), (unsigned)((kk + 63) / 64));
    hipLaunchKernelGGL((transpose_kernel<T>), tgrid, dim3(256), 0, s, n, kk, B, ldb, Bt, ck.ldt);
    return check_launch("transpose_kernel");
}

// The product of one chunk over m rows (rows of A, or segments when rowend is
// given): C[:, 0:kk] (ldc) = alpha * A[rows, :] * Bsrc + beta * C, rows
// flagged in row_skip left untouched.  nnz_rows: the entries these rows hold
// (for the group kernel's steps per load).
template <typename T>
int spmm_chunk_launch(int64_t m, int64_t kk, int64_t nnz_rows, int32_t origin, const int32_t *rowptr,
                      const int32_t *rowend, const uint8_t *row_skip, const int32_t *colind, const T *val,
                      const T *Bsrc, const SpmmChunk &ck, T alpha, T beta, T *Cc, int64_t ldc,
                      int skip_empty_rows, hipStream_t s)
{
    if (m == 0) return JLUST_STATUS_SUCCESS;
    const dim3 grid((unsigned)((m + SPMM_ROWS - 1) / SPMM_ROWS));
    const int bz = beta == T(0);
    const int64_t ldt = ck.ldt;
    const int vec = (sizeof(T) == 4) ? (kk <= 64 ? 1 : kk <= 128 ? 2 : 4) : (kk <= 64 ? 1 : 2);
#define JLUST_GROUP_U(KV, U)                                                                           \
    hipLaunchKernelGGL((csr_spmm_group_kernel<T, KV, U>), grid, dim3(SPMM_BLOCK), 0, s, m, kk, origin,    \
                       rowptr, colind, val, Bsrc, ldt, alpha, beta, bz, Cc, ldc, skip_empty_rows, rowend, \
                       row_skip)
#define JLUST_GROUP(KV)                                                                                \
    do {                                                                                               \
        const int64_t steps = (nnz_rows + m * (64 / KV) - 1) / (m * (64 / KV));  /* per row */          \
        if (steps <= 1) JLUST_GROUP_U(KV, 1);                                                          \
        else if (steps <= 2) JLUST_GROUP_U(KV, 2);                                                     \
        else if (steps <= 4) JLUST_GROUP_U(KV, 4);                                                     \
        else JLUST_GROUP_U(KV, 8);                                                                     \
    } while (0)
#define JLUST_WIDE(V)                                                                                  \
    hipLaunchKernelGGL((csr_spmm_kernel<T, V>), grid, dim3(SPMM_BLOCK), 0, s, m, kk, origin, rowptr,      \
                       colind, val, Bsrc, ldt, alpha, beta, bz, Cc, ldc, skip_empty_rows, rowend, row_skip)
    if (ck.group) {
        if (kk == 1) JLUST_GROUP(1);
        else if (kk == 2) JLUST_GROUP(2);
        else if (kk <= 4) JLUST_GROUP(4);
        else if (kk <= 8) JLUST_GROUP(8);
        else if (kk <= 16) JLUST_GROUP(16);
        else JLUST_GROUP(32);
    } else if (vec == 1) {
        JLUST_WIDE(1);
    } else if (vec == 2) {
        JLUST_WIDE(2);
    } else {
        JLUST_WIDE(4);
    }
#undef JLUST_WIDE
#undef JLUST_GROUP
#undef JLUST_GROUP_U
    return check_launch(ck.group ? "csr_spmm_group_kernel" : "csr_spmm_kernel");
}

int check_spmm_args(const char *who, int64_t m, int64_t n, int64_t k, int64_t nnz, int32_t origin,
                    const void *rowptr, const void *colind, const void *val)
{
    if (m < 0 || n < 0 || k < 0 || nnz < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: negative extent", who);
    if (m > INT32_MAX - 1 || n > INT32_MAX || nnz > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: extents exceed the Int32 index range", who);
    if (int st = check_origin(origin)) return st;
    if ((m > 0 && !rowptr) || bad_ptr(colind, nnz) || bad_ptr(val, nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: null device pointer", who);
    if (nnz > 0 && n == 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: nnz > 0 with n == 0", who);
    return JLUST_STATUS_SUCCESS;
}

int check_dense_args(const char *who, int64_t m, int64_t n, int64_t k, int64_t nnz, const void *B, int64_t ldb,
                     const void *C, int64_t ldc)
{
    if (ldb < (n > 0 ? n : 1) || ldc < (m > 0 ? m : 1))
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "%s: leading dimensions too small (ldb=%lld < n=%lld or ldc=%lld < m=%lld)", who,
                    (long long)ldb, (long long)n, (long long)ldc, (long long)m);
    if (bad_ptr(B, (nnz > 0 && k > 0) ? n : 0) || bad_ptr(C, m * k))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: null device pointer", who);
    return JLUST_STATUS_SUCCESS;
}

template <typename T>
int csr_spmm(int64_t m, int64_t n, int64_t k, int64_t nnz, int32_t origin,
             const int32_t *rowptr, const int32_t *colind, const T *val, T alpha, const T *B,
             int64_t ldb, T beta, T *C, int64_t ldc, int skip_empty_rows, jlust_stream_t stream)
{
    clear_error();
    if (int st = check_spmm_args("csr_spmm", m, n, k, nnz, origin, rowptr, colind, val)) return st;
    if (int st = check_dense_args("csr_spmm", m, n, k, nnz, B, ldb, C, ldc)) return st;
    if (int st = require_device(nullptr)) return st;
    if (m == 0 || k == 0) return JLUST_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;

    // Column chunks: every B row a nonzero gathers is a random row of the
    // row-major copy; when that copy is larger than the MALL budget the
    // gathers come from HBM, so B is processed in column chunks whose copy
    // fits (config 3: 2 chunks of 64 columns, 3.14 -> 2.56 ms).
    const int64_t kc = spmm_kchunk(n, k, sizeof(T));
    const int64_t ldt_max = (min(kc, k) + 3) / 4 * 4;    // keeps every row of Bt 16-byte aligned
    void *ws = nullptr;
    const int64_t nt = n > 0 ? n : 1;
    if (int st = scratch(stream, sizeof(T) * (size_t)(nt * ldt_max), &ws)) return st;
    T *Bt = (T *)ws;
    for (int64_t c0 = 0; c0 < k; c0 += kc) {
        const int64_t kk = min(kc, k - c0);
        const SpmmChunk ck = spmm_chunk_kind(kk);
        if (int st = spmm_copy_chunk<T>(n, kk, B + c0 * ldb, ldb, ck, Bt, s)) return st;
        const T *Bsrc = ck.direct ? B + c0 * ldb : Bt;
        if (int st = spmm_chunk_launch<T>(m, kk, nnz, origin, rowptr, nullptr, nullptr, colind, val, Bsrc, ck,
                                          alpha, beta, C + c0 * ldc, ldc, skip_empty_rows, s))
            return st;
    }
    return JLUST_STATUS_SUCCESS;
}

}  // namespace
}  // namespace jlust

using namespace jlust;

extern "C" int jlust_hip_csr_spmm_f64_i32(int64_t m, int64_t n, int64_t k, int64_t nnz,
                                          int32_t origin, const int32_t *rowptr,
                                          const int32_t *colind, const double *val, double alpha,
                                          const double *B, int64_t ldb, double beta, double *C,
                                          int64_t ldc, int skip_empty_rows, jlust_stream_t stream)
{
    return csr_spmm<double>(m, n, k, nnz, origin, rowptr, colind, val, alpha, B, ldb, beta, C,
                            ldc, skip_empty_rows, stream);
}

extern "C" int jlust_hip_csr_spmm_f32_i32(int64_t m, int64_t n, int64_t k, int64_t nnz,
                                          int32_t origin, const int32_t *rowptr,
                                          const int32_t *colind, const float *val, float alpha,
                                          const float *B, int64_t ldb, float beta, float *C,
                                          int64_t ldc, int skip_empty_rows, jlust_stream_t stream)
{
    return csr_spmm<float>(m, n, k, nnz, origin, rowptr, colind, val, alpha, B, ldb, beta, C,
                           ldc, skip_empty_rows, stream);
}

// ------------------------------------------------------------------- plans

// A prepared CSR SpMM (the cuSPARSE SpMM handle contract: analysis and
// workspace once, execute many times, update_values! for new values of the
// same pattern; ext/CUDAExt/ops/spmm.jl:8-70).  Analysis: the column chunk
// per pass for the plan's k; the rows longer than SPMM_LONG_ROW, cut into
// segments; the entries left to the row kernels (for their steps per load).
// Workspace: the row-major copy of one column chunk of B and the segments'
// partial rows, so an execute allocates nothing and can be captured.
struct jlust_spmm_plan {
    int64_t m = 0, n = 0, k = 0, nnz = 0;
    int32_t origin = 0;
    int value_type = 0;
    const int32_t *rowptr = nullptr;
    const int32_t *colind = nullptr;
    const void *val = nullptr;
    int device = 0;
    int64_t kc = 1;                 // columns per pass
    void *mem = nullptr;            // one allocation holds everything below
    void *Bt = nullptr;             // n x ldt row-major copy of one column chunk of B
    uint8_t *row_skip = nullptr;    // [m] 1 for a split row (null: none)
    int64_t nlong = 0, nseg = 0;
    int32_t *long_rows = nullptr;   // [nlong] the split rows
    int32_t *seg_first = nullptr;   // [nlong + 1] first segment of each split row
    int32_t *seg_lo = nullptr;      // [nseg] segment start (origin-based, like rowptr)
    int32_t *seg_hi = nullptr;      // [nseg] segment end
    void *part = nullptr;           // nseg x kc partial rows, column-major (ld nseg)
    int64_t nnz_rows = 0;           // entries of the rows that are not split
    // COO/CSC plans (coo_csc.hip): the row order the plan runs on is owned in
    // own_mem; perm (null when the source was already in row order) maps its
    // entries to the caller's, and val_copy holds the values in that order.
    void *own_mem = nullptr;
    const int32_t *perm = nullptr;
    void *val_copy = nullptr;
};

namespace jlust {
int spmm_plan_adopt_reorder(jlust_spmm_plan_t plan, void *mem, const int32_t *perm, void *val_copy)
{
    plan->own_mem = mem;
    plan->perm = perm;
    plan->val_copy = val_copy;
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust

static int csr_spmm_plan_create_body(int64_t m, int64_t n, int64_t k, int64_t nnz, int32_t origin,
                                     int value_type, const int32_t *rowptr, const int32_t *colind,
                                     const void *val, jlust_stream_t stream,
                                     jlust_spmm_plan_t *plan_out)
{
    clear_error();
    if (!plan_out) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmm_plan_create: null plan_out");
    *plan_out = nullptr;
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE,
                    "spmm_plan_create: value_type %d (0 = Float64, 1 = Float32)", value_type);
    if (int st = check_spmm_args("spmm_plan_create", m, n, k, nnz, origin, rowptr, colind, val)) return st;
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    hipStream_t s = (hipStream_t)stream;
    const size_t tsz = value_type == 0 ? sizeof(double) : sizeof(float);
    std::unique_ptr<jlust_spmm_plan> p(new jlust_spmm_plan());
    p->m = m;
    p->n = n;
    p->k = k;
    p->nnz = nnz;
    p->origin = origin;
    p->value_type = value_type;
    p->rowptr = rowptr;
    p->colind = colind;
    p->val = val;
    p->device = dev;
    p->kc = k > 0 ? spmm_kchunk(n, k, tsz) : 1;
    p->nnz_rows = nnz;

    // Row analysis on the host copy of rowptr: which rows to split.
    std::vector<int32_t> rp((size_t)(m + 1));
    if (m > 0) {
        JLUST_HIP_TRY(hipMemcpyAsync(rp.data(), rowptr, sizeof(int32_t) * (size_t)(m + 1), hipMemcpyDeviceToHost, s));
        JLUST_HIP_TRY(hipStreamSynchronize(s));
        if ((int64_t)rp[0] != origin || (int64_t)rp[m] - origin != nnz)
            return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                        "spmm_plan_create: rowptr runs from %d to %d, expected %d to %lld", rp[0], rp[m], origin,
                        (long long)(nnz + origin));
    }
    std::vector<int32_t> long_rows, seg_first, seg_lo, seg_hi;
    for (int64_t i = 0; i < m; ++i) {
        const int64_t len = (int64_t)rp[i + 1] - rp[i];
        if (len < 0)
            return fail(JLUST_STATUS_NONCANONICAL_STORAGE, "spmm_plan_create: rowptr decreases at row %lld",
                        (long long)i);
        if (len <= SPMM_LONG_ROW) continue;
        long_rows.push_back((int32_t)i);
        seg_first.push_back((int32_t)seg_lo.size());
        for (int64_t a = rp[i]; a < rp[i + 1]; a += SPMM_SEG) {
            seg_lo.push_back((int32_t)a);
            seg_hi.push_back((int32_t)min(a + SPMM_SEG, (int64_t)rp[i + 1]));
        }
        p->nnz_rows -= len;
    }
    seg_first.push_back((int32_t)seg_lo.size());
    p->nlong = (int64_t)long_rows.size();
    p->nseg = (int64_t)seg_lo.size();
    std::vector<uint8_t> skip(p->nlong ? (size_t)m : 0, 0);   // host tables before the device allocation
    for (int32_t r : long_rows) skip[(size_t)r] = 1;

    // One allocation: B copy, row flags, segment tables, partial rows.
    const int64_t ldt_max = (min(p->kc, k > 0 ? k : 1) + 3) / 4 * 4;
    const size_t sz_bt = align_up(tsz * (size_t)(n > 0 ? n : 1) * (size_t)ldt_max, 256);
    const size_t sz_skip = p->nlong ? align_up((size_t)m, 256) : 0;
    const size_t sz_lr = align_up(sizeof(int32_t) * (size_t)(p->nlong + 1), 256);
    const size_t sz_sg = align_up(sizeof(int32_t) * (size_t)(p->nseg > 0 ? p->nseg : 1), 256);
    const size_t sz_part = p->nseg ? align_up(tsz * (size_t)p->nseg * (size_t)p->kc, 256) : 0;
    JLUST_HIP_TRY(hipMalloc(&p->mem, sz_bt + sz_skip + 2 * sz_lr + 2 * sz_sg + sz_part));
    char *b = (char *)p->mem;
    p->Bt = b;                           b += sz_bt;
    if (p->nlong) { p->row_skip = (uint8_t *)b; b += sz_skip; }
    p->long_rows = (int32_t *)b;         b += sz_lr;
    p->seg_first = (int32_t *)b;         b += sz_lr;
    p->seg_lo = (int32_t *)b;            b += sz_sg;
    p->seg_hi = (int32_t *)b;            b += sz_sg;
    if (p->nseg) p->part = b;
    int st = JLUST_STATUS_SUCCESS;
    if (p->nlong) {
        hipError_t e = hipMemcpyAsync(p->row_skip, skip.data(), (size_t)m, hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync(p->long_rows, long_rows.data(), sizeof(int32_t) * long_rows.size(),
                               hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync(p->seg_first, seg_first.data(), sizeof(int32_t) * seg_first.size(),
                               hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync(p->seg_lo, seg_lo.data(), sizeof(int32_t) * seg_lo.size(), hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync(p->seg_hi, seg_hi.data(), sizeof(int32_t) * seg_hi.size(), hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);   // the host tables go out of scope
        if (e != hipSuccess) st = hip_fail(e, "spmm_plan_create: table upload");
    }
    if (st) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(p->mem);
        return st;
    }
    *plan_out = p.release();
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_csr_spmm_plan_create(int64_t m, int64_t n, int64_t k, int64_t nnz, int32_t origin,
                                              int value_type, const int32_t *rowptr, const int32_t *colind,
                                              const void *val, jlust_stream_t stream,
                                              jlust_spmm_plan_t *plan_out)
{
    return jlust::host_guard("csr_spmm_plan_create", [&] {
        return csr_spmm_plan_create_body(m, n, k, nnz, origin, value_type, rowptr, colind, val, stream,
                                         plan_out);
    });
}

extern "C" int jlust_hip_csr_spmm_plan_update_values(jlust_spmm_plan_t plan, const void *val,
                                                     jlust_stream_t stream)
{
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmm_plan_update_values: null plan");
    if (bad_ptr(val, plan->nnz)) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmm_plan_update_values: null values");
    if (!plan->perm) {
        plan->val = val;    // the kernels read the values in place: nothing to copy
        return JLUST_STATUS_SUCCESS;
    }
    // A reordered COO/CSC plan: the values into its row order, on the stream.
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    if (dev != plan->device)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "spmm_plan_update_values: plan belongs to device %d, current device is %d", plan->device, dev);
    return perm_gather(plan->value_type, plan->nnz, plan->perm, val, plan->val_copy, (hipStream_t)stream);
}

template <typename T>
static int spmm_plan_execute(jlust_spmm_plan_t p, int want_type, T alpha, const T *B, int64_t ldb, T beta, T *C,
                             int64_t ldc, int skip_empty_rows, jlust_stream_t stream)
{
    clear_error();
    if (!p) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmm_plan_execute: null plan");
    if (p->value_type != want_type)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "spmm_plan_execute: plan was created for %s values",
                    p->value_type == 0 ? "Float64" : "Float32");
    if (int st = check_dense_args("spmm_plan_execute", p->m, p->n, p->k, p->nnz, B, ldb, C, ldc)) return st;
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    if (dev != p->device)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmm_plan_execute: plan belongs to device %d, current device is %d",
                    p->device, dev);
    if (p->m == 0 || p->k == 0) return JLUST_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;
    const T *val = (const T *)p->val;
    T *Bt = (T *)p->Bt;
    T *part = (T *)p->part;
    const int bz = beta == T(0);
    for (int64_t c0 = 0; c0 < p->k; c0 += p->kc) {
        const int64_t kk = min(p->kc, p->k - c0);
        const SpmmChunk ck = spmm_chunk_kind(kk);
        if (int st = spmm_copy_chunk<T>(p->n, kk, B + c0 * ldb, ldb, ck, Bt, s)) return st;
        const T *Bsrc = ck.direct ? B + c0 * ldb : Bt;
        if (int st = spmm_chunk_launch<T>(p->m, kk, p->nnz_rows, p->origin, p->rowptr, nullptr, p->row_skip,
                                          p->colind, val, Bsrc, ck, alpha, beta, C + c0 * ldc, ldc,
                                          skip_empty_rows, s))
            return st;
        if (p->nseg == 0) continue;
        if (int st = spmm_chunk_launch<T>(p->nseg, kk, p->nnz - p->nnz_rows, p->origin, p->seg_lo, p->seg_hi,
                                          nullptr, p->colind, val, Bsrc, ck, T(1), T(0), part, p->nseg, 0, s))
            return st;
        const int64_t t = p->nlong * kk;
        hipLaunchKernelGGL((spmm_long_reduce_kernel<T>), dim3((unsigned)((t + 255) / 256)), dim3(256), 0, s,
                           p->nlong, kk, p->long_rows, p->seg_first, part, p->nseg, alpha, beta, bz,
                           C + c0 * ldc, ldc);
        if (int st = check_launch("spmm_long_reduce_kernel")) return st;
    }
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_csr_spmm_plan_execute_f64(jlust_spmm_plan_t plan, double alpha, const double *B,
                                                   int64_t ldb, double beta, double *C, int64_t ldc,
                                                   int skip_empty_rows, jlust_stream_t stream)
{
    return spmm_plan_execute<double>(plan, 0, alpha, B, ldb, beta, C, ldc, skip_empty_rows, stream);
}

extern "C" int jlust_hip_csr_spmm_plan_execute_f32(jlust_spmm_plan_t plan, float alpha, const float *B,
                                                   int64_t ldb, float beta, float *C, int64_t ldc,
                                                   int skip_empty_rows, jlust_stream_t stream)
{
    return spmm_plan_execute<float>(plan, 1, alpha, B, ldb, beta, C, ldc, skip_empty_rows, stream);
}

extern "C" int jlust_hip_csr_spmm_plan_info(jlust_spmm_plan_t plan, int64_t *split_rows, int64_t *segments,
                                            int64_t *cols_per_pass, int32_t *reordered)
{
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmm_plan_info: null plan");
    if (split_rows) *split_rows = plan->nlong;
    if (segments) *segments = plan->nseg;
    if (cols_per_pass) *cols_per_pass = plan->kc;
    if (reordered) *reordered = plan->perm != nullptr;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_csr_spmm_plan_destroy(jlust_spmm_plan_t plan)
{
    clear_error();
    if (!plan) return JLUST_STATUS_SUCCESS;
    // Work queued on any stream may still read the plan's buffers.
    hipError_t e = hipDeviceSynchronize();
    for (void *m : {plan->mem, plan->own_mem}) {
        if (!m) continue;
        const hipError_t e2 = hipFree(m);
        if (e == hipSuccess) e = e2;
    }
    delete plan;
    if (e != hipSuccess) return hip_fail(e, "spmm_plan_destroy");
    return JLUST_STATUS_SUCCESS;
}

namespace jlust {
int preload_spmm()
{
    JLUST_PRELOAD_KERNEL(transpose_kernel<float>);
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
