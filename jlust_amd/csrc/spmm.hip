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

namespace jlust {
namespace {

constexpr int SPMM_BLOCK = 256;
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
    int skip_empty_rows)
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
        hi_n = rowptr[row0 + wave + 1];
    }
    for (int rr = wave; rr < nrows; rr += NW) {
        const int64_t lo = (int64_t)lo_n - origin;
        const int64_t hi = (int64_t)hi_n - origin;
        if (rr + NW < nrows) {                 // the wave's next row
            lo_n = rowptr[row0 + rr + NW];
            hi_n = rowptr[row0 + rr + NW + 1];
        }
        if (lane == 0) s_empty[rr] = hi <= lo;
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
        if (skip_empty_rows && s_empty[rr]) continue;
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
    int skip_empty_rows)
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
            const int64_t hi = (int64_t)rowptr[row + 1] - origin;
            if (lane == 0 && c0 == 0) s_empty[rr] = hi <= lo;
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
            if (skip_empty_rows && s_empty[rr]) continue;
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

template <typename T>
int csr_spmm(int64_t m, int64_t n, int64_t k, int64_t nnz, int32_t origin,
             const int32_t *rowptr, const int32_t *colind, const T *val, T alpha, const T *B,
             int64_t ldb, T beta, T *C, int64_t ldc, int skip_empty_rows, jlust_stream_t stream)
{
    clear_error();
    if (m < 0 || n < 0 || k < 0 || nnz < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_spmm: negative extent");
    if (m > INT32_MAX || n > INT32_MAX || nnz > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_spmm: extents exceed the Int32 index range");
    if (int st = check_origin(origin)) return st;
    if (ldb < (n > 0 ? n : 1) || ldc < (m > 0 ? m : 1))
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "csr_spmm: leading dimensions too small (ldb=%lld < n=%lld or ldc=%lld < m=%lld)",
                    (long long)ldb, (long long)n, (long long)ldc, (long long)m);
    if ((m > 0 && !rowptr) || bad_ptr(colind, nnz) || bad_ptr(val, nnz) ||
        bad_ptr(B, (nnz > 0 && k > 0) ? n : 0) || bad_ptr(C, m * k))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_spmm: null device pointer");
    if (nnz > 0 && n == 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_spmm: nnz > 0 with n == 0");
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
    const dim3 grid((unsigned)((m + SPMM_ROWS - 1) / SPMM_ROWS));
    const int bz = beta == T(0);
    for (int64_t c0 = 0; c0 < k; c0 += kc) {
        const int64_t kk = min(kc, k - c0);
        const bool group = kk <= 32 && spmm_group();
        // One column needs no row-major copy: B's column is contiguous.  The
        // group kernel reads single elements, so its copy is unpadded (a
        // smaller footprint for the gathers); the wide kernel's rows are
        // padded to 16 bytes for its vector loads.
        const bool direct = group && kk == 1;
        const int64_t ldt = group ? kk : (kk + 3) / 4 * 4;
        const T *Bsrc = direct ? B + c0 * ldb : Bt;
        if (n > 0 && !direct) {
            dim3 tgrid((unsigned)((n + 63) / 64), (unsigned)((kk + 63) / 64));
            hipLaunchKernelGGL((transpose_kernel<T>), tgrid, dim3(256), 0, s, n, kk, B + c0 * ldb, ldb, Bt,
                               ldt);
            if (int st = check_launch("transpose_kernel")) return st;
        }
        const int vec = (sizeof(T) == 4) ? (kk <= 64 ? 1 : kk <= 128 ? 2 : 4) : (kk <= 64 ? 1 : 2);
        T *Cc = C + c0 * ldc;
#define JLUST_GROUP_U(KV, U)                                                                           \
    hipLaunchKernelGGL((csr_spmm_group_kernel<T, KV, U>), grid, dim3(SPMM_BLOCK), 0, s, m, kk, origin,    \
                       rowptr, colind, val, Bsrc, ldt, alpha, beta, bz, Cc, ldc, skip_empty_rows)
#define JLUST_GROUP(KV)                                                                                \
    do {                                                                                               \
        const int64_t steps = (nnz + m * (64 / KV) - 1) / (m * (64 / KV));  /* per row, rounded up */   \
        if (steps <= 1) JLUST_GROUP_U(KV, 1);                                                          \
        else if (steps <= 2) JLUST_GROUP_U(KV, 2);                                                     \
        else if (steps <= 4) JLUST_GROUP_U(KV, 4);                                                     \
        else JLUST_GROUP_U(KV, 8);                                                                     \
    } while (0)
        if (group) {
            if (kk == 1) JLUST_GROUP(1);
            else if (kk == 2) JLUST_GROUP(2);
            else if (kk <= 4) JLUST_GROUP(4);
            else if (kk <= 8) JLUST_GROUP(8);
            else if (kk <= 16) JLUST_GROUP(16);
            else JLUST_GROUP(32);
        }
#undef JLUST_GROUP_U
#undef JLUST_GROUP
        else if (vec == 1)
            hipLaunchKernelGGL((csr_spmm_kernel<T, 1>), grid, dim3(SPMM_BLOCK), 0, s, m, kk, origin,
                               rowptr, colind, val, Bt, ldt, alpha, beta, bz, Cc, ldc, skip_empty_rows);
        else if (vec == 2)
            hipLaunchKernelGGL((csr_spmm_kernel<T, 2>), grid, dim3(SPMM_BLOCK), 0, s, m, kk, origin,
                               rowptr, colind, val, Bt, ldt, alpha, beta, bz, Cc, ldc, skip_empty_rows);
        else
            hipLaunchKernelGGL((csr_spmm_kernel<T, 4>), grid, dim3(SPMM_BLOCK), 0, s, m, kk, origin,
                               rowptr, colind, val, Bt, ldt, alpha, beta, bz, Cc, ldc, skip_empty_rows);
        if (int st = check_launch("csr_spmm_kernel")) return st;
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
