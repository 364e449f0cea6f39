// sddmm.hip -- CSR SDDMM for gfx950 (wave64):
//   Cval[p] = alpha*dot(A[i,:], B[:,j]) (*mask[p]) + beta*Cval[p]
// for every stored (i, j) of the CSR pattern.  A is m x K (lda) and B is
// K x n (ldb), both column-major (Julia layout), so a column B[:, j] is
// contiguous and a row A[i, :] is strided by lda.
//
// Replaces execute(::EmitterBackend, ::Op{:SDDMM}, ...)
// (ext/KernelAbstractionsExt/ops/sddmm.jl:49-65; body :23-30).
//
// A block owns R consecutive rows of the pattern.  It first stages A[rows, :]
// in LDS, row-major, reading each column segment A[i0:i0+R, kk] coalesced.
// Its nonzeros (contiguous in colind) are then shared out to groups of G
// lanes, one nonzero per group at a time: each lane multiplies a 16-byte
// slice of B[:, j] (one vector load; the group reads the column as contiguous
// 128-byte lines) with the matching slice of the staged A row, and the group
// reduces its G partial dots with xor-shuffles.  G = 8 for K above 8 slices
// (K of 16, 32 or 64 slices: the lane's 2, 4 or 8 loads of B are issued
// together, the rest loop); for smaller K, G is the smallest power of two
// whose slices cover K, and each group takes U nonzeros per step with their
// loads issued together (indices clamped into the block's nonzeros, results
// of the clamped copies dropped), so K = 1 puts 64 nonzeros on a wave per
// load instead of 8.
#include <algorithm>
#include <memory>
#include <vector>

#include "common.hpp"

namespace jlust {
namespace {

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

constexpr int SD_BLOCK = 256;
constexpr int SD_GROUP = 8;
constexpr int SD_GROUPS = SD_BLOCK / SD_GROUP;
constexpr size_t SD_LDS_BUDGET = 48 * 1024;
constexpr int64_t SD_GRID_MAX = 1 << 20;     // grid cap of the grid-stride kernels

template <typename T> struct V16;
template <> struct alignas(16) V16<float> { float v[4]; static constexpr int N = 4; };
template <> struct alignas(16) V16<double> { double v[2]; static constexpr int N = 2; };

template <int G, typename T>
__device__ __forceinline__ T group_sum(T v)
{
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// VECB: B columns and the LDS rows allow 16-byte vector access.  KS >= 1: a
// group covers K in exactly KS steps of its G slices (KS = 1: at most one
// step, lanes past K idle), so all KS loads of U nonzeros are issued before
// any arithmetic; KS = 0: U = 1 and the lanes loop over K.
template <typename T, bool VECB, int G, int U, int KS>
__global__ __launch_bounds__(SD_BLOCK) void csr_sddmm_kernel(
    int64_t m, int64_t K, int32_t origin, const int32_t *__restrict__ rowptr,
    const int32_t *__restrict__ colind, T alpha, const T *__restrict__ A, int64_t lda,
    const T *__restrict__ B, int64_t ldb, T beta, int beta_zero, T *Cval,
    const T *mask, int R, int64_t lds_ld, const int32_t *__restrict__ items, int64_t chunk,
    const int32_t *__restrict__ perm, const int32_t *__restrict__ rowmap, int64_t a_rows)
{
    static_assert(KS >= 1 || U == 1, "several nonzeros per group need a fixed step count over K");
    static_assert(KS <= 1 || VECB, "several steps over K need vector loads");
    constexpr int GROUPS = SD_BLOCK / G;
    constexpr int NE = VECB ? V16<T>::N : 1;   // elements per lane load
    extern __shared__ unsigned char sd_smem[];
    T *s_a = reinterpret_cast<T *>(sd_smem);                       // R x lds_ld
    int32_t *s_rp = reinterpret_cast<int32_t *>(s_a + (int64_t)R * lds_ld);  // R + 1
    int32_t *s_ar = s_rp + R + 1;            // R: A's row of each pattern row

    const int tid = threadIdx.x;
    const int g = tid / G;                   // group in block
    const int q = tid % G;                   // lane in group
    // A plan's work item: (row block, part) -- the part-th run of `chunk`
    // nonzeros of that block; without items, block b is row block b whole.
    const int64_t rb = items ? items[2 * (int64_t)blockIdx.x] : (int64_t)blockIdx.x;
    const int64_t part = items ? items[2 * (int64_t)blockIdx.x + 1] : 0;
    const int64_t i0 = rb * R;
    const int nr = (int)min((int64_t)R, m - i0);

    for (int r = tid; r <= nr; r += SD_BLOCK) s_rp[r] = rowptr[i0 + r] - origin;
    // A DCSR mask walks its stored rows: pattern row i is A's row rowmap[i]
    // (clamped into A, so a malformed row index reads no memory outside it).
    for (int r = tid; r < nr; r += SD_BLOCK)
        s_ar[r] = rowmap ? (int32_t)min(max((int64_t)rowmap[i0 + r] - origin, (int64_t)0), a_rows - 1)
                         : (int32_t)(i0 + r);
    __syncthreads();
    for (int64_t idx = tid; idx < (int64_t)nr * K; idx += SD_BLOCK) {
        const int rr = (int)(idx % nr);
        const int64_t kk = idx / nr;
        s_a[rr * lds_ld + kk] = A[(int64_t)s_ar[rr] + kk * lda];
    }
    __syncthreads();

    int64_t p_lo = s_rp[0], p_hi = s_rp[nr];
    if (items) {
        p_lo += part * chunk;
        p_hi = min(p_hi, p_lo + chunk);
    }
    // This lane's slice of K in the one-step case, clamped into range.
    const int64_t k1 = (int64_t)q * NE;
    const bool k1_ok = k1 < K;
    const int64_t k1c = k1_ok ? k1 : K - NE;
    // 64-bit positions: p0 + GROUPS*U may pass INT32_MAX near the end.
    for (int64_t p0 = (int64_t)p_lo + g; p0 < p_hi; p0 += GROUPS * U) {
        int64_t pc[U];
        int64_t j[U];
        const T *arow[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t p = p0 + u * GROUPS;
            pc[u] = p < p_hi ? p : p0;
            j[u] = (int64_t)colind[pc[u]] - origin;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int lo = 0, hi = nr - 1;             // row rr with s_rp[rr] <= p < s_rp[rr+1]
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (s_rp[mid] <= pc[u]) lo = mid;
                else hi = mid - 1;
            }
            arow[u] = s_a + lo * lds_ld;
        }
        T dot[U];
        if (KS >= 1) {
            if (VECB) {
                // Step s of lane q covers K elements (s*G + q)*NE ..+NE, the order of
                // the looping form below, so both give the same sums.
                constexpr int KS1 = KS >= 1 ? KS : 1;
                V16<T> bv[U][KS1];
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int st = 0; st < KS1; ++st)
                        bv[u][st] = *reinterpret_cast<const V16<T> *>(B + j[u] * ldb + k1c + st * G * NE);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    T d = T(0);
#pragma unroll
                    for (int st = 0; st < KS1; ++st) {
                        const V16<T> av = *reinterpret_cast<const V16<T> *>(arow[u] + k1c + st * G * NE);
#pragma unroll
                        for (int e = 0; e < NE; ++e) d += av.v[e] * bv[u][st].v[e];
                    }
                    dot[u] = k1_ok ? d : T(0);
                }
            } else {
                T bv[U];
#pragma unroll
                for (int u = 0; u < U; ++u) bv[u] = B[j[u] * ldb + k1c];
#pragma unroll
                for (int u = 0; u < U; ++u) dot[u] = k1_ok ? arow[u][k1c] * bv[u] : T(0);
            }
        } else {
            const T *bcol = B + j[0] * ldb;
            T d = T(0);
            if (VECB) {
                for (int64_t kk = k1; kk < K; kk += G * NE) {
                    const V16<T> bv = *reinterpret_cast<const V16<T> *>(bcol + kk);
                    const V16<T> av = *reinterpret_cast<const V16<T> *>(arow[0] + kk);
#pragma unroll
                    for (int e = 0; e < NE; ++e) d += av.v[e] * bv.v[e];
                }
            } else {
                for (int64_t kk = q; kk < K; kk += G) d += arow[0][kk] * bcol[kk];
            }
            dot[0] = d;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) dot[u] = group_sum<G>(dot[u]);
        if (q == 0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t p = p0 + u * GROUPS;
                if (p < p_hi) {
                    const int64_t o = perm ? (int64_t)perm[p] : p;   // output position
                    T out = alpha * dot[u];
                    if (mask) out = mask[o] * out;
                    if (!beta_zero) out += beta * Cval[o];
                    Cval[o] = out;
                }
            }
        }
    }
}

// No-LDS fallback for very large K (A row read with stride lda).
template <typename T>
__global__ __launch_bounds__(SD_BLOCK) void csr_sddmm_direct_kernel(
    int64_t m, int64_t K, int32_t origin, const int32_t *__restrict__ rowptr,
    const int32_t *__restrict__ colind, T alpha, const T *__restrict__ A, int64_t lda,
    const T *__restrict__ B, int64_t ldb, T beta, int beta_zero, T *Cval, const T *mask,
    const int32_t *__restrict__ perm, const int32_t *__restrict__ rowmap, int64_t a_rows)
{
    const int g = threadIdx.x / SD_GROUP, q = threadIdx.x % SD_GROUP;
    // Rows by grid stride: the grid is capped, so any m launches.
    for (int64_t i = blockIdx.x; i < m; i += gridDim.x) {
        const int64_t lo = (int64_t)rowptr[i] - origin, hi = (int64_t)rowptr[i + 1] - origin;
        const int64_t ai = rowmap ? min(max((int64_t)rowmap[i] - origin, (int64_t)0), a_rows - 1) : i;
        for (int64_t p = lo + g; p < hi; p += SD_GROUPS) {
            const int64_t j = (int64_t)colind[p] - origin;
            T dot = T(0);
            for (int64_t kk = q; kk < K; kk += SD_GROUP) dot += A[ai + kk * lda] * B[kk + j * ldb];
            dot = group_sum<SD_GROUP>(dot);
            if (q == 0) {
                const int64_t o = perm ? (int64_t)perm[p] : p;
                T out = alpha * dot;
                if (mask) out = mask[o] * out;
                if (!beta_zero) out += beta * Cval[o];
                Cval[o] = out;
            }
        }
    }
}

// COO mask, no analysis (the plain COO SDDMM call): a group of SD_GROUP
// lanes per stored entry in storage order, A's row read with stride lda.
template <typename T>
__global__ __launch_bounds__(SD_BLOCK) void coo_sddmm_kernel(
    int64_t nnz, int64_t K, int32_t origin, const int32_t *__restrict__ rows,
    const int32_t *__restrict__ cols, T alpha, const T *__restrict__ A, int64_t lda,
    const T *__restrict__ B, int64_t ldb, T beta, int beta_zero, T *Cval, const T *mask)
{
    const int g = threadIdx.x / SD_GROUP, q = threadIdx.x % SD_GROUP;
    // Entries by grid stride (the grid is capped); the 8 lanes of a group share p.
    for (int64_t p = (int64_t)blockIdx.x * SD_GROUPS + g; p < nnz; p += (int64_t)gridDim.x * SD_GROUPS) {
        const int64_t i = (int64_t)rows[p] - origin, j = (int64_t)cols[p] - origin;
        T dot = T(0);
        for (int64_t kk = q; kk < K; kk += SD_GROUP) dot += A[i + kk * lda] * B[kk + j * ldb];
        dot = group_sum<SD_GROUP>(dot);
        if (q == 0) {
            T out = alpha * dot;
            if (mask) out = mask[p] * out;
            if (!beta_zero) out += beta * Cval[p];
            Cval[p] = out;
        }
    }
}

// Rows per block for A's staging: as many (up to 32) as fit the LDS budget
// with rows padded to 16 bytes; 0 = K too large, the direct kernel runs.
template <typename T>
int sddmm_rows(int64_t K, int64_t *lds_ld)
{
    constexpr int N = V16<T>::N;
    *lds_ld = (K + N - 1) / N * N + N;       // padded, keeps rows 16-byte aligned
    int64_t R = (int64_t)((SD_LDS_BUDGET - 128 * sizeof(int32_t)) / (sizeof(T) * (size_t)*lds_ld));
    return (int)(R > 32 ? 32 : R);
}

// The SDDMM launch over the CSR pattern (rowptr, colind) of m rows, plain or
// from a plan: items/chunk cut row blocks into runs of nonzeros (null: one
// block per row block), perm maps CSR positions to the output's (null:
// identity), rowmap gives A's row (of a_rows) of each pattern row (null:
// the same row; a DCSR mask's stored rows otherwise).
template <typename T>
int sddmm_launch(int64_t m, int64_t K, int32_t origin, const int32_t *rowptr, const int32_t *colind, T alpha,
                 const T *A, int64_t lda, const T *B, int64_t ldb, T beta, T *Cval, const T *mask,
                 const int32_t *items, int64_t nitems, int64_t chunk, const int32_t *perm,
                 const int32_t *rowmap, int64_t a_rows, hipStream_t s)
{
    const int bz = beta == T(0);
    constexpr int N = V16<T>::N;
    int64_t lds_ld = 0;
    const int R = sddmm_rows<T>(K, &lds_ld);
    if (R < 1) {
        hipLaunchKernelGGL((csr_sddmm_direct_kernel<T>), dim3((unsigned)std::min<int64_t>(m, SD_GRID_MAX)),
                           dim3(SD_BLOCK), 0, s, m,
                           K, origin, rowptr, colind, alpha, A, lda, B, ldb, beta, bz, Cval, mask, perm, rowmap,
                           a_rows);
        return check_launch("csr_sddmm_direct_kernel");
    }
    const bool vecb = (K % N == 0) && (ldb % N == 0) && (((uintptr_t)B) % 16 == 0);
    const size_t smem = sizeof(T) * (size_t)R * (size_t)lds_ld + sizeof(int32_t) * (size_t)(2 * R + 1);
    const dim3 grid((unsigned)(items ? nitems : (m + R - 1) / R));
    // Lane loads that cover K: G = the smallest power of two >= that, up to 8.
    const int64_t slices = vecb ? K / N : K;
#define JLUST_SD(V, G, U, KS)                                                                         \
    hipLaunchKernelGGL((csr_sddmm_kernel<T, V, G, U, KS>), grid, dim3(SD_BLOCK), smem, s, m, K, origin, \
                       rowptr, colind, alpha, A, lda, B, ldb, beta, bz, Cval, mask, R, lds_ld, items,  \
                       chunk, perm, rowmap, a_rows)
#define JLUST_SD_V(V)                                                                                 \
    do {                                                                                              \
        if (slices == 0) JLUST_SD(V, 8, 1, 0);     /* K = 0: no loads of B at all */                 \
        else if (slices <= 1) JLUST_SD(V, 1, 4, 1);                                                   \
        else if (slices <= 2) JLUST_SD(V, 2, 4, 1);                                                   \
        else if (slices <= 4) JLUST_SD(V, 4, 2, 1);                                                   \
        else if (slices <= 8) JLUST_SD(V, 8, 1, 1);                                                   \
        else JLUST_SD(V, 8, 1, 0);                                                                    \
    } while (0)
    // K a multiple of 2, 4 or 8 whole steps of 8 lanes: every load of the column
    // issued at once (one nonzero per group; two per group measured slower).
    if (vecb && slices == 16) JLUST_SD(true, 8, 1, 2);
    else if (vecb && slices == 32) JLUST_SD(true, 8, 1, 4);
    else if (vecb && slices == 64) JLUST_SD(true, 8, 1, 8);
    else if (vecb) JLUST_SD_V(true);
    else JLUST_SD_V(false);
#undef JLUST_SD_V
#undef JLUST_SD
    return check_launch("csr_sddmm_kernel");
}

int check_sddmm_dense(const char *who, int64_t m, int64_t n, int64_t K, int64_t nnz, const void *A, int64_t lda,
                      const void *B, int64_t ldb, const void *Cval)
{
    if (lda < (m > 0 ? m : 1) || ldb < (K > 0 ? K : 1))
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "%s: leading dimensions too small (lda=%lld < m=%lld or ldb=%lld < K=%lld)", who,
                    (long long)lda, (long long)m, (long long)ldb, (long long)K);
    if (bad_ptr(Cval, nnz) || bad_ptr(A, (nnz > 0 && K > 0) ? m : 0) || bad_ptr(B, (nnz > 0 && K > 0) ? n : 0))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: null device pointer", who);
    return JLUST_STATUS_SUCCESS;
}

int check_sddmm_extents(const char *who, int64_t m, int64_t n, int64_t K, int64_t nnz, int32_t origin)
{
    if (m < 0 || n < 0 || K < 0 || nnz < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: negative extent", who);
    if (m > INT32_MAX - 1 || n > INT32_MAX || nnz > INT32_MAX - 1)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: extents exceed the Int32 index range", who);
    return check_origin(origin);
}

template <typename T>
int csr_sddmm(int64_t m, int64_t n, int64_t K, int64_t nnz, int32_t origin,
              const int32_t *rowptr, const int32_t *colind, T alpha, const T *A, int64_t lda,
              const T *B, int64_t ldb, T beta, T *Cval, const T *mask, jlust_stream_t stream)
{
    clear_error();
    if (int st = check_sddmm_extents("csr_sddmm", m, n, K, nnz, origin)) return st;
    if (int st = check_sddmm_dense("csr_sddmm", m, n, K, nnz, A, lda, B, ldb, Cval)) return st;
    if ((m > 0 && !rowptr) || bad_ptr(colind, nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_sddmm: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (m == 0 || nnz == 0) return JLUST_STATUS_SUCCESS;
    return sddmm_launch<T>(m, K, origin, rowptr, colind, alpha, A, lda, B, ldb, beta, Cval, mask, nullptr, 0, 0,
                           nullptr, nullptr, m, (hipStream_t)stream);
}

// DCSR mask: the CSR kernel over the nout stored rows (pos, cols), reading A's
// row rows[r] for stored row r; outputs in the mask's storage order.
template <typename T>
int dcsr_sddmm(int64_t m, int64_t n, int64_t K, int64_t nout, int64_t nnz, int32_t origin, const int32_t *rows,
               const int32_t *pos, const int32_t *cols, T alpha, const T *A, int64_t lda, const T *B, int64_t ldb,
               T beta, T *Cval, const T *mask, jlust_stream_t stream)
{
    clear_error();
    if (int st = check_sddmm_extents("dcsr_sddmm", m, n, K, nnz, origin)) return st;
    if (nout < 0 || nout > m)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "dcsr_sddmm: %lld stored rows in a matrix of %lld rows",
                    (long long)nout, (long long)m);
    if (int st = check_sddmm_dense("dcsr_sddmm", m, n, K, nnz, A, lda, B, ldb, Cval)) return st;
    if (bad_ptr(rows, nout) || (nout > 0 && !pos) || bad_ptr(cols, nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "dcsr_sddmm: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (nout == 0 || nnz == 0) return JLUST_STATUS_SUCCESS;
    return sddmm_launch<T>(nout, K, origin, pos, cols, alpha, A, lda, B, ldb, beta, Cval, mask, nullptr, 0, 0,
                           nullptr, rows, m, (hipStream_t)stream);
}

template <typename T>
int coo_sddmm(int64_t m, int64_t n, int64_t K, int64_t nnz, int32_t origin, const int32_t *rows,
              const int32_t *cols, T alpha, const T *A, int64_t lda, const T *B, int64_t ldb, T beta, T *Cval,
              const T *mask, jlust_stream_t stream)
{
    clear_error();
    if (int st = check_sddmm_extents("coo_sddmm", m, n, K, nnz, origin)) return st;
    if (int st = check_sddmm_dense("coo_sddmm", m, n, K, nnz, A, lda, B, ldb, Cval)) return st;
    if (bad_ptr(rows, nnz) || bad_ptr(cols, nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_sddmm: null device pointer");
    if (nnz > 0 && (m == 0 || n == 0))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "coo_sddmm: entries in an empty matrix");
    if (int st = require_device(nullptr)) return st;
    if (nnz == 0) return JLUST_STATUS_SUCCESS;
    hipLaunchKernelGGL((coo_sddmm_kernel<T>),
                       dim3((unsigned)std::min<int64_t>((nnz + SD_GROUPS - 1) / SD_GROUPS, SD_GRID_MAX)), dim3(SD_BLOCK),
                       0, (hipStream_t)stream, nnz, K, origin, rows, cols, alpha, A, lda, B, ldb, beta,
                       (int)(beta == T(0)), Cval, mask);
    return check_launch("coo_sddmm_kernel");
}

}  // namespace
}  // namespace jlust

using namespace jlust;

extern "C" int jlust_hip_csr_sddmm_f64_i32(int64_t m, int64_t n, int64_t K, int64_t nnz,
                                           int32_t origin, const int32_t *rowptr,
                                           const int32_t *colind, double alpha, const double *A,
                                           int64_t lda, const double *B, int64_t ldb, double beta,
                                           double *Cval, const double *mask, jlust_stream_t stream)
{
    return csr_sddmm<double>(m, n, K, nnz, origin, rowptr, colind, alpha, A, lda, B, ldb, beta,
                             Cval, mask, stream);
}

extern "C" int jlust_hip_csr_sddmm_f32_i32(int64_t m, int64_t n, int64_t K, int64_t nnz,
                                           int32_t origin, const int32_t *rowptr,
                                           const int32_t *colind, float alpha, const float *A,
                                           int64_t lda, const float *B, int64_t ldb, float beta,
                                           float *Cval, const float *mask, jlust_stream_t stream)
{
    return csr_sddmm<float>(m, n, K, nnz, origin, rowptr, colind, alpha, A, lda, B, ldb, beta,
                            Cval, mask, stream);
}

extern "C" int jlust_hip_coo_sddmm_f64_i32(int64_t m, int64_t n, int64_t K, int64_t nnz, int32_t origin,
                                           const int32_t *rows, const int32_t *cols, double alpha,
                                           const double *A, int64_t lda, const double *B, int64_t ldb,
                                           double beta, double *Cval, const double *mask, jlust_stream_t stream)
{
    return coo_sddmm<double>(m, n, K, nnz, origin, rows, cols, alpha, A, lda, B, ldb, beta, Cval, mask, stream);
}

extern "C" int jlust_hip_coo_sddmm_f32_i32(int64_t m, int64_t n, int64_t K, int64_t nnz, int32_t origin,
                                           const int32_t *rows, const int32_t *cols, float alpha,
                                           const float *A, int64_t lda, const float *B, int64_t ldb,
                                           float beta, float *Cval, const float *mask, jlust_stream_t stream)
{
    return coo_sddmm<float>(m, n, K, nnz, origin, rows, cols, alpha, A, lda, B, ldb, beta, Cval, mask, stream);
}

extern "C" int jlust_hip_dcsr_sddmm_f64_i32(int64_t m, int64_t n, int64_t K, int64_t nout, int64_t nnz,
                                            int32_t origin, const int32_t *rows, const int32_t *pos,
                                            const int32_t *cols, double alpha, const double *A, int64_t lda,
                                            const double *B, int64_t ldb, double beta, double *Cval,
                                            const double *mask, jlust_stream_t stream)
{
    return dcsr_sddmm<double>(m, n, K, nout, nnz, origin, rows, pos, cols, alpha, A, lda, B, ldb, beta, Cval,
                              mask, stream);
}

extern "C" int jlust_hip_dcsr_sddmm_f32_i32(int64_t m, int64_t n, int64_t K, int64_t nout, int64_t nnz,
                                            int32_t origin, const int32_t *rows, const int32_t *pos,
                                            const int32_t *cols, float alpha, const float *A, int64_t lda,
                                            const float *B, int64_t ldb, float beta, float *Cval,
                                            const float *mask, jlust_stream_t stream)
{
    return dcsr_sddmm<float>(m, n, K, nout, nnz, origin, rows, pos, cols, alpha, A, lda, B, ldb, beta, Cval,
                             mask, stream);
}

// ------------------------------------------------------------------- plans

// A prepared SDDMM (the cuSPARSE SDDMM handle contract, ext/CUDAExt/ops/
// sddmm.jl:10-76).  Analysis: the mask in CSR order (a COO mask is put in row
// order once: rowptr, columns and the permutation back to its storage order,
// so outputs and mask values stay in the caller's order), then the work
// items: every row block of R rows holding nonzeros, cut into runs of at
// most SD_CHUNK nonzeros.  Row blocks without nonzeros get no item (their A
// rows are never read), and a block holding a very long row is shared by
// several workgroups instead of one.
constexpr int64_t SD_CHUNK = 4096;

struct jlust_sddmm_plan {
    int64_t m = 0, n = 0, K = 0, nnz = 0;
    int64_t nrows = 0;                 // pattern rows walked (m; a DCSR mask's stored rows)
    int32_t origin = 0;
    int value_type = 0;
    int device = 0;
    const int32_t *rowptr = nullptr;   // CSR order: the caller's, or owned (COO, CSC)
    const int32_t *colind = nullptr;
    const int32_t *perm = nullptr;     // output position of CSR position q (null: q)
    const int32_t *rowmap = nullptr;   // A's row of pattern row r (DCSR; null: r)
    int32_t *items = nullptr;          // [2 * nitems] (row block, part)
    int64_t nitems = 0;
    void *mem = nullptr;
};

// mask_format CSR: idx1 = rowptr, idx2 = colind; COO: idx1 = rows, idx2 =
// cols; CSC: idx1 = colptr, idx2 = rowind; DCSR: dcsr_rows[nout] with idx1 =
// pos[nout+1], idx2 = cols.
static int sddmm_plan_create_body(int32_t mask_format, int64_t m, int64_t n, int64_t K, int64_t nnz,
                                  int32_t origin, int value_type, const int32_t *idx1,
                                  const int32_t *idx2, int64_t nout, const int32_t *dcsr_rows,
                                  jlust_stream_t stream, jlust_sddmm_plan_t *plan_out)
{
    clear_error();
    if (!plan_out) return fail(JLUST_STATUS_INVALID_ARGUMENT, "sddmm_plan_create: null plan_out");
    *plan_out = nullptr;
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE,
                    "sddmm_plan_create: value_type %d (0 = Float64, 1 = Float32)", value_type);
    if (mask_format != JLUST_FORMAT_CSR && mask_format != JLUST_FORMAT_COO && mask_format != JLUST_FORMAT_CSC &&
        mask_format != JLUST_FORMAT_DCSR)
        return fail(JLUST_STATUS_UNSUPPORTED_FORMAT, "sddmm_plan_create: the mask must be CSR, COO, CSC or DCSR");
    if (int st = check_sddmm_extents("sddmm_plan_create", m, n, K, nnz, origin)) return st;
    const bool coo = mask_format == JLUST_FORMAT_COO, csc = mask_format == JLUST_FORMAT_CSC;
    const bool dcsr = mask_format == JLUST_FORMAT_DCSR;
    if (dcsr && (nout < 0 || nout > m))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "sddmm_plan_create: %lld stored rows in a matrix of %lld rows",
                    (long long)nout, (long long)m);
    const int64_t nrows = dcsr ? nout : m;
    if ((!coo && nrows > 0 && !idx1) || (coo && bad_ptr(idx1, nnz)) || bad_ptr(idx2, nnz) ||
        (dcsr && bad_ptr(dcsr_rows, nout)))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "sddmm_plan_create: null device pointer");
    if (nnz > 0 && (m == 0 || n == 0))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "sddmm_plan_create: entries in an empty matrix");
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    hipStream_t s = (hipStream_t)stream;
    std::unique_ptr<jlust_sddmm_plan> p(new jlust_sddmm_plan());
    p->m = m;
    p->n = n;
    p->K = K;
    p->nnz = nnz;
    p->nrows = nrows;
    p->origin = origin;
    p->value_type = value_type;
    p->device = dev;
    p->rowptr = idx1;
    p->colind = idx2;
    p->rowmap = dcsr ? dcsr_rows : nullptr;
    int64_t lds_ld = 0;
    const int R = value_type == 0 ? sddmm_rows<double>(K, &lds_ld) : sddmm_rows<float>(K, &lds_ld);
    const int64_t nblk = R >= 1 ? (nrows + R - 1) / R : 0;
    const size_t nz = (size_t)(nnz > 0 ? nnz : 1);
    // Owned: [rowptr, perm, columns (COO, CSC), CSC's column per entry],
    // items (at most 2 per block plus one per SD_CHUNK nonzeros).
    const bool reorder = coo || csc;
    const size_t sz_rp = reorder ? align_up(4 * (size_t)(m + 1), 256) : 0;
    const size_t sz_i = reorder ? align_up(4 * nz, 256) : 0;
    const size_t sz_ce = csc ? align_up(4 * nz, 256) : 0;
    const int64_t max_items = nblk + nnz / SD_CHUNK + 1;
    const size_t sz_items = align_up(8 * (size_t)max_items, 256);
    // Host tables before the device allocation (a failed host allocation then
    // leaks nothing): the row pointers and the work items (row block, part).
    const bool analyse = R >= 1 && nrows > 0;
    std::vector<int32_t> rp(analyse ? (size_t)(nrows + 1) : 0);
    std::vector<int32_t> items;
    if (analyse) items.reserve(2 * (size_t)max_items);
    JLUST_HIP_TRY(hipMalloc(&p->mem, sz_rp + 2 * sz_i + sz_ce + sz_items));
    char *b = (char *)p->mem;
    int st = JLUST_STATUS_SUCCESS;
    if (reorder) {
        int32_t *rowptr = (int32_t *)b;
        int32_t *perm = (int32_t *)(b + sz_rp);
        int32_t *cols_s = (int32_t *)(b + sz_rp + sz_i);
        const int32_t *rows = idx1, *cols = idx2;
        if (csc) {
            // The column of every entry: the mask as COO (rowind, column) in storage order.
            int32_t *ce = (int32_t *)(b + sz_rp + 2 * sz_i);
            st = expand_pos(n, nnz, origin, idx1, nullptr, ce, s);
            rows = idx2;
            cols = ce;
        }
        bool sorted = true;
        if (!st) st = coo_row_order(m, nnz, origin, rows, cols, rowptr, perm, cols_s, &sorted, s);
        p->rowptr = rowptr;
        p->colind = cols;
        if (!sorted) {
            p->perm = perm;
            p->colind = cols_s;
        }
    }
    p->items = (int32_t *)(b + sz_rp + 2 * sz_i + sz_ce);
    // Work items from the row pointers of each row block (host analysis).
    if (!st && dcsr && nout > 0)
        st = check_pos("sddmm_plan_create", nout, nnz, origin, p->rowptr, s);
    if (!st && analyse) {
        hipError_t e = hipMemcpyAsync(rp.data(), p->rowptr, sizeof(int32_t) * (size_t)(nrows + 1),
                                      hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) st = hip_fail(e, "sddmm_plan_create: rowptr copy");
        if (!st && ((int64_t)rp[0] != origin || (int64_t)rp[nrows] - origin != nnz))
            st = fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                      "sddmm_plan_create: rowptr runs from %d to %d, expected %d to %lld", rp[0], rp[nrows], origin,
                      (long long)(nnz + origin));
        for (int64_t rb = 0; !st && rb < nblk; ++rb) {
            const int64_t r1 = min((rb + 1) * (int64_t)R, nrows);
            const int64_t cnt = (int64_t)rp[r1] - rp[rb * R];
            if (cnt < 0) {
                st = fail(JLUST_STATUS_NONCANONICAL_STORAGE, "sddmm_plan_create: rowptr decreases near row %lld",
                          (long long)(rb * R));
                break;
            }
            for (int64_t part = 0; !st && part * SD_CHUNK < cnt; ++part) {
                if ((int64_t)items.size() >= 2 * max_items) {   // stays within the reserved tables
                    st = fail(JLUST_STATUS_HIP_ERROR, "sddmm_plan_create: item overflow");
                    break;
                }
                items.push_back((int32_t)rb);
                items.push_back((int32_t)part);
            }
        }
        p->nitems = (int64_t)items.size() / 2;
        if (!st && p->nitems > 0) {
            e = hipMemcpyAsync(p->items, items.data(), sizeof(int32_t) * items.size(), hipMemcpyHostToDevice, s);
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            if (e != hipSuccess) st = hip_fail(e, "sddmm_plan_create: item upload");
        }
    }
    if (st) {
        (void)hipStreamSynchronize(s);
        (void)hipFree(p->mem);
        return st;
    }
    *plan_out = p.release();
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_sddmm_plan_create(int32_t mask_format, int64_t m, int64_t n, int64_t K, int64_t nnz,
                                           int32_t origin, int value_type, const int32_t *idx1,
                                           const int32_t *idx2, jlust_stream_t stream,
                                           jlust_sddmm_plan_t *plan_out)
{
    if (mask_format == JLUST_FORMAT_DCSR) {
        clear_error();
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "sddmm_plan_create: DCSR masks use jlust_hip_dcsr_sddmm_plan_create");
    }
    return jlust::host_guard("sddmm_plan_create", [&] {
        return sddmm_plan_create_body(mask_format, m, n, K, nnz, origin, value_type, idx1, idx2, 0, nullptr, stream,
                                      plan_out);
    });
}

extern "C" int jlust_hip_dcsr_sddmm_plan_create(int64_t m, int64_t n, int64_t K, int64_t nout, int64_t nnz,
                                                int32_t origin, int value_type, const int32_t *rows,
                                                const int32_t *pos, const int32_t *cols, jlust_stream_t stream,
                                                jlust_sddmm_plan_t *plan_out)
{
    return jlust::host_guard("dcsr_sddmm_plan_create", [&] {
        return sddmm_plan_create_body(JLUST_FORMAT_DCSR, m, n, K, nnz, origin, value_type, pos, cols, nout, rows,
                                      stream, plan_out);
    });
}

template <typename T>
static int sddmm_plan_execute(jlust_sddmm_plan_t p, int want_type, T alpha, const T *A, int64_t lda, const T *B,
                              int64_t ldb, T beta, T *Cval, const T *mask, jlust_stream_t stream)
{
    clear_error();
    if (!p) return fail(JLUST_STATUS_INVALID_ARGUMENT, "sddmm_plan_execute: null plan");
    if (p->value_type != want_type)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "sddmm_plan_execute: plan was created for %s values",
                    p->value_type == 0 ? "Float64" : "Float32");
    if (int st = check_sddmm_dense("sddmm_plan_execute", p->m, p->n, p->K, p->nnz, A, lda, B, ldb, Cval)) return st;
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    if (dev != p->device)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "sddmm_plan_execute: plan belongs to device %d, current device is %d", p->device, dev);
    if (p->nrows == 0 || p->nnz == 0) return JLUST_STATUS_SUCCESS;
    return sddmm_launch<T>(p->nrows, p->K, p->origin, p->rowptr, p->colind, alpha, A, lda, B, ldb, beta, Cval,
                           mask, p->nitems > 0 ? p->items : nullptr, p->nitems, SD_CHUNK, p->perm, p->rowmap, p->m,
                           (hipStream_t)stream);
}

extern "C" int jlust_hip_sddmm_plan_execute_f64(jlust_sddmm_plan_t plan, double alpha, const double *A,
                                                int64_t lda, const double *B, int64_t ldb, double beta,
                                                double *Cval, const double *mask, jlust_stream_t stream)
{
    return sddmm_plan_execute<double>(plan, 0, alpha, A, lda, B, ldb, beta, Cval, mask, stream);
}

extern "C" int jlust_hip_sddmm_plan_execute_f32(jlust_sddmm_plan_t plan, float alpha, const float *A,
                                                int64_t lda, const float *B, int64_t ldb, float beta,
                                                float *Cval, const float *mask, jlust_stream_t stream)
{
    return sddmm_plan_execute<float>(plan, 1, alpha, A, lda, B, ldb, beta, Cval, mask, stream);
}

extern "C" int jlust_hip_sddmm_plan_info(jlust_sddmm_plan_t plan, int64_t *work_items, int32_t *reordered)
{
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "sddmm_plan_info: null plan");
    if (work_items) *work_items = plan->nitems;
    if (reordered) *reordered = plan->perm != nullptr;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_sddmm_plan_destroy(jlust_sddmm_plan_t plan)
{
    clear_error();
    if (!plan) return JLUST_STATUS_SUCCESS;
    hipError_t e = hipDeviceSynchronize();          // queued executes may still read the tables
    if (plan->mem) {
        const hipError_t e2 = hipFree(plan->mem);
        if (e == hipSuccess) e = e2;
    }
    delete plan;
    if (e != hipSuccess) return hip_fail(e, "sddmm_plan_destroy");
    return JLUST_STATUS_SUCCESS;
}

namespace jlust {
int preload_sddmm()
{
    JLUST_PRELOAD_KERNEL(coo_sddmm_kernel<float>);
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
