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
// reduces its G partial dots with xor-shuffles.  G = 8 for K above 8 slices;
// for smaller K, G is the smallest power of two whose slices cover K, and
// each group takes U nonzeros per step with their loads issued together
// (indices clamped into the block's nonzeros, results of the clamped copies
// dropped), so K = 1 puts 64 nonzeros on a wave per load instead of 8.
#include "common.hpp"

namespace jlust {
namespace {

constexpr int SD_BLOCK = 256;
constexpr int SD_GROUP = 8;
constexpr int SD_GROUPS = SD_BLOCK / SD_GROUP;
constexpr size_t SD_LDS_BUDGET = 48 * 1024;

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

// VECB: B columns and the LDS rows allow 16-byte vector access.  ONE: a
// group's G slices cover all of K (one step per nonzero), so U nonzeros per
// group can be loaded at once; otherwise U = 1 and the lanes loop over K.
template <typename T, bool VECB, int G, int U, bool ONE>
__global__ __launch_bounds__(SD_BLOCK) void csr_sddmm_kernel(
    int64_t m, int64_t K, int32_t origin, const int32_t *__restrict__ rowptr,
    const int32_t *__restrict__ colind, T alpha, const T *__restrict__ A, int64_t lda,
    const T *__restrict__ B, int64_t ldb, T beta, int beta_zero, T *Cval,
    const T *mask, int R, int64_t lds_ld)
{
    static_assert(ONE || U == 1, "several nonzeros per group need one step over K");
    constexpr int GROUPS = SD_BLOCK / G;
    constexpr int NE = VECB ? V16<T>::N : 1;   // elements per lane load
    extern __shared__ unsigned char sd_smem[];
    T *s_a = reinterpret_cast<T *>(sd_smem);                       // R x lds_ld
    int32_t *s_rp = reinterpret_cast<int32_t *>(s_a + (int64_t)R * lds_ld);  // R + 1

    const int tid = threadIdx.x;
    const int g = tid / G;                   // group in block
    const int q = tid % G;                   // lane in group
    const int64_t i0 = (int64_t)blockIdx.x * R;
    const int nr = (int)min((int64_t)R, m - i0);

    for (int r = tid; r <= nr; r += SD_BLOCK) s_rp[r] = rowptr[i0 + r] - origin;
    for (int64_t idx = tid; idx < (int64_t)nr * K; idx += SD_BLOCK) {
        const int rr = (int)(idx % nr);
        const int64_t kk = idx / nr;
        s_a[rr * lds_ld + kk] = A[(i0 + rr) + kk * lda];
    }
    __syncthreads();

    const int p_lo = s_rp[0], p_hi = s_rp[nr];
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
        if (ONE) {
            if (VECB) {
                V16<T> bv[U];
#pragma unroll
                for (int u = 0; u < U; ++u) bv[u] = *reinterpret_cast<const V16<T> *>(B + j[u] * ldb + k1c);
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const V16<T> av = *reinterpret_cast<const V16<T> *>(arow[u] + k1c);
                    T d = T(0);
#pragma unroll
                    for (int e = 0; e < NE; ++e) d += av.v[e] * bv[u].v[e];
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
                    T out = alpha * dot[u];
                    if (mask) out = mask[p] * out;
                    if (!beta_zero) out += beta * Cval[p];
                    Cval[p] = out;
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
    const T *__restrict__ B, int64_t ldb, T beta, int beta_zero, T *Cval, const T *mask)
{
    const int64_t i = blockIdx.x;
    if (i >= m) return;
    const int g = threadIdx.x / SD_GROUP, q = threadIdx.x % SD_GROUP;
    const int64_t lo = (int64_t)rowptr[i] - origin, hi = (int64_t)rowptr[i + 1] - origin;
    for (int64_t p = lo + g; p < hi; p += SD_GROUPS) {
        const int64_t j = (int64_t)colind[p] - origin;
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

template <typename T>
int csr_sddmm(int64_t m, int64_t n, int64_t K, int64_t nnz, int32_t origin,
              const int32_t *rowptr, const int32_t *colind, T alpha, const T *A, int64_t lda,
              const T *B, int64_t ldb, T beta, T *Cval, const T *mask, jlust_stream_t stream)
{
    clear_error();
    if (m < 0 || n < 0 || K < 0 || nnz < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_sddmm: negative extent");
    if (m > INT32_MAX || n > INT32_MAX || nnz > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_sddmm: extents exceed the Int32 index range");
    if (int st = check_origin(origin)) return st;
    if (lda < (m > 0 ? m : 1) || ldb < (K > 0 ? K : 1))
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "csr_sddmm: leading dimensions too small (lda=%lld < m=%lld or ldb=%lld < K=%lld)",
                    (long long)lda, (long long)m, (long long)ldb, (long long)K);
    if ((m > 0 && !rowptr) || bad_ptr(colind, nnz) || bad_ptr(Cval, nnz) ||
        bad_ptr(A, (nnz > 0 && K > 0) ? m : 0) || bad_ptr(B, (nnz > 0 && K > 0) ? n : 0))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_sddmm: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (m == 0 || nnz == 0) return JLUST_STATUS_SUCCESS;
    hipStream_t s = (hipStream_t)stream;
    const int bz = beta == T(0);
    constexpr int N = V16<T>::N;
    const int64_t lds_ld = (K + N - 1) / N * N + N;       // padded, keeps rows 16-byte aligned
    int R = (int)((SD_LDS_BUDGET - 64 * sizeof(int32_t)) / (sizeof(T) * (size_t)lds_ld));
    if (R > 32) R = 32;
    if (R < 1) {
        hipLaunchKernelGGL((csr_sddmm_direct_kernel<T>), dim3((unsigned)m), dim3(SD_BLOCK), 0, s, m,
                           K, origin, rowptr, colind, alpha, A, lda, B, ldb, beta, bz, Cval, mask);
        return check_launch("csr_sddmm_direct_kernel");
    }
    const bool vecb = (K % N == 0) && (ldb % N == 0) && (((uintptr_t)B) % 16 == 0);
    const size_t smem = sizeof(T) * (size_t)R * (size_t)lds_ld + sizeof(int32_t) * (size_t)(R + 1);
    const dim3 grid((unsigned)((m + R - 1) / R));
    // Lane loads that cover K: G = the smallest power of two >= that, up to 8.
    const int64_t slices = vecb ? K / N : K;
#define JLUST_SD(V, G, U, ONE)                                                                        \
    hipLaunchKernelGGL((csr_sddmm_kernel<T, V, G, U, ONE>), grid, dim3(SD_BLOCK), smem, s, m, K, origin, \
                       rowptr, colind, alpha, A, lda, B, ldb, beta, bz, Cval, mask, R, lds_ld)
#define JLUST_SD_V(V)                                                                                 \
    do {                                                                                              \
        if (slices == 0) JLUST_SD(V, 8, 1, false);     /* K = 0: no loads of B at all */             \
        else if (slices <= 1) JLUST_SD(V, 1, 4, true);                                                \
        else if (slices <= 2) JLUST_SD(V, 2, 4, true);                                                \
        else if (slices <= 4) JLUST_SD(V, 4, 2, true);                                                \
        else if (slices <= 8) JLUST_SD(V, 8, 1, true);                                                \
        else JLUST_SD(V, 8, 1, false);                                                                \
    } while (0)
    if (vecb) JLUST_SD_V(true);
    else JLUST_SD_V(false);
#undef JLUST_SD_V
#undef JLUST_SD
    return check_launch("csr_sddmm_kernel");
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
