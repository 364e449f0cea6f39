/*
 * jlust_cpu.c -- CPU restatement of JLUST's EmitterBackend CPU path for the
 * sparse hot path (CSR/COO SpMV, CSR SpMM, CSR SDDMM, BSR SpMM via its CSR
 * expansion, CSR<->CSC/COO conversions).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the timed CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker.  The product (libjlust_hip.so and
 * the jlust_amd package) never calls it.
 *
 * JLUST is Julia; its CPU path is KernelAbstractions' CPU backend running the
 * "scalar walker" (one logical thread per outer fiber, 64 per work-group,
 * src/backends.jl:17,25,35).  Each output is accumulated sequentially from
 * zero in storage order, and Julia does not contract a*b+c into an FMA, so
 * this file must be compiled with -ffp-contract=off (see oracle/Makefile) to
 * reproduce the reference's rounding exactly.
 *
 * Parity pinning (tests/test_oracle.py):
 *   - the reference's own known-answer fixtures (test/test_emitter.jl:97-319,
 *     test/test_convert.jl:34-116), transcribed to tests/golden/;
 *   - scipy.sparse csr_matvec / csr_matvecs, whose per-output loop is the same
 *     sequential non-FMA sum from zero, so results must be bit-identical;
 *   - brute force in extended precision on tiny inputs, closed forms
 *     (identity / permutation / shifted diagonal) and invariants
 *     (SpMM column c == SpMV with B[:,c]; BSR == dense block product).
 *
 * Index convention: every index array is Int32 as stored by JLUST, with the
 * tensor's index origin (0 or 1) subtracted at use, like `_origin_off`
 * (ext/KernelAbstractionsExt/ops/_walker.jl:125-128).  Dense matrices are
 * column-major with a leading dimension, like Julia arrays.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* KernelAbstractions CPU work-group size (src/backends.jl:25). */
#define ORACLE_WG 64

static int clamp_threads(int nt) { return nt < 1 ? 1 : nt; }

/* ------------------------------------------------------------------------- */
/* CSR SpMV                                                                  */
/* ------------------------------------------------------------------------- */
/*
 * y = alpha*A*x (+ beta*y iff beta != 0).
 * Follows ext/KernelAbstractionsExt/ops/_walker.jl:123-132 (inner Compressed
 * walk, vs == 1: `for k in lo+1:hi; _acc += nz[k]*x[crd[k]-o+1]`) and the row
 * body of ext/KernelAbstractionsExt/ops/spmv.jl:154-169 (`_acc = zero(T)`,
 * then `y = alpha*acc` when beta == 0, else `alpha*acc + beta*y`).
 * alpha and beta arrive already cast to T (spmv.jl:377-378).
 */
#define DEF_CSR_SPMV(SUF, T)                                                   \
void oracle_csr_spmv_##SUF(int32_t m, int32_t origin, const int32_t *rowptr,   \
                           const int32_t *colind, const T *val, T alpha,       \
                           const T *x, T beta, T *y, int nthreads)             \
{                                                                              \
    const int zero_beta = (beta == (T)0);                                      \
    const int64_t nchunks = ((int64_t)m + ORACLE_WG - 1) / ORACLE_WG;          \
    _Pragma("omp parallel for schedule(static) num_threads(clamp_threads(nthreads))") \
    for (int64_t c = 0; c < nchunks; ++c) {                                    \
        int64_t r0 = c * ORACLE_WG, r1 = r0 + ORACLE_WG;                       \
        if (r1 > m) r1 = m;                                                    \
        for (int64_t i = r0; i < r1; ++i) {                                    \
            int64_t lo = (int64_t)rowptr[i] - origin;                          \
            int64_t hi = (int64_t)rowptr[i + 1] - origin;                      \
            T acc = (T)0;                                                      \
            for (int64_t k = lo; k < hi; ++k)                                  \
                acc += val[k] * x[colind[k] - origin];                         \
            if (zero_beta) y[i] = alpha * acc;                                 \
            else           y[i] = alpha * acc + beta * y[i];                   \
        }                                                                      \
    }                                                                          \
}
DEF_CSR_SPMV(f64, double)
DEF_CSR_SPMV(f32, float)

/*
 * Elementwise magnitude reference for the tolerance checks:
 *   absref[i] = |alpha| * sum_k |val[k]| * |x[col[k]]| + |beta| * |y0[i]|
 * computed in double whatever T is.  y0 may be NULL (beta term dropped).
 */
#define DEF_CSR_ABSREF(SUF, T)                                                 \
void oracle_csr_spmv_absref_##SUF(int32_t m, int32_t origin,                   \
                                  const int32_t *rowptr, const int32_t *colind,\
                                  const T *val, double alpha, const T *x,      \
                                  double beta, const T *y0, double *absref,    \
                                  int nthreads)                                \
{                                                                              \
    _Pragma("omp parallel for schedule(static) num_threads(clamp_threads(nthreads))") \
    for (int64_t i = 0; i < m; ++i) {                                          \
        double s = 0.0;                                                        \
        for (int64_t k = (int64_t)rowptr[i] - origin;                          \
             k < (int64_t)rowptr[i + 1] - origin; ++k)                         \
            s += fabs((double)val[k]) * fabs((double)x[colind[k] - origin]);   \
        s *= fabs(alpha);                                                      \
        if (y0) s += fabs(beta) * fabs((double)y0[i]);                         \
        absref[i] = s;                                                         \
    }                                                                          \
}
DEF_CSR_ABSREF(f64, double)
DEF_CSR_ABSREF(f32, float)

/* ------------------------------------------------------------------------- */
/* COO SpMV                                                                  */
/* ------------------------------------------------------------------------- */
/*
 * ext/KernelAbstractionsExt/ops/spmv.jl:407-448: y is first pre-scaled by beta
 * (filled with zero when beta == 0).  On the CPU backend (no warp shuffles)
 * identity transforms with alpha == 1 take `_coo_spmv_chunked!`
 * (spmv.jl:217-243): each logical thread owns 8 consecutive nonzeros,
 * accumulates locally and adds into y at every row change.  Otherwise the
 * generic walker adds `alpha * nz * x` per nonzero (spmv.jl:158-162).
 * The reference applies the adds with atomics from concurrent work-groups, so
 * their order is not fixed; this restatement applies them in ascending chunk
 * order (sequential), which is one of the reference's admissible orders.
 */
#define COO_CHUNK 8
#define DEF_COO_SPMV(SUF, T)                                                   \
void oracle_coo_spmv_##SUF(int64_t nnz, int32_t m, int32_t origin,             \
                           const int32_t *rows, const int32_t *cols,           \
                           const T *val, T alpha, const T *x, T beta, T *y)    \
{                                                                              \
    if (beta == (T)0) { for (int64_t i = 0; i < m; ++i) y[i] = (T)0; }         \
    else              { for (int64_t i = 0; i < m; ++i) y[i] *= beta; }        \
    if (alpha == (T)1) {                                                       \
        int64_t nchunks = (nnz + COO_CHUNK - 1) / COO_CHUNK;                   \
        for (int64_t t = 0; t < nchunks; ++t) {                                \
            int64_t lo = t * COO_CHUNK, hi = lo + COO_CHUNK;                   \
            if (hi > nnz) hi = nnz;                                            \
            int64_t cur = -1; T acc = (T)0;                                    \
            for (int64_t i = lo; i < hi; ++i) {                                \
                int64_t r = (int64_t)rows[i] - origin;                         \
                if (r != cur) {                                                \
                    if (cur >= 0) y[cur] += acc;                               \
                    cur = r; acc = (T)0;                                       \
                }                                                              \
                acc += val[i] * x[cols[i] - origin];                           \
            }                                                                  \
            if (cur >= 0) y[cur] += acc;                                       \
        }                                                                      \
    } else {                                                                   \
        for (int64_t i = 0; i < nnz; ++i)                                      \
            y[rows[i] - origin] += alpha * val[i] * x[cols[i] - origin];       \
    }                                                                          \
}
DEF_COO_SPMV(f64, double)
DEF_COO_SPMV(f32, float)

/* ------------------------------------------------------------------------- */
/* CSC SpMV (scatter mode)                                                   */
/* ------------------------------------------------------------------------- */
/*
 * y = beta*y (filled with zero when beta == 0), then for every column j in
 * order and every stored entry p of it in storage order:
 *   y[rowind[p]] += (alpha * val[p]) * x[j].
 * Follows the scatter branch of execute(::EmitterBackend, ::Op{:SpMV})
 * (ext/KernelAbstractionsExt/ops/spmv.jl:391-408: the pre-scale at :401 and
 * the launch with the dense outer level walking columns) and the scatter leaf
 * `@atomic _y[_y_idx] += _alpha * _nzval[_nnz_pos] * input_fn(_x[_x_idx])`
 * (spmv.jl:140-141; Julia evaluates alpha*val first).  The atomics' order is
 * not fixed in the reference; this restatement applies them sequentially in
 * storage order, one of its admissible orders.
 */
#define DEF_CSC_SPMV(SUF, T)                                                   \
void oracle_csc_spmv_##SUF(int32_t m, int32_t n, int32_t origin,               \
                           const int32_t *colptr, const int32_t *rowind,       \
                           const T *val, T alpha, const T *x, T beta, T *y)    \
{                                                                              \
    if (beta == (T)0) { for (int64_t i = 0; i < m; ++i) y[i] = (T)0; }         \
    else              { for (int64_t i = 0; i < m; ++i) y[i] *= beta; }        \
    for (int64_t j = 0; j < n; ++j)                                            \
        for (int64_t p = (int64_t)colptr[j] - origin;                          \
             p < (int64_t)colptr[j + 1] - origin; ++p)                         \
            y[rowind[p] - origin] += (alpha * val[p]) * x[j];                  \
}
DEF_CSC_SPMV(f64, double)
DEF_CSC_SPMV(f32, float)

/* ------------------------------------------------------------------------- */
/* CSR SpMM                                                                  */
/* ------------------------------------------------------------------------- */
/*
 * C = alpha*A*B + beta*C with B (n x k, ldb) and C (m x k, ldc) column-major.
 *
 * Strategy selection restates `_spmm_strategy` (spmm.jl:329-349) for a CSR
 * operand on the CPU backend, whose SM-count probe falls back to 80
 * (spmm.jl:91), giving the 2-D row threshold 192*80 = 15360 (spmm.jl:111-115):
 *   k <= 32: 2D if skip_empty_rows || m <= 15360 || nnz > 3*m, else NNZFirst;
 *   k >  32: Tiled (8-column strips) if k % 8 == 0, else ColFirst.
 * Every strategy forms each output as a sequential sum over the row's nonzeros
 * in storage order from zero(T) (spmm.jl:31-38, 137-148, 195-201, 272-279).
 * They differ only in the final write:
 *   2D / NNZFirst with beta == 0: C = alpha*acc            (write-only)
 *   2D / NNZFirst with beta != 0: C = alpha*acc + beta*C
 *   Tiled / ColFirst:             C = alpha*acc + beta*C   (C read even when
 *                                 beta == 0, spmm.jl:38,273-276)
 *   2D with skip_empty_rows: empty rows are left untouched (spmm.jl:203).
 * Returned value: the strategy id (0 ColFirst, 1 NNZFirst, 2 Tiled, 3 2D).
 * The loop nest below is the Tiled one (rows outer, 8-column strips, nonzeros
 * inner) for every strategy; the per-output arithmetic is identical.
 */
enum { SPMM_COLFIRST = 0, SPMM_NNZFIRST = 1, SPMM_TILED = 2, SPMM_2D = 3 };

int oracle_spmm_strategy(int64_t m, int64_t k, int64_t nnz, int skip_empty_rows)
{
    if (k <= 32) {
        if (skip_empty_rows || m <= 192 * 80 || nnz > 3 * m) return SPMM_2D;
        return SPMM_NNZFIRST;
    }
    if (k % 8 == 0) return SPMM_TILED;
    return SPMM_COLFIRST;
}

#define SPMM_TILE_K 8
#define DEF_CSR_SPMM(SUF, T)                                                   \
int oracle_csr_spmm_##SUF(int32_t m, int32_t origin, const int32_t *rowptr,    \
                          const int32_t *colind, const T *val, int64_t k,      \
                          T alpha, const T *B, int64_t ldb, T beta, T *C,      \
                          int64_t ldc, int skip_empty_rows, int nthreads)      \
{                                                                              \
    int64_t nnz = (int64_t)rowptr[m] - rowptr[0];                              \
    int strat = oracle_spmm_strategy(m, k, nnz, skip_empty_rows);              \
    int read_c = (strat == SPMM_TILED || strat == SPMM_COLFIRST) ||            \
                 beta != (T)0;                                                 \
    int guard = (strat == SPMM_2D) && skip_empty_rows;                         \
    const int64_t nchunks = ((int64_t)m + ORACLE_WG - 1) / ORACLE_WG;          \
    _Pragma("omp parallel for schedule(static) num_threads(clamp_threads(nthreads))") \
    for (int64_t ch = 0; ch < nchunks; ++ch) {                                 \
        int64_t r0 = ch * ORACLE_WG, r1 = r0 + ORACLE_WG;                      \
        if (r1 > m) r1 = m;                                                    \
        for (int64_t i = r0; i < r1; ++i) {                                    \
            int64_t lo = (int64_t)rowptr[i] - origin;                          \
            int64_t hi = (int64_t)rowptr[i + 1] - origin;                      \
            if (guard && !(lo < hi)) continue;                                 \
            for (int64_t t0 = 0; t0 < k; t0 += SPMM_TILE_K) {                  \
                int64_t tw = k - t0 < SPMM_TILE_K ? k - t0 : SPMM_TILE_K;      \
                T acc[SPMM_TILE_K];                                            \
                for (int c = 0; c < SPMM_TILE_K; ++c) acc[c] = (T)0;           \
                for (int64_t p = lo; p < hi; ++p) {                            \
                    int64_t j = (int64_t)colind[p] - origin;                   \
                    T v = val[p];                                              \
                    for (int64_t c = 0; c < tw; ++c)                           \
                        acc[c] += v * B[j + (t0 + c) * ldb];                   \
                }                                                              \
                for (int64_t c = 0; c < tw; ++c) {                             \
                    T *dst = &C[i + (t0 + c) * ldc];                           \
                    if (read_c) *dst = alpha * acc[c] + beta * *dst;           \
                    else        *dst = alpha * acc[c];                         \
                }                                                              \
            }                                                                  \
        }                                                                      \
    }                                                                          \
    return strat;                                                              \
}
DEF_CSR_SPMM(f64, double)
DEF_CSR_SPMM(f32, float)

/* |alpha| * |A| * |B| + |beta| * |C0| elementwise, in double (m x k, ld = m). */
#define DEF_SPMM_ABSREF(SUF, T)                                                \
void oracle_csr_spmm_absref_##SUF(int32_t m, int32_t origin,                   \
                                  const int32_t *rowptr, const int32_t *colind,\
                                  const T *val, int64_t k, double alpha,       \
                                  const T *B, int64_t ldb, double beta,        \
                                  const T *C0, int64_t ldc, double *absref,    \
                                  int nthreads)                                \
{                                                                              \
    _Pragma("omp parallel for schedule(static) num_threads(clamp_threads(nthreads))") \
    for (int64_t i = 0; i < m; ++i) {                                          \
        for (int64_t c = 0; c < k; ++c) {                                      \
            double s = 0.0;                                                    \
            for (int64_t p = (int64_t)rowptr[i] - origin;                      \
                 p < (int64_t)rowptr[i + 1] - origin; ++p)                     \
                s += fabs((double)val[p]) *                                    \
                     fabs((double)B[(colind[p] - origin) + c * ldb]);          \
            s *= fabs(alpha);                                                  \
            if (C0) s += fabs(beta) * fabs((double)C0[i + c * ldc]);           \
            absref[i + c * (int64_t)m] = s;                                    \
        }                                                                      \
    }                                                                          \
}
DEF_SPMM_ABSREF(f64, double)
DEF_SPMM_ABSREF(f32, float)

/* ------------------------------------------------------------------------- */
/* COO and CSC SpMM (atomic / scatter modes)                                 */
/* ------------------------------------------------------------------------- */
/*
 * C = alpha*A*B + beta*C for a COO A.  execute(::EmitterBackend, ::Op{:SpMM})
 * pre-scales C by beta for COO-like and scatter formats, filling zero when
 * beta == 0 (ext/KernelAbstractionsExt/ops/spmm.jl:412-416), then runs COO as
 * ColFirst (spmm.jl:331-335): one thread per stored entry loops over the k
 * columns of B with the atomic leaf
 *   @atomic C[row, col] += alpha * nzval[p] * B[x, col]     (spmm.jl:32-33)
 * (Julia evaluates alpha*nzval first).  The atomics' order is not fixed in the
 * reference; this restatement applies them sequentially, entry by entry in
 * storage order, then column by column, one of its admissible orders.
 */
#define DEF_COO_SPMM(SUF, T)                                                   \
void oracle_coo_spmm_##SUF(int64_t nnz, int32_t m, int32_t origin,             \
                           const int32_t *rows, const int32_t *cols,           \
                           const T *val, int64_t k, T alpha, const T *B,       \
                           int64_t ldb, T beta, T *C, int64_t ldc)             \
{                                                                              \
    for (int64_t c = 0; c < k; ++c)                                            \
        for (int64_t i = 0; i < m; ++i) {                                      \
            T *o = &C[i + c * ldc];                                            \
            *o = beta == (T)0 ? (T)0 : *o * beta;                              \
        }                                                                      \
    for (int64_t p = 0; p < nnz; ++p) {                                        \
        int64_t r = (int64_t)rows[p] - origin, j = (int64_t)cols[p] - origin;  \
        T av = alpha * val[p];                                                 \
        for (int64_t c = 0; c < k; ++c)                                        \
            C[r + c * ldc] += av * B[j + c * ldb];                             \
    }                                                                          \
}
DEF_COO_SPMM(f64, double)
DEF_COO_SPMM(f32, float)

/*
 * CSC A (colptr[n+1], rowind): the same pre-scale, then the walker's scatter
 * direction (_walker.jl:41-66: the dense outer level walks the input column
 * j, the compressed inner level binds the output row) with the scatter leaf
 *   @atomic C[rowind[p], col] += alpha * nzval[p] * B[j, col]  (spmm.jl:18-19)
 * for every strategy _spmm_strategy picks under scatter (spmm.jl:329-349).
 * Applied sequentially: column j in order, its entries in storage order,
 * then the k columns of B.
 */
#define DEF_CSC_SPMM(SUF, T)                                                   \
void oracle_csc_spmm_##SUF(int32_t m, int32_t n, int32_t origin,               \
                           const int32_t *colptr, const int32_t *rowind,       \
                           const T *val, int64_t k, T alpha, const T *B,       \
                           int64_t ldb, T beta, T *C, int64_t ldc)             \
{                                                                              \
    for (int64_t c = 0; c < k; ++c)                                            \
        for (int64_t i = 0; i < m; ++i) {                                      \
            T *o = &C[i + c * ldc];                                            \
            *o = beta == (T)0 ? (T)0 : *o * beta;                              \
        }                                                                      \
    for (int64_t j = 0; j < n; ++j)                                            \
        for (int64_t p = (int64_t)colptr[j] - origin;                          \
             p < (int64_t)colptr[j + 1] - origin; ++p) {                       \
            int64_t r = (int64_t)rowind[p] - origin;                           \
            T av = alpha * val[p];                                             \
            for (int64_t c = 0; c < k; ++c)                                    \
                C[r + c * ldc] += av * B[j + c * ldb];                         \
        }                                                                      \
}
DEF_CSC_SPMM(f64, double)
DEF_CSC_SPMM(f32, float)

/* ------------------------------------------------------------------------- */
/* CSR SDDMM                                                                 */
/* ------------------------------------------------------------------------- */
/*
 * C.val[p] = alpha * sum_{kk<K} A[i,kk]*B[kk,j] + beta*C.val[p] for every
 * stored (i, j) of C.  A is m x K (lda), B is K x n (ldb), both column-major.
 * Follows ext/KernelAbstractionsExt/ops/sddmm.jl:23-30 (`_dot = zero(T)`,
 * sequential k loop, then the write, which always reads C.val) and the launch
 * at sddmm.jl:49-62 (alpha, beta cast to T).
 * The benchmark's masked form out_ij = S_ij * dot(A[i,:], B[:,j]) is this
 * operator with alpha = 1, beta = 0, followed by a multiply by the stored
 * mask value: when `mask` is non-NULL the write is
 *   C.val[p] = mask[p] * (alpha*dot) + beta*C.val[p].
 */
#define DEF_SDDMM(SUF, T)                                                      \
void oracle_csr_sddmm_##SUF(int32_t m, int32_t origin, const int32_t *rowptr,  \
                            const int32_t *colind, int64_t K, T alpha,         \
                            const T *A, int64_t lda, const T *B, int64_t ldb,  \
                            T beta, T *Cval, const T *mask, int nthreads)      \
{                                                                              \
    const int64_t nchunks = ((int64_t)m + ORACLE_WG - 1) / ORACLE_WG;          \
    _Pragma("omp parallel for schedule(static) num_threads(clamp_threads(nthreads))") \
    for (int64_t ch = 0; ch < nchunks; ++ch) {                                 \
        int64_t r0 = ch * ORACLE_WG, r1 = r0 + ORACLE_WG;                      \
        if (r1 > m) r1 = m;                                                    \
        for (int64_t i = r0; i < r1; ++i) {                                    \
            for (int64_t p = (int64_t)rowptr[i] - origin;                      \
                 p < (int64_t)rowptr[i + 1] - origin; ++p) {                   \
                int64_t j = (int64_t)colind[p] - origin;                       \
                T dot = (T)0;                                                  \
                for (int64_t kk = 0; kk < K; ++kk)                             \
                    dot += A[i + kk * lda] * B[kk + j * ldb];                  \
                T term = alpha * dot;                                          \
                if (mask) term = mask[p] * term;                               \
                Cval[p] = term + beta * Cval[p];                               \
            }                                                                  \
        }                                                                      \
    }                                                                          \
}
DEF_SDDMM(f64, double)
DEF_SDDMM(f32, float)

/*
 * SDDMM with a COO mask (coo_tensor storage, src/interop.jl:248-260): the
 * same per-entry arithmetic as above for every stored (rows[p], cols[p]) in
 * storage order -- the walker visits each stored entry once whatever its outer
 * level (sddmm.jl:23-30 is format-generic; reference answer
 * test/test_emitter.jl:289-307).
 */
#define DEF_COO_SDDMM(SUF, T)                                                  \
void oracle_coo_sddmm_##SUF(int64_t nnz, int32_t origin, const int32_t *rows,  \
                            const int32_t *cols, int64_t K, T alpha,           \
                            const T *A, int64_t lda, const T *B, int64_t ldb,  \
                            T beta, T *Cval, const T *mask)                    \
{                                                                              \
    for (int64_t p = 0; p < nnz; ++p) {                                        \
        int64_t i = (int64_t)rows[p] - origin, j = (int64_t)cols[p] - origin;  \
        T dot = (T)0;                                                          \
        for (int64_t kk = 0; kk < K; ++kk)                                     \
            dot += A[i + kk * lda] * B[kk + j * ldb];                          \
        T term = alpha * dot;                                                  \
        if (mask) term = mask[p] * term;                                       \
        Cval[p] = term + beta * Cval[p];                                       \
    }                                                                          \
}
DEF_COO_SDDMM(f64, double)
DEF_COO_SDDMM(f32, float)

/* |alpha| * |mask| * sum|A||B| + |beta| |C0| per stored entry, in double. */
#define DEF_SDDMM_ABSREF(SUF, T)                                               \
void oracle_csr_sddmm_absref_##SUF(int32_t m, int32_t origin,                  \
                                   const int32_t *rowptr,                      \
                                   const int32_t *colind, int64_t K,           \
                                   double alpha, const T *A, int64_t lda,      \
                                   const T *B, int64_t ldb, double beta,       \
                                   const T *C0, const T *mask, double *absref, \
                                   int nthreads)                               \
{                                                                              \
    _Pragma("omp parallel for schedule(static) num_threads(clamp_threads(nthreads))") \
    for (int64_t i = 0; i < m; ++i) {                                          \
        for (int64_t p = (int64_t)rowptr[i] - origin;                          \
             p < (int64_t)rowptr[i + 1] - origin; ++p) {                       \
            int64_t j = (int64_t)colind[p] - origin;                           \
            double s = 0.0;                                                    \
            for (int64_t kk = 0; kk < K; ++kk)                                 \
                s += fabs((double)A[i + kk * lda]) *                           \
                     fabs((double)B[kk + j * ldb]);                            \
            s *= fabs(alpha);                                                  \
            if (mask) s *= fabs((double)mask[p]);                              \
            if (C0) s += fabs(beta) * fabs((double)C0[p]);                     \
            absref[p] = s;                                                     \
        }                                                                      \
    }                                                                          \
}
DEF_SDDMM_ABSREF(f64, double)
DEF_SDDMM_ABSREF(f32, float)

/* ------------------------------------------------------------------------- */
/* BSR -> CSR expansion (bit-exact) and BSR SpMM                             */
/* ------------------------------------------------------------------------- */
/*
 * JLUST's BSR layout (Formats.BSRRight/BSRLeft, src/named_formats.jl:106-128;
 * storage per the CuSparseMatrixBSR adapter, ext/CUDAExt/CUDAExt.jl:144-156):
 * block-row pointers and block-column indices at level 2, values block-major,
 * row-major inside a block for BSRRight (dir 'R') and column-major for
 * BSRLeft.  The reference has no sound BSR compute path (its walker never
 * advances through the inner Dense levels), so the operator is pinned by its
 * mathematical definition: expand to CSR and run the CSR path.
 * Expansion (b1 x b2 blocks): scalar row b1*R + r lists, for each stored block
 * q of block-row R in storage order, columns b2*bcol[q] + s for s = 0..b2-1
 * (ascending when the block-columns are sorted).  Every stored entry is kept
 * (explicit zeros too).  Output CSR uses the input's origin.  rowptr has
 * mb*b1 + 1 entries, colind and val nnzb*b1*b2 entries.  Block q's entry
 * (r, s) is bval[q*b1*b2 + r*b2 + s] for row-major blocks and
 * bval[q*b1*b2 + s*b1 + r] for column-major ones.
 */
#define DEF_BSR2CSR(SUF, T)                                                    \
void oracle_bsr_to_csr_##SUF(int32_t mb, int32_t b1, int32_t b2,               \
                             int32_t origin, const int32_t *browptr,           \
                             const int32_t *bcolind, const T *bval,            \
                             int row_major_blocks, int32_t *rowptr,            \
                             int32_t *colind, T *val)                          \
{                                                                              \
    int64_t bb = (int64_t)b1 * b2;                                             \
    rowptr[0] = origin;                                                        \
    for (int64_t R = 0; R < mb; ++R) {                                         \
        int64_t q0 = (int64_t)browptr[R] - origin;                             \
        int64_t q1 = (int64_t)browptr[R + 1] - origin;                         \
        int64_t nb_row = q1 - q0;                                              \
        for (int64_t r = 0; r < b1; ++r) {                                     \
            int64_t row = R * b1 + r;                                          \
            int64_t base = (int64_t)rowptr[row] - origin;                      \
            int64_t w = 0;                                                     \
            for (int64_t q = q0; q < q1; ++q) {                                \
                int64_t bc = (int64_t)bcolind[q] - origin;                     \
                for (int64_t s = 0; s < b2; ++s) {                             \
                    colind[base + w] = (int32_t)(bc * b2 + s + origin);        \
                    val[base + w] = row_major_blocks ? bval[q * bb + r * b2 + s] \
                                                     : bval[q * bb + s * b1 + r]; \
                    ++w;                                                       \
                }                                                              \
            }                                                                  \
            rowptr[row + 1] = (int32_t)(rowptr[row] + nb_row * b2);            \
        }                                                                      \
    }                                                                          \
}
DEF_BSR2CSR(f64, double)
DEF_BSR2CSR(f32, float)

/* ------------------------------------------------------------------------- */
/* Conversions (bit-exact): CSR -> CSC, CSR -> COO, COO -> CSR               */
/* ------------------------------------------------------------------------- */
/*
 * src/convert.jl:302-388: decompose in storage order, drop explicit zeros
 * (convert.jl:316), sort by the target's level coordinates (a stable sort,
 * `_lexsort_cols` convert.jl:419-424), then count-then-fill pos/crd
 * (TensorComposer convert.jl:271-292).  The output keeps the source origin:
 * pos and crd are shifted by it (convert.jl:365-380).
 * A stable counting sort on the target's outer coordinate over entries already
 * sorted by the inner coordinate gives the same order as the lexicographic
 * sort, which is how the CSR -> CSC case is done here.
 * Return value: the number of entries kept (nnz after dropping zeros).
 */
#define DEF_CSR2CSC(SUF, T)                                                    \
int64_t oracle_csr_to_csc_##SUF(int32_t m, int32_t n, int32_t origin,          \
                                const int32_t *rowptr, const int32_t *colind,  \
                                const T *val, int32_t *colptr,                 \
                                int32_t *rowind, T *cval)                      \
{                                                                              \
    int64_t *cnt = (int64_t *)calloc((size_t)n + 1, sizeof(int64_t));          \
    for (int64_t i = 0; i < m; ++i)                                            \
        for (int64_t p = (int64_t)rowptr[i] - origin;                          \
             p < (int64_t)rowptr[i + 1] - origin; ++p)                         \
            if (val[p] != (T)0) cnt[colind[p] - origin + 1]++;                 \
    for (int64_t j = 0; j < n; ++j) cnt[j + 1] += cnt[j];                      \
    int64_t nkeep = cnt[n];                                                    \
    for (int64_t j = 0; j <= n; ++j) colptr[j] = (int32_t)(cnt[j] + origin);   \
    for (int64_t i = 0; i < m; ++i)                                            \
        for (int64_t p = (int64_t)rowptr[i] - origin;                          \
             p < (int64_t)rowptr[i + 1] - origin; ++p) {                       \
            if (val[p] == (T)0) continue;                                      \
            int64_t j = colind[p] - origin;                                    \
            int64_t dst = cnt[j]++;                                            \
            rowind[dst] = (int32_t)(i + origin);                               \
            cval[dst] = val[p];                                                \
        }                                                                      \
    free(cnt);                                                                 \
    return nkeep;                                                              \
}
DEF_CSR2CSC(f64, double)
DEF_CSR2CSC(f32, float)

/*
 * CSR -> COO: level 1 (rows, compressed non-unique) gets pos = [0, nnz] (+origin)
 * and crd = row of each entry; level 2 crd = column (test/test_convert.jl:62-79).
 * The source is already sorted by (row, col) when its columns are sorted.
 */
#define DEF_CSR2COO(SUF, T)                                                    \
int64_t oracle_csr_to_coo_##SUF(int32_t m, int32_t origin,                     \
                                const int32_t *rowptr, const int32_t *colind,  \
                                const T *val, int32_t *pos, int32_t *rows,     \
                                int32_t *cols, T *cval)                        \
{                                                                              \
    int64_t w = 0;                                                             \
    for (int64_t i = 0; i < m; ++i)                                            \
        for (int64_t p = (int64_t)rowptr[i] - origin;                          \
             p < (int64_t)rowptr[i + 1] - origin; ++p) {                       \
            if (val[p] == (T)0) continue;                                      \
            rows[w] = (int32_t)(i + origin);                                   \
            cols[w] = colind[p];                                               \
            cval[w] = val[p];                                                  \
            ++w;                                                               \
        }                                                                      \
    pos[0] = origin;                                                           \
    pos[1] = (int32_t)(w + origin);                                            \
    return w;                                                                  \
}
DEF_CSR2COO(f64, double)
DEF_CSR2COO(f32, float)

/*
 * COO -> CSR: entries sorted by (row, col) with a stable sort (duplicates keep
 * their storage order), explicit zeros dropped, rowptr by count-then-fill.
 * Stable two-pass counting sort: by column, then by row.
 */
#define DEF_COO2CSR(SUF, T)                                                    \
int64_t oracle_coo_to_csr_##SUF(int64_t nnz, int32_t m, int32_t n,             \
                                int32_t origin, const int32_t *rows,           \
                                const int32_t *cols, const T *val,             \
                                int32_t *rowptr, int32_t *colind, T *cval)     \
{                                                                              \
    int64_t *idx = (int64_t *)malloc(sizeof(int64_t) * (size_t)(nnz + 1));    \
    int64_t *tmp = (int64_t *)malloc(sizeof(int64_t) * (size_t)(nnz + 1));    \
    int64_t *cc = (int64_t *)calloc((size_t)n + 1, sizeof(int64_t));           \
    int64_t *rc = (int64_t *)calloc((size_t)m + 1, sizeof(int64_t));           \
    int64_t nk = 0;                                                            \
    for (int64_t p = 0; p < nnz; ++p)                                          \
        if (val[p] != (T)0) { idx[nk++] = p; cc[cols[p] - origin + 1]++; }     \
    for (int64_t j = 0; j < n; ++j) cc[j + 1] += cc[j];                        \
    for (int64_t t = 0; t < nk; ++t) tmp[cc[cols[idx[t]] - origin]++] = idx[t];\
    for (int64_t t = 0; t < nk; ++t) rc[rows[tmp[t]] - origin + 1]++;          \
    for (int64_t i = 0; i < m; ++i) rc[i + 1] += rc[i];                        \
    for (int64_t i = 0; i <= m; ++i) rowptr[i] = (int32_t)(rc[i] + origin);    \
    for (int64_t t = 0; t < nk; ++t) {                                         \
        int64_t p = tmp[t];                                                    \
        int64_t dst = rc[rows[p] - origin]++;                                  \
        colind[dst] = cols[p];                                                 \
        cval[dst] = val[p];                                                    \
    }                                                                          \
    free(idx); free(tmp); free(cc); free(rc);                                   \
    return nk;                                                                 \
}
DEF_COO2CSR(f64, double)
DEF_COO2CSR(f32, float)

int oracle_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
