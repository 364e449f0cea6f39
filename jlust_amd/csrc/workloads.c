/*
 * workloads.c -- deterministic synthetic inputs for the five benchmark
 * configurations (CSR SpMV uniform / power-law, CSR SpMM, CSR SDDMM, banded
 * BSR SpMM).  Host code, OpenMP-parallel, and independent of the thread count:
 * every row draws from its own xoshiro256** stream seeded from
 * (seed, tag, row) through SplitMix64, and dense arrays use a counter-based
 * hash of (seed, tag, linear index).
 *
 * The reference ships no generator for these shapes (its random_sparse in
 * benchmark/bench_formats.jl:21-33 uses another distribution), so the recipes
 * here are this build's own:
 *   - columns per row: distinct, uniform over the row's candidate range
 *     (Floyd's sampling for short rows, sample-sort-dedupe top-up for long
 *     ones), then sorted ascending;
 *   - uniform [-1, 1] = 2*u - 1 with u a 53-bit uniform;
 *   - N(0, 1) by Box-Muller in double (cast to float for fp32 arrays);
 *   - power-law row lengths: L = u^(-1/alpha) (Pareto, x_m = 1) clamped to
 *     [lmin, lmax], rescaled so the mean is `mean`, rounded, re-clamped.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint64_t splitmix64(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline uint64_t mix3(uint64_t seed, uint64_t tag, uint64_t idx)
{
    uint64_t s = seed * 0xD1B54A32D192ED03ull ^ tag * 0xABC98388FB8FAC03ull;
    s ^= idx * 0x8CB92BA72F3D8DD7ull;
    (void)splitmix64(&s);
    return splitmix64(&s);
}

typedef struct { uint64_t s[4]; } xoshiro;

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static inline uint64_t xo_next(xoshiro *r)
{
    uint64_t *s = r->s;
    uint64_t res = rotl(s[1] * 5, 7) * 9;
    uint64_t t = s[1] << 17;
    s[2] ^= s[0]; s[3] ^= s[1]; s[1] ^= s[2]; s[0] ^= s[3];
    s[2] ^= t; s[3] = rotl(s[3], 45);
    return res;
}

static inline void xo_seed(xoshiro *r, uint64_t seed, uint64_t tag, uint64_t row)
{
    uint64_t s = mix3(seed, tag, row);
    for (int i = 0; i < 4; ++i) r->s[i] = splitmix64(&s);
}

static inline double u53(uint64_t h) { return (double)(h >> 11) * 0x1.0p-53; }

/* uniform integer in [0, bound) by multiply-shift (bias < 2^-40 here). */
static inline uint64_t below(xoshiro *r, uint64_t bound)
{
    return (uint64_t)(((unsigned __int128)xo_next(r) * bound) >> 64);
}

static int nthr(int nt) { return nt < 1 ? 1 : nt; }

/* ---------------------------- dense arrays ------------------------------ */

void wl_uniform_f64(uint64_t seed, uint64_t tag, int64_t count, double lo,
                    double hi, double *out, int nthreads)
{
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
    for (int64_t i = 0; i < count; ++i)
        out[i] = lo + (hi - lo) * u53(mix3(seed, tag, (uint64_t)i));
}

void wl_uniform_f32(uint64_t seed, uint64_t tag, int64_t count, double lo,
                    double hi, float *out, int nthreads)
{
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
    for (int64_t i = 0; i < count; ++i)
        out[i] = (float)(lo + (hi - lo) * u53(mix3(seed, tag, (uint64_t)i)));
}

static inline double normal_at(uint64_t seed, uint64_t tag, uint64_t i)
{
    double u1 = u53(mix3(seed, tag, 2 * i)) + 0x1.0p-54;      /* (0, 1) */
    double u2 = u53(mix3(seed, tag, 2 * i + 1));
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

void wl_normal_f64(uint64_t seed, uint64_t tag, int64_t count, double *out,
                   int nthreads)
{
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
    for (int64_t i = 0; i < count; ++i) out[i] = normal_at(seed, tag, (uint64_t)i);
}

void wl_normal_f32(uint64_t seed, uint64_t tag, int64_t count, float *out,
                   int nthreads)
{
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
    for (int64_t i = 0; i < count; ++i)
        out[i] = (float)normal_at(seed, tag, (uint64_t)i);
}

/* --------------------------- row lengths -------------------------------- */

/*
 * Pareto(alpha, x_m = 1) row lengths clamped to [lmin, lmax] and rescaled to
 * the given mean.  Returns the total (nnz).
 */
int64_t wl_pareto_rowlens(int64_t m, double alpha, int64_t lmin, int64_t lmax,
                          double mean, uint64_t seed, int32_t *len,
                          int nthreads)
{
    double *xs = (double *)malloc(sizeof(double) * (size_t)(m > 0 ? m : 1));
#pragma omp parallel for schedule(static) num_threads(nthr(nthreads))
    for (int64_t i = 0; i < m; ++i) {
        double u = 1.0 - u53(mix3(seed, 0x5041524554ull, (uint64_t)i)); /* (0,1] */
        double x = pow(u, -1.0 / alpha);
        if (x < (double)lmin) x = (double)lmin;
        if (x > (double)lmax) x = (double)lmax;
        xs[i] = x;
    }
    double sum = 0.0;
    for (int64_t i = 0; i < m; ++i) sum += xs[i];   /* fixed order */
    double scale = sum > 0 ? mean * (double)m / sum : 0.0;
    int64_t total = 0;
    for (int64_t i = 0; i < m; ++i) {
        int64_t L = llround(xs[i] * scale);
        if (L < 1) L = 1;
        if (L < lmin) L = lmin;
        if (L > lmax) L = lmax;
        len[i] = (int32_t)L;
        total += L;
    }
    free(xs);
    return total;
}

/* ------------------------------ columns --------------------------------- */

static int cmp_i64(const void *a, const void *b)
{
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    return (x > y) - (x < y);
}

static int64_t sort_unique(int64_t *v, int64_t n)
{
    if (n <= 1) return n;
    qsort(v, (size_t)n, sizeof(int64_t), cmp_i64);
    int64_t w = 1;
    for (int64_t i = 1; i < n; ++i)
        if (v[i] != v[w - 1]) v[w++] = v[i];
    return w;
}

/* k distinct values of [0, N) into out (sorted).  scratch holds >= 2k. */
static void sample_distinct(xoshiro *r, int64_t N, int64_t k, int64_t *out,
                            int64_t *scratch)
{
    if (k <= 64) {                             /* Floyd's algorithm */
        int64_t c = 0;
        for (int64_t j = N - k; j < N; ++j) {
            int64_t t = (int64_t)below(r, (uint64_t)(j + 1));
            int dup = 0;
            for (int64_t q = 0; q < c; ++q) if (out[q] == t) { dup = 1; break; }
            out[c++] = dup ? j : t;
        }
        sort_unique(out, c);
        return;
    }
    int64_t have = 0;
    while (have < k) {                          /* sample, sort, dedupe, top up */
        int64_t need = k - have;
        memcpy(scratch, out, sizeof(int64_t) * (size_t)have);
        for (int64_t q = 0; q < need; ++q)
            scratch[have + q] = (int64_t)below(r, (uint64_t)N);
        int64_t u = sort_unique(scratch, have + need);
        memcpy(out, scratch, sizeof(int64_t) * (size_t)u);
        have = u;
    }
}

/*
 * Fill colind for a CSR pattern whose rowptr (with origin) is given.  Row r
 * draws its distinct columns from [lo, hi): [0, n) when band < 0, else
 * [max(0, r - band), min(n, r + band + 1)).  Written with the origin added.
 */
int wl_fill_columns(int64_t m, int64_t n, const int32_t *rowptr,
                    int32_t origin, int64_t band, uint64_t seed,
                    int32_t *colind, int nthreads)
{
    int bad = 0;
    int64_t maxlen = 0;
    for (int64_t i = 0; i < m; ++i) {
        int64_t L = (int64_t)rowptr[i + 1] - rowptr[i];
        if (L > maxlen) maxlen = L;
    }
#pragma omp parallel num_threads(nthr(nthreads)) reduction(| : bad)
    {
        int64_t *buf = (int64_t *)malloc(sizeof(int64_t) * (size_t)(3 * maxlen + 8));
        int64_t *scr = buf + maxlen + 4;
#pragma omp for schedule(dynamic, 1024)
        for (int64_t i = 0; i < m; ++i) {
            int64_t L = (int64_t)rowptr[i + 1] - rowptr[i];
            int64_t lo = 0, hi = n;
            if (band >= 0) {
                lo = i - band < 0 ? 0 : i - band;
                hi = i + band + 1 > n ? n : i + band + 1;
            }
            if (L > hi - lo) { bad = 1; continue; }
            xoshiro r;
            xo_seed(&r, seed, 0x434F4C53ull, (uint64_t)i);
            sample_distinct(&r, hi - lo, L, buf, scr);
            int32_t *dst = colind + ((int64_t)rowptr[i] - origin);
            for (int64_t q = 0; q < L; ++q) dst[q] = (int32_t)(buf[q] + lo + origin);
        }
        free(buf);
    }
    return bad ? -1 : 0;
}
