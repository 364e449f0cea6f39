// spmv_binned.hip -- CSR SpMV through an LDS-binned layout, for prepared plans
// whose x is far larger than an XCD's L2 and whose columns are scattered.
//
// The per-row arithmetic is that of the reference's CSR SpMV,
// y[i] = alpha * sum_k val[k] * x[col[k]] (+ beta * y[i])
// (ext/KernelAbstractionsExt/ops/spmv.jl:154-169, _walker.jl:123-132); only the
// association of the row sum differs: it is summed per column slice, and the
// slice sums are added in slice order (deterministic run to run).
//
// Why: a random 8-byte gather of x from HBM or the MALL costs a whole line and
// queues on the L1/L2 miss capacity; even x cut into eight 4 MB slices, one per
// XCD L2, gathers at only ~190 G/s.  Here no gather ever leaves a CU's LDS:
//
//   slice pass (G workgroups per column slice c of W columns, W*sizeof(T) <=
//   128 KB of LDS; G = 1 unless x is small, see geometry()): x[cW, (c+1)W) is
//   copied into each workgroup's LDS; the slice's entries,
//   stored slice-major and inside a slice in (row bin, row, k) order, are
//   streamed once (value + 16-bit local column), multiplied by their x from LDS
//   and summed per row with a wave64 segmented scan.  Each (row, slice) pair
//   with entries yields one partial sum, written contiguously.
//
//   bin pass (one workgroup per bin b of H rows, H*sizeof(T) <= 128 KB of
//   LDS): the partials of bin b come in S runs, one per slice, each run sorted
//   by row with every row at most once.  Runs are added into an LDS copy of
//   y[bH, (b+1)H) in slice order, a workgroup barrier between runs (so no two
//   adds to one row ever race), and y is written once.
//
// HBM bytes per entry: value + 2-byte column, then a partial (written, read)
// and its 2-byte row: about 28 B for fp64 against 12 B + a 128-byte line per
// missed gather for the plain layout.  The partial of a (row, slice) pair with
// several entries covers all of them, so long rows cost less.
//
// Layout build (once per plan, on the device): row of each entry by a prefix
// count of row starts, key = slice * B + bin, a stable radix sort of the keys
// (entry order inside a run stays the CSR order), the "last entry of a partial"
// flags, their prefix count (= partial indices), run and chunk boundaries.
#include <algorithm>
#include <cstdlib>
#include <vector>

#include <rocprim/device/device_radix_sort.hpp>

#include "spmv_binned.hpp"
#include "wave.hpp"

namespace jlust {
namespace {

constexpr int BN_THREADS = 1024;
constexpr int BN_WAVES = BN_THREADS / 64;
constexpr int BN_LDS = 128 * 1024;       // x slice / y bin in LDS
constexpr int BN_SMAX = 1024;            // slices (the bin pass keeps two run bounds per slice in LDS)
constexpr int64_t BN_MAX_RUNS = (int64_t)1 << 22;
constexpr uint32_t BN_END = 0x8000u;     // scol flag: last entry of its partial
constexpr uint32_t BN_COL = 0x7fffu;

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }
size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Slice width / bin height.  Bins: about one per CU, at most BN_LDS bytes of
// y each.  Slices: about one per CU while that needs slices of nearly BN_LDS
// bytes anyway; when x is smaller (its widest slices number at most half the
// CUs), the slices are as wide as LDS allows and G = cu / S workgroups share
// each one.  Fewer slices mean fewer partial sums (a row's entries fall into
// fewer slices) and a shorter bin pass (one step per slice), for the price of
// each workgroup copying a whole slice from L2: a 1M x 1M matrix with 16 random
// columns per row (f64) runs in 92 us against 134 us with one slice per CU.
bool geometry(int value_type, int64_t m, int64_t n, int64_t nnz, int cu, int32_t *W, int32_t *S,
              int32_t *G, int32_t *H, int32_t *B)
{
    if (m <= 0 || n <= 0 || nnz <= 0 || nnz > (int64_t)INT32_MAX - 4096) return false;
    if (cu < 1) cu = 1;
    const int64_t tsz = value_type == 0 ? 8 : 4;
    const int64_t wmax = BN_LDS / tsz;    // <= 32768: the column fits 15 bits
    int64_t w = std::min(wmax, round_up((n + cu - 1) / cu, 64));
    const int64_t swide = (n + wmax - 1) / wmax;
    if (swide * 2 <= cu) w = round_up((n + swide - 1) / swide, 64);   // <= wmax, a multiple of 64
    const int64_t s = (n + w - 1) / w;
    const int64_t h = std::min(wmax, round_up((m + cu - 1) / cu, 64));
    const int64_t b = (m + h - 1) / h;
    if (s > BN_SMAX || s * b > BN_MAX_RUNS) return false;
    *W = (int32_t)w;
    *S = (int32_t)s;
    *G = (int32_t)std::max<int64_t>(1, cu / s);
    *H = (int32_t)h;
    *B = (int32_t)b;
    return true;
}

template <typename T>
__device__ __forceinline__ T readlane63(T v)
{
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int32_t, v), 63));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int32_t)u, 63);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int32_t)(u >> 32), 63);
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    }
}

// ---- slice pass.  Workgroup g of slice c = blockIdx / G; wave w streams chunk
// c*nch + g*BN_WAVES + w, a run of whole partials [cst[q], cst[q+1]) whose
// first partial is cpi[q].
template <typename T, bool NT>
__global__ __launch_bounds__(BN_THREADS) void binned_slice_kernel(
    int64_t n, int32_t W, int32_t G, int32_t nch, const T *__restrict__ sval,
    const uint16_t *__restrict__ scol, const int32_t *__restrict__ cst,
    const int32_t *__restrict__ cpi, const T *__restrict__ x, T *__restrict__ pval)
{
    constexpr int XMAX = BN_LDS / sizeof(T);
    constexpr int XPT = XMAX / BN_THREADS;
    __shared__ T xs[XMAX];
    const int c = blockIdx.x / G;
    const int g = blockIdx.x % G;
    const int64_t c0 = (int64_t)c * W;
    const int wn = (int)min((int64_t)W, n - c0);     // >= 1: slice c starts inside x
    const int lane = threadIdx.x & 63;
    // Wave-uniform (scalar) chunk bounds: the stream loop is then scalar
    // control flow and the two load buffers stay apart.
    const int q = __builtin_amdgcn_readfirstlane(c * nch + g * BN_WAVES + (int)(threadIdx.x >> 6));
    const int32_t ea = cst[q], eb = cst[q + 1];
    int32_t pk = cpi[q];
    T carry = T(0);

    constexpr int U = 8;            // steps of 64 entries per load group
    constexpr int GS = U * 64;
    T va[U], vb[U];
    uint32_t ka[U], kb[U];
    // Loads are clamped into the chunk, never predicated: a load under an
    // exec-masked branch makes the compiler wait for every outstanding one.
    // An empty chunk (ea == eb) clamps to its start, a valid entry or, for the
    // last chunk, entry nnz - 1 (the layout has nnz >= 1 entries).
    auto load = [&](T(&v)[U], uint32_t(&k)[U], int32_t e) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t p = (uint32_t)min(e + u * 64 + lane, max(eb - 1, 0));
            v[u] = NT ? __builtin_nontemporal_load(sval + p) : sval[p];
            k[u] = NT ? __builtin_nontemporal_load(scol + p) : scol[p];
        }
    };
    // The first group of entries is in flight while x's slice is copied to LDS.
    load(va, ka, ea);
    {
        T t[XPT];
#pragma unroll
        for (int u = 0; u < XPT; ++u) t[u] = x[c0 + min((int)threadIdx.x + u * BN_THREADS, wn - 1)];
#pragma unroll
        for (int u = 0; u < XPT; ++u) {
            const int j = threadIdx.x + u * BN_THREADS;
            if (j < wn) xs[j] = t[u];
        }
    }
    __syncthreads();
    if (ea >= eb) return;

    auto process = [&](const T(&v)[U], const uint32_t(&k)[U], int32_t e) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int32_t eu = e + u * 64;
            if (eu >= eb) break;
            const bool ok = eu + lane < eb;
            const uint32_t kk = k[u];
            T p = v[u] * xs[kk & BN_COL];
            p = ok ? p : T(0);
            const bool endf = ok && (kk & BN_END);
            const uint64_t mask = __ballot(endf);
            // Partials ended by earlier lanes of this step: this lane's segment.
            const int32_t seg = (int32_t)__builtin_amdgcn_mbcnt_hi(
                (uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
            T sum = wave_seg_scan<T>(seg, p);
            if (seg == 0) sum += carry;
            if (endf) pval[pk + seg] = sum;
            const T last = readlane63(sum);
            carry = (mask >> 63) ? T(0) : last;
            pk += (int32_t)__popcll(mask);
        }
    };
    int32_t e = ea;
    for (;;) {
        load(vb, kb, e + GS);
        process(va, ka, e);
        e += GS;
        if (e >= eb) break;
        load(va, ka, e + GS);
        process(vb, kb, e);
        e += GS;
        if (e >= eb) break;
    }
}

// ---- bin pass.  Workgroup b adds the runs of bin b, slice by slice, into
// ys = y[bH, bH + hn) and writes y.  Each thread takes K slots of a run; the
// slots of the next D runs are loaded ahead in registers.  The S runs are a
// chain of S steps, each waiting on loads issued D steps earlier, so a step
// costs about the memory latency / D: the plan picks the deepest ring whose K
// slots per thread hold its longest run (D*K = 24).
template <typename T, bool BZ, int D, int K, bool NT>
__global__ __launch_bounds__(BN_THREADS) void binned_bin_kernel(
    int64_t m, int32_t S, int32_t B, int32_t H, const int32_t *__restrict__ pr,
    const uint16_t *__restrict__ prow, const T *__restrict__ pval, T alpha, T beta,
    T *__restrict__ y)
{
    constexpr int YMAX = BN_LDS / sizeof(T);
    __shared__ T ys[YMAX];
    __shared__ int32_t rs[2 * BN_SMAX];
    const int b = blockIdx.x;
    const int t = threadIdx.x;
    const int64_t r0 = (int64_t)b * H;
    const int hn = (int)min((int64_t)H, m - r0);
    for (int j = t; j < hn; j += BN_THREADS) ys[j] = T(0);
    for (int c = t; c < S; c += BN_THREADS) {
        rs[2 * c] = pr[(int64_t)c * B + b];
        rs[2 * c + 1] = pr[(int64_t)c * B + b + 1];
    }
    __syncthreads();

    // Ring of the next D runs' slots: slot d holds run c with c % D == d.  A
    // slot is consumed before it is reloaded, and loaded values are not touched
    // before their use (flags apart), so waits only ever reach the oldest run.
    T pv[D][K];
    uint32_t pw[D][K];
    bool pok[D][K];
    auto load = [&](int c, int d) {
        const int cc = c < S ? c : S - 1;
        const int32_t lo = rs[2 * cc];
        const int32_t hi = c < S ? rs[2 * cc + 1] : lo;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int32_t a = lo + t + k * BN_THREADS;
            pok[d][k] = a < hi;
            // pval/prow hold P + 1 elements, so a run start is always readable.
            const uint32_t p = (uint32_t)(a < hi ? a : lo);
            pv[d][k] = NT ? __builtin_nontemporal_load(pval + p) : pval[p];
            pw[d][k] = NT ? __builtin_nontemporal_load(prow + p) : prow[p];
        }
    };
    auto consume = [&](int c, int d) {
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (pok[d][k]) ys[pw[d][k]] += pv[d][k];
        // Runs longer than K * BN_THREADS (rows of the bin with entries in this
        // slice): the rest, unpipelined.
        const int32_t hi = rs[2 * c + 1];
        for (int32_t a = rs[2 * c] + t + K * BN_THREADS; a < hi; a += BN_THREADS)
            ys[prow[a]] += pval[a];
    };
#pragma unroll
    for (int d = 0; d < D; ++d) load(d, d);
    int c0 = 0;
    for (; c0 + D <= S; c0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            consume(c0 + d, d);
            load(c0 + d + D, d);
            __syncthreads();
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (c0 + d < S) {
            consume(c0 + d, d);
            __syncthreads();
        }
    }
    for (int j = t; j < hn; j += BN_THREADS) {
        const T r = alpha * ys[j];
        y[r0 + j] = BZ ? r : r + beta * y[r0 + j];
    }
}

// ---- layout build

// cnt[rowptr[i] - origin] += 1 for i in [1, m): after an exclusive scan over
// nnz + 1 counts, cnt[k + 1] is the row of entry k (rows are counted, so a
// malformed rowptr still gives rows in [0, m) in non-decreasing order).
__global__ void bn_rowmark_kernel(int64_t m, int64_t nnz, int32_t origin,
                                  const int32_t *__restrict__ rowptr, int32_t *__restrict__ cnt)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x + 1;
    if (i >= m) return;
    int64_t v = (int64_t)rowptr[i] - origin;
    v = v < 0 ? 0 : (v > nnz ? nnz : v);
    atomicAdd(&cnt[v], 1);
}

__device__ __forceinline__ int32_t bn_row(const int32_t *erow, int64_t k, int64_t m)
{
    const int32_t r = erow[k];
    return r < 0 ? 0 : (r >= m ? (int32_t)(m - 1) : r);
}

__global__ void bn_key_kernel(int64_t nnz, int64_t m, int32_t origin, const int32_t *__restrict__ colind,
                              const int32_t *__restrict__ erow, int32_t W, int32_t S, int32_t H,
                              int32_t B, uint32_t *__restrict__ key, int32_t *__restrict__ iota)
{
    const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (k >= nnz) return;
    int64_t c = ((int64_t)colind[k] - origin) / W;
    c = c < 0 ? 0 : (c >= S ? S - 1 : c);
    const int32_t b = bn_row(erow, k, m) / H;
    key[k] = (uint32_t)(c * B + b);
    iota[k] = (int32_t)k;
}

// prow[partial] = bin-local row, for the entry that ends each partial.
__global__ void bn_prow_kernel(int64_t nnz, const uint16_t *__restrict__ erl, const uint16_t *__restrict__ scol,
                               const int32_t *__restrict__ fpre, uint16_t *__restrict__ prow)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nnz || !(scol[e] & BN_END)) return;
    prow[fpre[e]] = erl[e];
}

// Run bounds from the sorted keys: est[r] = first entry with key >= r, for
// r in [0, R]; every r is written once.
__global__ void bn_est_kernel(int64_t nnz, int64_t R, const uint32_t *__restrict__ skey,
                              int32_t *__restrict__ est)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e > nnz) return;
    const int64_t prev = e == 0 ? -1 : (int64_t)skey[e - 1];
    const int64_t cur = e == nnz ? R : (int64_t)skey[e];
    for (int64_t r = prev + 1; r <= cur; ++r) est[r] = (int32_t)e;
}

// pr[r] = the partial index of run r's first entry, r in [0, R].
__global__ void bn_pr_kernel(int64_t R, const int32_t *__restrict__ est, const int32_t *__restrict__ fpre,
                             int32_t *__restrict__ pr)
{
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r <= R) pr[r] = fpre[est[r]];
}

// Longest run, in partials: a wave's maximum, one atomic per wave.
__global__ void bn_maxrun_kernel(int64_t R, const int32_t *__restrict__ pr, int32_t *__restrict__ out)
{
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int32_t v = r < R ? pr[r + 1] - pr[r] : 0;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    if (__lane_id() == 0 && v > 0) atomicMax(out, v);
}

// Chunk q = c*nch + w of slice c starts at the first partial start at or after
// the slice's entries split evenly nch ways.
__global__ void bn_chunk_kernel(int64_t nnz, int32_t S, int32_t B, int32_t nch,
                                const int32_t *__restrict__ est, const int32_t *__restrict__ fpre,
                                int32_t *__restrict__ cst, int32_t *__restrict__ cpi)
{
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q == (int64_t)S * nch) cst[q] = (int32_t)nnz;
    if (q >= (int64_t)S * nch) return;
    const int64_t c = q / nch, w = q % nch;
    const int64_t s0 = est[c * B], s1 = est[(c + 1) * B];
    int64_t e = s0 + (s1 - s0) * w / nch;
    while (e > s0 && e < s1 && fpre[e] == fpre[e - 1]) ++e;
    cst[q] = (int32_t)e;
    cpi[q] = fpre[e];
}

// First CSR entry of each bin: bst[b] = rowptr[min(b H, m)] - origin, clamped.
__global__ void bn_binstart_kernel(int64_t m, int64_t nnz, int32_t origin, int32_t H, int32_t B,
                                   const int32_t *__restrict__ rowptr, int32_t *__restrict__ bst)
{
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b > B) return;
    int64_t v = (int64_t)rowptr[min(b * H, m)] - origin;
    bst[b] = (int32_t)(v < 0 ? 0 : (v > nnz ? nnz : v));
}

// rtab[row * S + c] for row = rtb[b] + k: the first entry e of run (c, b)
// with perm[e] >= bst[b] + k * chunk (a run's entries are in CSR order, so
// perm increases along it), by binary search.  One thread per (row, c).
__global__ void bn_rtable_kernel(int64_t nrows, int32_t S, int32_t B, int64_t chunk,
                                 const int32_t *__restrict__ rtb, const int32_t *__restrict__ bst,
                                 const int32_t *__restrict__ est, const int32_t *__restrict__ perm,
                                 int32_t *__restrict__ rtab)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nrows * S) return;
    const int64_t row = t / S, c = t % S;
    int lo = 0, hi = B;                   // the bin b with rtb[b] <= row < rtb[b + 1]
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (rtb[mid] <= row) lo = mid; else hi = mid;
    }
    const int64_t b = lo;
    const int64_t want = (int64_t)bst[b] + (row - rtb[b]) * chunk;
    int64_t a = est[c * B + b], z = est[c * B + b + 1];
    while (a < z) {
        const int64_t mid = (a + z) / 2;
        if ((int64_t)perm[mid] < want) a = mid + 1; else z = mid;
    }
    rtab[t] = (int32_t)a;
}

// loff[e]: the offset of sorted entry e's CSR entry perm[e] within its
// bin's refresh chunk, (perm[e] - bst[b]) mod chunk, b = the bin of its key.
__global__ void bn_loff_kernel(int64_t nnz, int32_t B, int32_t chunk, const uint32_t *__restrict__ skey,
                               const int32_t *__restrict__ bst, const int32_t *__restrict__ perm,
                               uint16_t *__restrict__ loff)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= nnz) return;
    const int64_t d = (int64_t)perm[e] - bst[skey[e] % (uint32_t)B];
    loff[e] = (uint16_t)(d < 0 ? 0 : d % chunk);
}

// New values into the layout by chunks: workgroup g holds chunk k of bin b,
// CSR entries [c0, c1) = [bst[b] + k L, min(bst[b] + (k+1) L, bst[b+1])), in
// LDS (L = RF_LDS / sizeof(T)), read once and coalesced; every run (c, b)
// holds those entries as one contiguous range [rtab[row][c], rtab[row+1][c]),
// so the workgroup writes the ranges of all S runs, each entry e taking
// v[loff[e]] from LDS; the outputs are the chunk's S ranges laid end to end.
// Indices are clamped into the chunk and the layout.  The chunks are dealt
// to the XCDs in contiguous ranges (workgroup g, on XCD g % 8, takes chunk
// (g % 8) * per + g / 8): a bin's neighbouring chunks then write the two ends
// of their shared output lines into one L2, which writes each line back once.
#ifndef JLUST_RF_THREADS
#define JLUST_RF_THREADS 1024
#endif
#ifndef JLUST_RF_LDS_KB
#define JLUST_RF_LDS_KB 64
#endif
constexpr int RF_THREADS = JLUST_RF_THREADS;        // refresh workgroup (two per CU)
constexpr int RF_LDS = JLUST_RF_LDS_KB * 1024;      // values of a refresh chunk in LDS
constexpr int RF_SPT = (BN_SMAX + RF_THREADS - 1) / RF_THREADS;   // runs per thread in the scan
static_assert(RF_LDS / sizeof(float) <= 65536, "a refresh chunk's offsets must fit 16 bits (loff)");

template <typename T>
__global__ __launch_bounds__(RF_THREADS) void bn_refresh_lds_kernel(int64_t nnz, int32_t S, int32_t B,
                                                                    int32_t nrch,
                                                                    const int32_t *__restrict__ rch,
                                                                    const int32_t *__restrict__ bst,
                                                                    const int32_t *__restrict__ rtb,
                                                                    const int32_t *__restrict__ rtab,
                                                                    const uint16_t *__restrict__ loff,
                                                                    const T *__restrict__ src,
                                                                    T *__restrict__ dst)
{
    constexpr int L = RF_LDS / sizeof(T);
    constexpr int PER = L / RF_THREADS;   // values (and outputs) per thread
    __shared__ T v[L];
    __shared__ int32_t pre[BN_SMAX + 1], beg[BN_SMAX], tsum[RF_THREADS];
    const int t = threadIdx.x;
    const int per = (nrch + NUM_XCD - 1) / NUM_XCD;
    const int g = (int)(blockIdx.x % NUM_XCD) * per + (int)(blockIdx.x / NUM_XCD);
    if (g >= nrch) return;                // whole workgroup
    const int64_t b = rch[2 * g], k = rch[2 * g + 1];
    const int64_t lo = bst[b], hi = bst[b + 1];
    const int64_t c0 = min(lo + k * L, hi), c1 = min(c0 + L, hi);
    const int nv = (int)(c1 - c0);
    // The runs' range bounds are loaded first, then the chunk's values, every
    // load issued before any is used.
    const int64_t row = (int64_t)rtb[b] + k;
    int32_t rb0[RF_SPT], rb1[RF_SPT];
#pragma unroll
    for (int j = 0; j < RF_SPT; ++j) {
        const int c = t * RF_SPT + j;
        rb0[j] = c < S ? rtab[row * S + c] : 0;
        rb1[j] = c < S ? rtab[(row + 1) * S + c] : 0;
    }
    {
        T tmp[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = t + u * RF_THREADS;
            tmp[u] = i < nv ? src[c0 + i] : T(0);
        }
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = t + u * RF_THREADS;
            if (i < nv) v[i] = tmp[u];
        }
    }
    // Range starts and lengths of the S runs; pre[c] = outputs before run c.
    int32_t lens[RF_SPT], local = 0;
#pragma unroll
    for (int j = 0; j < RF_SPT; ++j) {
        const int c = t * RF_SPT + j;
        lens[j] = 0;
        if (c < S) {
            const int64_t e0 = min(max((int64_t)rb0[j], (int64_t)0), nnz);
            const int64_t e1 = min(max((int64_t)rb1[j], e0), nnz);
            beg[c] = (int32_t)e0;
            lens[j] = (int32_t)(e1 - e0);
        }
        local += lens[j];
    }
    tsum[t] = local;
    __syncthreads();
    for (int off = 1; off < RF_THREADS; off <<= 1) {   // inclusive scan of the per-thread sums
        const int32_t x = t >= off ? tsum[t - off] : 0;
        __syncthreads();
        tsum[t] += x;
        __syncthreads();
    }
    {
        int32_t run = tsum[t] - local;
#pragma unroll
        for (int j = 0; j < RF_SPT; ++j) {
            const int c = t * RF_SPT + j;
            if (c < S) pre[c] = run;
            run += lens[j];
        }
        if (t == RF_THREADS - 1) pre[S] = tsum[t];
    }
    __syncthreads();
    // At most nv <= L outputs.  Wave w owns outputs [w PER 64, (w+1) PER 64),
    // lane l takes every 64th of them from l, so a wave's step covers 64
    // consecutive outputs (consecutive entries of one or two runs); a lane
    // finds its first run by binary search and later ones by stepping
    // forward.  All the offset loads are issued before the LDS reads and
    // stores.
    const int32_t total = min(pre[S], (int32_t)L);
    const int32_t o0 = (t >> 6) * (PER * 64) + (t & 63);
    int c = 0;                             // the run with pre[c] <= o < pre[c + 1]
    {
        int z = S;
        while (z - c > 1) {
            const int mid = (c + z) / 2;
            if (pre[mid] <= o0) c = mid; else z = mid;
        }
    }
    int32_t ev[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const int32_t o = o0 + u * 64;
        while (c + 1 < S && pre[c + 1] <= o) ++c;
        ev[u] = o < total ? beg[c] + (o - pre[c]) : -1;
    }
    int32_t pk[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) pk[u] = ev[u] >= 0 ? loff[ev[u]] : 0;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        if (ev[u] < 0) continue;
        dst[ev[u]] = v[pk[u] >= nv ? nv - 1 : pk[u]];
    }
}

// Layout columns, end bits and rows by the refresh's chunks: workgroup g
// holds chunk k of bin b -- the columns and bin-local rows of CSR entries
// [c0, c1) in LDS -- and, for every layout entry e of the chunk's S ranges
// (entry e of run c at LDS slot loff[e]), writes
//   scol[e] = slice-local column | BN_END if e ends its partial,
//   flag[e] = that end bit, erl[e] = its bin-local row.
// e ends its partial when e + 1 starts another run or holds another row.
// Within the chunk's range of run c the next entry's row is in LDS; past it,
// the run's next entry lies in a later chunk and its row is read through
// perm.  Slots, rows and columns are clamped into range; entries no chunk
// reaches (a malformed rowptr) keep the zeros the caller cleared.
template <int L>
__global__ __launch_bounds__(RF_THREADS) void bn_fill_lds_kernel(
    int64_t nnz, int64_t m, int32_t origin, int32_t S, int32_t B, int32_t W, int32_t H, int32_t nrch,
    const int32_t *__restrict__ rch, const int32_t *__restrict__ bst, const int32_t *__restrict__ rtb,
    const int32_t *__restrict__ rtab, const int32_t *__restrict__ est, const uint16_t *__restrict__ loff,
    const int32_t *__restrict__ perm, const int32_t *__restrict__ colind, const int32_t *__restrict__ erow,
    uint16_t *__restrict__ scol, int32_t *__restrict__ flag, uint16_t *__restrict__ erl)
{
    constexpr int PER = L / RF_THREADS;   // outputs per thread
    __shared__ int32_t col[L];
    __shared__ uint16_t lrow[L];
    __shared__ int32_t pre[BN_SMAX + 1], beg[BN_SMAX], rend[BN_SMAX], tsum[RF_THREADS];
    const int t = threadIdx.x;
    const int per = (nrch + NUM_XCD - 1) / NUM_XCD;
    const int g = (int)(blockIdx.x % NUM_XCD) * per + (int)(blockIdx.x / NUM_XCD);
    if (g >= nrch) return;                // whole workgroup
    const int64_t b = rch[2 * g], k = rch[2 * g + 1];
    const int64_t lo = bst[b], hi = bst[b + 1];
    const int64_t c0 = min(lo + k * L, hi), c1 = min(c0 + L, hi);
    const int nv = (int)(c1 - c0);
    const int64_t row = (int64_t)rtb[b] + k;
    const int64_t r0 = b * H;             // the bin's first row
    int32_t rb0[RF_SPT], rb1[RF_SPT], re[RF_SPT];
#pragma unroll
    for (int j = 0; j < RF_SPT; ++j) {
        const int c = t * RF_SPT + j;
        rb0[j] = c < S ? rtab[row * S + c] : 0;
        rb1[j] = c < S ? rtab[(row + 1) * S + c] : 0;
        re[j] = c < S ? est[(int64_t)c * B + b + 1] : 0;
    }
    for (int i = t; i < nv; i += RF_THREADS) {
        col[i] = colind[c0 + i] - origin;
        const int64_t lr = (int64_t)bn_row(erow, c0 + i, m) - r0;
        lrow[i] = (uint16_t)(lr < 0 ? 0 : (lr >= H ? H - 1 : lr));
    }
    int32_t lens[RF_SPT], local = 0;
#pragma unroll
    for (int j = 0; j < RF_SPT; ++j) {
        const int c = t * RF_SPT + j;
        lens[j] = 0;
        if (c < S) {
            const int64_t e0 = min(max((int64_t)rb0[j], (int64_t)0), nnz);
            const int64_t e1 = min(max((int64_t)rb1[j], e0), nnz);
            beg[c] = (int32_t)e0;
            rend[c] = min(max(re[j], 0), (int32_t)nnz);
            lens[j] = (int32_t)(e1 - e0);
        }
        local += lens[j];
    }
    tsum[t] = local;
    __syncthreads();
    for (int off = 1; off < RF_THREADS; off <<= 1) {   // inclusive scan of the per-thread sums
        const int32_t x = t >= off ? tsum[t - off] : 0;
        __syncthreads();
        tsum[t] += x;
        __syncthreads();
    }
    {
        int32_t run = tsum[t] - local;
#pragma unroll
        for (int j = 0; j < RF_SPT; ++j) {
            const int c = t * RF_SPT + j;
            if (c < S) pre[c] = run;
            run += lens[j];
        }
        if (t == RF_THREADS - 1) pre[S] = tsum[t];
    }
    __syncthreads();
    // Outputs as in the refresh: wave w owns [w PER 64, (w+1) PER 64), lane l
    // every 64th of them from l.
    const int32_t total = min(pre[S], (int32_t)L);
    const int32_t o0 = (t >> 6) * (PER * 64) + (t & 63);
    int c = 0;                             // the run with pre[c] <= o < pre[c + 1]
    {
        int z = S;
        while (z - c > 1) {
            const int mid = (c + z) / 2;
            if (pre[mid] <= o0) c = mid; else z = mid;
        }
    }
#pragma unroll 4
    for (int u = 0; u < PER; ++u) {
        const int32_t o = o0 + u * 64;
        while (c + 1 < S && pre[c + 1] <= o) ++c;
        if (o >= total) continue;
        const int64_t e = (int64_t)beg[c] + (o - pre[c]);
        const int kk = min((int)loff[e], nv - 1);
        const int rowe = lrow[kk];
        bool end;
        if (e + 1 >= rend[c]) end = true;
        else if (o + 1 < pre[c + 1]) end = lrow[min((int)loff[e + 1], nv - 1)] != rowe;
        else end = (int64_t)bn_row(erow, perm[e + 1], m) - r0 != rowe;
        int64_t lc = (int64_t)col[kk] - (int64_t)c * W;
        lc = lc < 0 ? 0 : (lc >= W ? W - 1 : lc);
        scol[e] = (uint16_t)(lc | (end ? BN_END : 0u));
        flag[e] = end ? 1 : 0;
        erl[e] = (uint16_t)rowe;
    }
}

unsigned blocks256(int64_t n) { return (unsigned)((n + 255) / 256); }

// The value refresh over every chunk: sval from val (CSR order).
int launch_refresh(const BinnedLayout *L, const void *val, hipStream_t s)
{
    const unsigned grid = (unsigned)((L->nrch + NUM_XCD - 1) / NUM_XCD * NUM_XCD);
    if (L->value_type == 0)
        hipLaunchKernelGGL((bn_refresh_lds_kernel<double>), dim3(grid), dim3(RF_THREADS), 0, s, L->nnz, L->S, L->B,
                           L->nrch, L->rch, L->bst, L->rtb, L->rtab, L->loff, (const double *)val,
                           (double *)L->sval);
    else
        hipLaunchKernelGGL((bn_refresh_lds_kernel<float>), dim3(grid), dim3(RF_THREADS), 0, s, L->nnz, L->S, L->B,
                           L->nrch, L->rch, L->bst, L->rtb, L->rtab, L->loff, (const float *)val,
                           (float *)L->sval);
    return check_launch("bn_refresh_lds_kernel");
}

template <typename T>
int build(BinnedLayout *L, int32_t origin, const int32_t *rowptr, const int32_t *colind, const T *val,
          int64_t max_bytes, hipStream_t s)
{
    const int64_t m = L->m, nnz = L->nnz;
    const int64_t R = (int64_t)L->S * L->B;
    const int64_t nchunks = (int64_t)L->S * L->nch;
    // Persistent arrays.
    const size_t sz_v = align_up(sizeof(T) * (size_t)nnz, 256);
    const size_t sz_c = align_up(sizeof(uint16_t) * (size_t)nnz, 256);
    const size_t sz_lo = align_up(sizeof(uint16_t) * (size_t)nnz, 256);
    const size_t sz_ch = align_up(sizeof(int32_t) * (size_t)(nchunks + 1), 256);
    const size_t sz_pr = align_up(sizeof(int32_t) * (size_t)(R + 1), 256);
    const size_t sz_rw = align_up(sizeof(uint16_t) * (size_t)(nnz + 1), 256);
    const size_t sz_pv = align_up(sizeof(T) * (size_t)(nnz + 1), 256);
    const size_t sz_es = align_up(sizeof(int32_t) * (size_t)(R + 1), 256);
    // Refresh tables, sized for at most nnz / chunk + B chunks.
    const int64_t chunk = RF_LDS / (int64_t)sizeof(T);
    const int64_t nrch_max = nnz / chunk + L->B + 1;
    const size_t sz_rch = align_up(sizeof(int32_t) * (size_t)(2 * nrch_max), 256);
    const size_t sz_bb = align_up(sizeof(int32_t) * (size_t)(L->B + 1), 256);
    const size_t sz_rt = align_up(sizeof(int32_t) * (size_t)((nrch_max + L->B) * L->S), 256);
    const size_t persistent = sz_v + sz_c + sz_lo + 2 * sz_ch + sz_pr + sz_es + sz_rw + sz_pv + sz_rch + 2 * sz_bb +
                              sz_rt;
    // Temporaries: row counts / rows (nnz + 1), keys, sorted keys, iota,
    // the sort permutation, flags / partial indices (nnz + 1), sort storage.
    uint32_t *nk = nullptr;
    size_t sort_bytes = 0;
    int bits = 1;
    while (((int64_t)1 << bits) < R) ++bits;
    JLUST_HIP_TRY(rocprim::radix_sort_pairs(nullptr, sort_bytes, nk, nk, (int32_t *)nullptr,
                                            (int32_t *)nullptr, (size_t)nnz, 0, bits, s));
    const size_t sz_i = align_up(sizeof(int32_t) * (size_t)(nnz + 1), 256);
    const size_t temporary = 6 * sz_i + align_up(sort_bytes, 256);
    if (max_bytes > 0 && (int64_t)(persistent + temporary) > max_bytes)
        return fail(JLUST_STATUS_OUT_OF_MEMORY,
                    "binned spmv layout: %lld + %lld build bytes above JLUST_HIP_PLAN_MAX_BYTES (%lld)",
                    (long long)persistent, (long long)temporary, (long long)max_bytes);
    JLUST_HIP_TRY(hipMalloc(&L->mem, persistent));
    L->bytes = (int64_t)persistent;
    char *p = (char *)L->mem;
    L->sval = p;                 p += sz_v;
    L->scol = (uint16_t *)p;     p += sz_c;
    L->loff = (uint16_t *)p;     p += sz_lo;
    L->cst = (int32_t *)p;       p += sz_ch;
    L->cpi = (int32_t *)p;       p += sz_ch;
    L->pr = (int32_t *)p;        p += sz_pr;
    L->est = (int32_t *)p;       p += sz_es;
    L->rch = (int32_t *)p;       p += sz_rch;
    L->bst = (int32_t *)p;       p += sz_bb;
    L->rtb = (int32_t *)p;       p += sz_bb;
    L->rtab = (int32_t *)p;      p += sz_rt;
    L->prow = (uint16_t *)p;     p += sz_rw;
    L->pval = p;

    void *tmp = nullptr;
    JLUST_HIP_TRY(hipMalloc(&tmp, temporary));
    char *q = (char *)tmp;
    int32_t *cnt = (int32_t *)q;    q += sz_i;
    uint32_t *key = (uint32_t *)q;  q += sz_i;
    uint32_t *skey = (uint32_t *)q; q += sz_i;
    int32_t *iota = (int32_t *)q;   q += sz_i;
    int32_t *perm = (int32_t *)q;   q += sz_i;   // sorted entry e holds CSR entry perm[e]
    int32_t *fpre = (int32_t *)q;   q += sz_i;
    int32_t *est = L->est;
    void *sort_tmp = q;
    const int32_t *erow = cnt + 1;

    std::vector<int32_t> h_bst, h_rch, h_rtb;      // host side of the refresh tables
    int st = JLUST_STATUS_SUCCESS;
    hipError_t e = hipMemsetAsync(cnt, 0, sizeof(int32_t) * (size_t)(nnz + 1), s);
    if (e != hipSuccess) st = hip_fail(e, "hipMemsetAsync(binned row counts)");
    if (!st && m > 1) {
        hipLaunchKernelGGL(bn_rowmark_kernel, dim3(blocks256(m - 1)), dim3(256), 0, s, m, nnz, origin,
                           rowptr, cnt);
        st = check_launch("bn_rowmark_kernel");
    }
    if (!st) st = exclusive_scan_i32(cnt, cnt, nnz + 1, (jlust_stream_t)s);
    if (!st) {
        hipLaunchKernelGGL(bn_key_kernel, dim3(blocks256(nnz)), dim3(256), 0, s, nnz, m, origin, colind,
                           erow, L->W, L->S, L->H, L->B, key, iota);
        st = check_launch("bn_key_kernel");
    }
    if (!st) {
        e = rocprim::radix_sort_pairs(sort_tmp, sort_bytes, key, skey, iota, perm, (size_t)nnz, 0, bits,
                                      s);
        if (e != hipSuccess) st = hip_fail(e, "rocprim::radix_sort_pairs(binned keys)");
    }
    // Run starts; then the refresh tables; then the layout by the refresh's
    // chunks: the values through the refresh kernel, and the columns, end
    // bits and rows through bn_fill_lds_kernel.
    if (!st) {
        hipLaunchKernelGGL(bn_est_kernel, dim3(blocks256(nnz + 1)), dim3(256), 0, s, nnz, R, skey, est);
        st = check_launch("bn_est_kernel");
    }
    // Refresh tables: the bins' first entries, their chunks (host), and the
    // first entry of every run at every chunk boundary of its bin.
    if (!st) {
        hipLaunchKernelGGL(bn_binstart_kernel, dim3(blocks256(L->B + 1)), dim3(256), 0, s, m, nnz, origin, L->H,
                           L->B, rowptr, L->bst);
        st = check_launch("bn_binstart_kernel");
    }
    if (!st) {
        h_bst.resize((size_t)L->B + 1);
        e = hipMemcpyAsync(h_bst.data(), L->bst, sizeof(int32_t) * h_bst.size(), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) st = hip_fail(e, "binned refresh tables (bin starts)");
    }
    int64_t nrows = 0;
    if (!st) {
        h_rtb.resize((size_t)L->B + 1);
        for (int32_t b = 0; b < L->B; ++b) {
            h_rtb[b] = (int32_t)nrows;
            const int64_t nb = std::max<int64_t>(0, (int64_t)h_bst[b + 1] - h_bst[b]);
            const int64_t q = (nb + chunk - 1) / chunk;
            for (int64_t k = 0; k < q; ++k) {
                h_rch.push_back(b);
                h_rch.push_back((int32_t)k);
            }
            nrows += q + 1;
        }
        h_rtb[L->B] = (int32_t)nrows;
        L->nrch = (int32_t)(h_rch.size() / 2);
        if ((int64_t)L->nrch > nrch_max)
            st = fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                      "binned spmv layout: rowptr not non-decreasing (%d value chunks, at most %lld)", L->nrch,
                      (long long)nrch_max);
    }
    if (!st && L->nrch > 0) {
        e = hipMemcpyAsync(L->rch, h_rch.data(), sizeof(int32_t) * h_rch.size(), hipMemcpyHostToDevice, s);
        if (e == hipSuccess)
            e = hipMemcpyAsync(L->rtb, h_rtb.data(), sizeof(int32_t) * h_rtb.size(), hipMemcpyHostToDevice, s);
        if (e != hipSuccess) st = hip_fail(e, "binned refresh tables (chunks)");
        if (!st) {
            hipLaunchKernelGGL(bn_rtable_kernel, dim3(blocks256(nrows * L->S)), dim3(256), 0, s, nrows, L->S, L->B,
                               chunk, L->rtb, L->bst, est, perm, L->rtab);
            st = check_launch("bn_rtable_kernel");
        }
        if (!st) {
            hipLaunchKernelGGL(bn_loff_kernel, dim3(blocks256(nnz)), dim3(256), 0, s, nnz, L->B, (int32_t)chunk,
                               skey, L->bst, perm, L->loff);
            st = check_launch("bn_loff_kernel");
        }
        if (!st) st = launch_refresh(L, val, s);
    }
    // Every entry's column and end bit start at zero, so that entries no chunk
    // reaches (a malformed rowptr) still give partial indices in range.
    if (!st) {
        e = hipMemsetAsync(L->scol, 0, sizeof(uint16_t) * (size_t)nnz, s);
        if (e == hipSuccess) e = hipMemsetAsync(fpre, 0, sizeof(int32_t) * (size_t)(nnz + 1), s);
        if (e != hipSuccess) st = hip_fail(e, "hipMemsetAsync(binned columns and end bits)");
    }
    uint16_t *erl = reinterpret_cast<uint16_t *>(key);   // keys are dead after the sort
    if (!st && L->nrch > 0) {
        constexpr int CH = RF_LDS / (int)sizeof(T);
        const unsigned grid = (unsigned)((L->nrch + NUM_XCD - 1) / NUM_XCD * NUM_XCD);
        hipLaunchKernelGGL((bn_fill_lds_kernel<CH>), dim3(grid), dim3(RF_THREADS), 0, s, nnz, m, origin, L->S, L->B,
                           L->W, L->H, L->nrch, L->rch, L->bst, L->rtb, L->rtab, est, L->loff, perm, colind, erow,
                           L->scol, fpre, erl);
        st = check_launch("bn_fill_lds_kernel");
    }
    if (!st) st = exclusive_scan_i32(fpre, fpre, nnz + 1, (jlust_stream_t)s);
    if (!st) {
        hipLaunchKernelGGL(bn_prow_kernel, dim3(blocks256(nnz)), dim3(256), 0, s, nnz, erl, L->scol, fpre, L->prow);
        st = check_launch("bn_prow_kernel");
    }
    if (!st) {
        hipLaunchKernelGGL(bn_pr_kernel, dim3(blocks256(R + 1)), dim3(256), 0, s, R, est, fpre, L->pr);
        st = check_launch("bn_pr_kernel");
    }
    if (!st) {
        hipLaunchKernelGGL(bn_chunk_kernel, dim3(blocks256(nchunks + 1)), dim3(256), 0, s, nnz, L->S, L->B,
                           L->nch, est, fpre, L->cst, L->cpi);
        st = check_launch("bn_chunk_kernel");
    }
    // cnt is free again: cnt[0] receives the longest run.
    if (!st) {
        e = hipMemsetAsync(cnt, 0, sizeof(int32_t), s);
        if (e != hipSuccess) st = hip_fail(e, "hipMemsetAsync(binned longest run)");
    }
    if (!st) {
        hipLaunchKernelGGL(bn_maxrun_kernel, dim3(blocks256(R)), dim3(256), 0, s, R, L->pr, cnt);
        st = check_launch("bn_maxrun_kernel");
    }
    int32_t P = 0, maxrun = 0;
    if (!st) {
        e = hipMemcpyAsync(&P, fpre + nnz, sizeof(int32_t), hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipMemcpyAsync(&maxrun, cnt, sizeof(int32_t), hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) st = hip_fail(e, "hipMemcpyAsync(binned partial count)");
    }
    const hipError_t es = hipStreamSynchronize(s);
    (void)hipFree(tmp);
    if (st) return st;
    if (es != hipSuccess) return hip_fail(es, "hipStreamSynchronize(binned layout build)");
    L->P = P;
    L->maxrun = maxrun;
    return JLUST_STATUS_SUCCESS;
}

// Streams read once are loaded nontemporal: bit 0 = the entries in the slice
// pass, bit 1 = the partials and their rows in the bin pass.  Both (the
// default, JLUST_HIP_BINNED_NT=3) measured 0.326 ms per config-2 step against
// 0.368 ms with neither and 0.342 ms with the bin pass's alone: the entries then
// stop evicting the partials the bin pass is about to read.
int binned_nt()
{
    static const int v = [] {
        const char *e = getenv("JLUST_HIP_BINNED_NT");
        return e ? atoi(e) & 3 : 3;
    }();
    return v;
}

template <typename T>
int execute(const BinnedLayout *L, T alpha, const T *x, T beta, T *y, hipStream_t s)
{
    const int nt = binned_nt();
#define SL(N)                                                                                        \
    hipLaunchKernelGGL((binned_slice_kernel<T, N>), dim3((unsigned)(L->S * L->G)), dim3(BN_THREADS), 0, \
                       s, L->n, L->W, L->G, L->nch, (const T *)L->sval, L->scol, L->cst, L->cpi, x,    \
                       (T *)L->pval)
    if (nt & 1) SL(true);
    else SL(false);
#undef SL
    if (int st = check_launch("binned_slice_kernel")) return st;
#define BIN(Z, D, K, N)                                                                                \
    hipLaunchKernelGGL((binned_bin_kernel<T, Z, D, K, N>), dim3((unsigned)L->B), dim3(BN_THREADS), 0, s, \
                       L->m, L->S, L->B, L->H, L->pr, L->prow, (const T *)L->pval, alpha, beta, y)
#define BINN(Z, D, K) do { if (nt & 2) BIN(Z, D, K, true); else BIN(Z, D, K, false); } while (0)
#define BINZ(D, K) do { if (beta == T(0)) BINN(true, D, K); else BINN(false, D, K); } while (0)
    if (L->maxrun <= BN_THREADS) BINZ(24, 1);
    else if (L->maxrun <= 2 * BN_THREADS) BINZ(12, 2);
    else BINZ(6, 4);
#undef BINZ
#undef BINN
#undef BIN
    return check_launch("binned_bin_kernel");
}

}  // namespace

bool binned_fits(int value_type, int64_t m, int64_t n, int64_t nnz)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    int32_t W, S, G, H, B;
    return geometry(value_type, m, n, nnz, device_info(dev).cu_count, &W, &S, &G, &H, &B);
}

int64_t binned_bytes(const BinnedLayout *L) { return L ? L->bytes : 0; }

int binned_build(BinnedLayout **out, int value_type, int64_t m, int64_t n, int64_t nnz, int32_t origin,
                 const int32_t *rowptr, const int32_t *colind, const void *val, int64_t max_bytes,
                 hipStream_t s)
{
    *out = nullptr;
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    auto *L = new BinnedLayout();
    L->m = m;
    L->n = n;
    L->nnz = nnz;
    L->value_type = value_type;
    if (!geometry(value_type, m, n, nnz, device_info(dev).cu_count, &L->W, &L->S, &L->G, &L->H, &L->B)) {
        delete L;
        return fail(JLUST_STATUS_UNSUPPORTED_FORMAT,
                    "binned spmv layout: %lld x %lld with %lld entries does not fit its index widths",
                    (long long)m, (long long)n, (long long)nnz);
    }
    L->nch = L->G * BN_WAVES;
    const int st = value_type == 0 ? build<double>(L, origin, rowptr, colind, (const double *)val, max_bytes, s)
                                   : build<float>(L, origin, rowptr, colind, (const float *)val, max_bytes, s);
    if (st) {
        binned_destroy(L);
        return st;
    }
    *out = L;
    return JLUST_STATUS_SUCCESS;
}

int binned_update(BinnedLayout *L, const void *val, hipStream_t s)
{
    if (L->nrch <= 0) return JLUST_STATUS_SUCCESS;
    return launch_refresh(L, val, s);
}

int binned_execute_f64(const BinnedLayout *L, double alpha, const double *x, double beta, double *y,
                       hipStream_t s)
{
    return execute<double>(L, alpha, x, beta, y, s);
}

int binned_execute_f32(const BinnedLayout *L, float alpha, const float *x, float beta, float *y,
                       hipStream_t s)
{
    return execute<float>(L, alpha, x, beta, y, s);
}

void binned_destroy(BinnedLayout *L)
{
    if (!L) return;
    if (L->mem) (void)hipFree(L->mem);
    delete L;
}

}  // namespace jlust

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

int preload_binned(hipStream_t s)
{
    JLUST_PRELOAD_KERNEL(bn_rowmark_kernel);
    return preload_radix_sort<uint32_t, int32_t>(s, 20);
}
}  // namespace jlust
