// spmv.hip -- CSR SpMV y = alpha*A*x + beta*y for gfx950 (wave64).
//
// Replaces the CSR branch of execute(::EmitterBackend, ::Op{:SpMV}, ...)
// (ext/KernelAbstractionsExt/ops/spmv.jl:449-502), whose per-row arithmetic is
// `acc = 0; for k in row: acc += val[k]*x[col[k]]; y = alpha*acc (+beta*y)`
// (spmv.jl:154-169, _walker.jl:123-132).
//
// Work split (merge_range): the merge path of (m row ends, nnz nonzeros) is
// cut into tiles of TILE = BLOCK*IPT items, so every tile costs the same
// whatever the row lengths (a 10^5-nonzero row spans ~50 tiles; 10^4 empty
// rows share one).  Each block owns consecutive tiles and finds only its
// first coordinate in global memory (a 64-ary wave-parallel search of
// rowptr); the next tile starts where the previous one ended.  Per tile:
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
//
// Column-sliced plans.  A random gather of x costs a whole 128-byte line from
// the memory side whenever x does not fit the 4 MB L2 of an XCD (8 XCDs,
// workgroup b runs on XCD b % 8).  A prepared plan whose x exceeds that
// re-lays A out as 8 column slices (slice s = columns [s*w, (s+1)*w)): each
// slice is a CSR matrix over all m rows with local column indices.  The
// sliced kernel runs slice s on the workgroups with b % 8 == s, so XCD s only
// gathers from x[s*w : (s+1)*w] and keeps it in its own L2.  Slice s writes a
// partial y_s; a last pass forms y = alpha*(y_0 + ... + y_7) + beta*y in that
// fixed order.
//
// LDS-binned plans (spmv_binned.hip) go further for a large x with scattered
// columns: x is cut into one LDS-sized slice per CU and y into LDS-sized row
// bins, so no gather leaves a CU.  choose_layout() below picks row order,
// column slices or bins when a plan is made.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>

#include "common.hpp"
#include "spmv_binned.hpp"
#include "wave.hpp"

namespace jlust {
namespace {

constexpr int SPMV_BLOCK = 256;
constexpr size_t SLICE_MIN_X_BYTES = (size_t)4 << 20;   // one XCD's L2

// LDS of one block.  buf: the tile's products at [0, nloc), followed by the
// finished row sums of the tile at [nloc, nloc + rend) (nloc + rend is the
// tile length).  diag[r]: merge coordinate of the end of tile row r (local
// row-end position + r); every thread stores IPT+1 of them.
template <typename T, int TILE, int NW>
struct SpmvSmem {
    T buf[TILE];
    int32_t diag[TILE + 64 * NW];
    int64_t i0;
    int32_t wcnt[NW];
    int32_t wkey[NW];
    T wval[NW];
};

__device__ __forceinline__ int64_t uniform64(int64_t v)
{
    const int32_t lo = __builtin_amdgcn_readfirstlane((int32_t)v);
    const int32_t hi = __builtin_amdgcn_readfirstlane((int32_t)(v >> 32));
    return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// Smallest i in [max(0, d-nnz), min(d, m)] with (rowptr[i+1]-ptr_origin) + i >= d,
// taking i == m as true: the number of rows finished after the first d items
// of the merge path.  Called by a whole wave; every lane returns the answer.
__device__ int64_t wave_merge_search(const int32_t *__restrict__ rowptr, int64_t ptr_origin,
                                     int64_t m, int64_t nnz, int64_t d)
{
    const int lane = __lane_id();
    int64_t lo = d - nnz > 0 ? d - nnz : 0;
    int64_t hi = d < m ? d : m;
    while (lo < hi) {
        const int64_t n = hi - lo;
        const int64_t p = lo + (n * lane) / 64;
        const bool pred = (p >= m) || ((int64_t)rowptr[p + 1] - ptr_origin + p >= d);
        const uint64_t mask = __ballot(pred);
        if (mask & 1ull) return lo;
        const int f = mask ? __builtin_ctzll(mask) : 64;
        const int64_t new_hi = f < 64 ? lo + (n * f) / 64 : hi;
        lo = lo + (n * (f - 1)) / 64 + 1;
        hi = new_hi;
    }
    return lo;
}

// One block's share [dbeg, dend) of the merge path of a CSR matrix whose row
// pointers hold ptr_origin + (0-based position in colind/val); the x value of
// a stored column c is xs[c - col_origin], and xs[0] is readable.  start_row
// < 0: search.  Requires m >= 1 and, for PF, a
// nonempty nonzero array: colind/val + jmax is the last readable element (jmax
// < 0 when this range's own nonzeros are empty; the clamped prefetch then
// reads an element before them).  BZ: beta == 0 (y is only written).
// PF: prefetch the next tile's row ends and col/val into registers while the
// current tile is processed (pays off when x gathers hit L2).  NT: stream
// rowptr/col/val with nontemporal loads.
template <typename T, int BLOCK, int IPT, bool PF, bool NT, bool BZ>
__device__ __forceinline__ void merge_range(int64_t m, int64_t nnz, int64_t jmax, int64_t ptr_origin,
                            int32_t col_origin, const int32_t *__restrict__ rowptr,
                            const int32_t *__restrict__ colind, const T *__restrict__ val,
                            const T *__restrict__ xs, T *__restrict__ y,
                            T alpha, T beta, int64_t dbeg, int64_t dend, int64_t start_row,
                            int64_t *carry_row, T *carry_val, SpmvSmem<T, BLOCK * IPT, BLOCK / 64> &sm)
{
    constexpr int TILE = BLOCK * IPT;
    constexpr int NW = BLOCK / 64;
    constexpr int RPT = IPT + 1;               // row ends per thread (TILE + 1 per tile)
    constexpr int BIG = TILE + 1;              // any row end at or past the tile's end
    static_assert(RPT * BLOCK <= TILE + 64 * NW, "diag too small for the row-end stores");
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    if (start_row >= 0) {
        if (tid == 0) sm.i0 = start_row;
    } else if (wave == 0) {
        const int64_t r = wave_merge_search(rowptr, ptr_origin, m, nnz, dbeg);
        if (lane == 0) sm.i0 = r;
    }
    __syncthreads();
    int64_t i0 = uniform64(sm.i0);
    int64_t j0 = dbeg - i0;
    T carry = T(0);
    bool carry_has = false;

    // Loads use a block-uniform base plus a 32-bit lane offset clamped into
    // range, with no per-lane branch: a load under an exec-masked branch makes
    // the compiler wait for every outstanding load before the next one.
    int32_t ren[RPT];
    int32_t cn[IPT];
    T vn[IPT];
    // The lane offsets are unsigned and below 2^11, so the compiler can use
    // scalar-base + 32-bit-offset addressing.
    auto load_rowends = [&](int64_t is) {      // rowptr[row + 1] of rows is + tid + u*BLOCK
        const int64_t ib = min(is, m - 1);
        const uint32_t lim = (uint32_t)min(m - 1 - ib, (int64_t)(RPT * BLOCK));
        const int32_t *rp = rowptr + ib + 1;
#pragma unroll
        for (int u = 0; u < RPT; ++u) {
            const uint32_t q = min((uint32_t)(tid + u * BLOCK), lim);
            ren[u] = NT ? __builtin_nontemporal_load(rp + q) : rp[q];
        }
    };
    // col (and, with VALS, val) of nonzeros js + tid + u*BLOCK, clamped to jmx.
    auto load_nz = [&](int64_t js, int64_t jmx, bool cols, bool vals) {
        const int64_t jb = min(js, jmx);
        const uint32_t lim = (uint32_t)min(jmx - jb, (int64_t)TILE);
        const int32_t *cb = colind + jb;
        const T *vb = val + jb;
#pragma unroll
        for (int u = 0; u < IPT; ++u) {
            const uint32_t q = min((uint32_t)(tid + u * BLOCK), lim);
            if (cols) cn[u] = NT ? __builtin_nontemporal_load(cb + q) : cb[q];
            if (vals) vn[u] = NT ? __builtin_nontemporal_load(vb + q) : vb[q];
        }
    };
    // Row ends are issued before col/val here and in the loop, so the wait for
    // them at the top of the loop leaves the col/val loads in flight on both
    // the entry and the loop-back path.
    if (PF) {
        load_rowends(i0);
        __builtin_amdgcn_sched_barrier(0);
        load_nz(j0, jmax, true, false);
        __builtin_amdgcn_sched_barrier(0);
        load_nz(j0, jmax, false, true);
    }

    for (int64_t d = dbeg; d < dend; d += TILE) {
        const int tlen = (int)min((int64_t)TILE, dend - d);
        // (1) merge coordinates of the row ends of rows i0 .. i0+tlen, and the
        // number rend of rows finished in this tile (diag is increasing, so it
        // is the count of row ends inside the tile).
        if (!PF) load_rowends(i0);
        {
            const int32_t base = (int32_t)(ptr_origin + j0);
            const int32_t rows_left = (int32_t)min(m - i0, (int64_t)(RPT * BLOCK));
            int cnt = 0;
#pragma unroll
            for (int u = 0; u < RPT; ++u) {
                const int r = tid + u * BLOCK;
                const int32_t e = min(max(ren[u] - base, 0), BIG);
                const int32_t dg = (r < rows_left ? e : BIG) + r;
                sm.diag[r] = dg;
                cnt += __popcll(__ballot(r < tlen && dg < tlen));
            }
            if (lane == 0) sm.wcnt[wave] = cnt;
        }
        __syncthreads();
        int rend = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) rend += sm.wcnt[w];
        rend = __builtin_amdgcn_readfirstlane(rend);
        const int nlt = tlen - rend;                        // nonzeros in the tile
        const int64_t j1 = j0 + nlt;
        // The clamp keeps a malformed rowptr from reading past the nonzero arrays.
        const int nloc = (int)(min(j1, nnz) - j0);
        // Does the tile end inside row i0+rend (a partial sum carried on)?
        if (rend > 0) carry_has = sm.diag[rend - 1] < tlen - 1;
        else carry_has = carry_has || nlt > 0;

        // (2) this thread's slice [dl, dl_next) starts in row r_first: the
        // smallest r with diag[r] >= dl, which lies in [dl - nlt, dl] and [0, rend].
        const int dl = min(tid * IPT, tlen);
        const int dl_next = min(dl + IPT, tlen);
        int lo = max(0, dl - nlt), hi = min(dl, rend);
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (sm.diag[mid] >= dl) hi = mid;
            else lo = mid + 1;
        }
        const int r_first = lo;

        // (3) products of the tile's nonzeros into LDS: gather x (lanes past
        // the tile's nonzeros gather x[0]), then start the next tile's prefetch.
        // With PF every lane gathers, so no branch separates the gathers from
        // the prefetch.
        // The next tile's row ends and columns are prefetched right after the
        // gathers (the current columns are dead once the gathers are issued),
        // its values after the products (which consume the current ones), so
        // each prefetch lands in the registers the next iteration reads.
        const bool has_nz = PF || nloc > 0;
        const bool more = d + TILE < dend;
        const int64_t inext = more ? i0 + rend : i0;   // the last tile re-reads itself
        const int64_t jnext = more ? j1 : j0;          // (L2-resident) rather than branching
        T xv[IPT];
        if (has_nz) {
            if (!PF) {           // columns first, so the gathers wait only for them
                load_nz(j0, j0 + nloc - 1, true, false);
                __builtin_amdgcn_sched_barrier(0);
                load_nz(j0, j0 + nloc - 1, false, true);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int u = 0; u < IPT; ++u) {
                const int q = tid + u * BLOCK;
                xv[u] = xs[q < nloc ? (uint32_t)(cn[u] - col_origin) : 0u];
            }
            // All gathers are issued before the products wait for the first.
            if (!PF) __builtin_amdgcn_sched_barrier(0);
        }
        if (PF) {
            // Issued after the gathers, so waiting for the gathers leaves the
            // prefetch in flight (loads return in order).
            load_rowends(inext);
            __builtin_amdgcn_sched_barrier(0);
            load_nz(jnext, jmax, true, false);
            __builtin_amdgcn_sched_barrier(0);
        }
        // Stored unconditionally: entries past nloc are scratch until the row
        // sums of step (4) overwrite them (a conditional store would let the
        // compiler sink its gather under the branch).
        if (has_nz) {
#pragma unroll
            for (int u = 0; u < IPT; ++u) sm.buf[tid + u * BLOCK] = vn[u] * xv[u];
        }
        if (PF) load_nz(jnext, jmax, false, true);
        __syncthreads();

        // (4) sequential walk of this thread's slice of the merge path: merge
        // item s is nonzero s - r of the tile while s < diag[r], else the end
        // of row r.
        T *ysum = sm.buf + nloc;
        T acc = T(0);
        int r = r_first;
        for (int s = dl; s < dl_next; ++s) {
            if (s < sm.diag[r]) {
                acc += sm.buf[s - r];
            } else {
                ysum[r] = acc;
                acc = T(0);
                ++r;
            }
        }
        if (tid == 0) {          // partial sum of row i0 left by the previous tile
            if (r > 0) ysum[0] += carry;
            else acc += carry;
        }

        // Segmented scan of (row, partial) over the block in thread order:
        // within each wave by DPP, across the NW waves from their totals.
        T sv = wave_seg_scan<T>(r, acc);
        if (lane == 63) {
            sm.wkey[wave] = r;
            sm.wval[wave] = sv;
        }
        __syncthreads();
        T pre = T(0);            // inclusive total of the waves before this one
        T run = T(0);
        int32_t pkey = -1, rkey = -1;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int32_t kw = sm.wkey[w];
            const T vw = sm.wval[w];
            run = kw == rkey ? vw + run : vw;
            rkey = kw;
            if (w == wave - 1) {
                pre = run;
                pkey = kw;
            }
        }
        if (r == pkey) sv += pre;
        // Value of the previous thread (lane 0: the previous waves' total).
        const T prev = dpp_val<0x138, 0xf>(pre, sv);
        if (tid > 0 && r > r_first) ysum[r_first] += prev;
        __syncthreads();

        // (5) finished rows i0 .. i0+rend-1.  With beta == 0 every thread
        // stores RPT times (lanes past rend repeat the tile's last row, same
        // value), so the count of outstanding memory operations is the same
        // on every path and the next tile's waits stay exact.
        if (BZ) {
            if (rend > 0) {
                T *yt = y + i0;
#pragma unroll
                for (int u = 0; u < RPT; ++u) {
                    const int q = min(tid + u * BLOCK, rend - 1);
                    yt[q] = alpha * ysum[q];
                }
            }
        } else {
            for (int q = tid; q < rend; q += BLOCK) {
                const int64_t row = i0 + q;
                y[row] = alpha * ysum[q] + beta * y[row];
            }
        }
        carry = run;
        i0 += rend;
        j0 = j1;
    }
    if (tid == 0) {
        *carry_row = (i0 < m && carry_has) ? i0 : -1;
        *carry_val = carry;
    }
}

template <typename T, int BLOCK, int IPT, bool PF, bool BZ>
__global__ __launch_bounds__(BLOCK) void csr_spmv_merge_kernel(
    int64_t m, int64_t nnz, int32_t origin, const int32_t *__restrict__ rowptr,
    const int32_t *__restrict__ colind, const T *__restrict__ val, const T *__restrict__ x,
    T *__restrict__ y, T alpha, T beta, int64_t tiles_per_block,
    const int64_t *__restrict__ start_rows, int64_t *__restrict__ carry_row,
    T *__restrict__ carry_val)
{
    constexpr int TILE = BLOCK * IPT;
    __shared__ SpmvSmem<T, TILE, BLOCK / 64> sm;
    // XCD-major order: the grid is a multiple of 8 blocks and workgroup b runs
    // on XCD b % 8, so logical block L = (b % 8) * (grid / 8) + b / 8 gives
    // each XCD one contiguous eighth of the merge path.  Rows of one eighth
    // gather from one window of x when the matrix is banded or block
    // structured, and that window stays in the XCD's own L2.
    const int64_t per_xcd = gridDim.x / NUM_XCD;
    const int64_t L = (int64_t)(blockIdx.x % NUM_XCD) * per_xcd + blockIdx.x / NUM_XCD;
    const int64_t total = m + nnz;
    const int64_t dbeg = L * tiles_per_block * TILE;
    if (dbeg >= total) return;
    const int64_t dend = min(total, dbeg + tiles_per_block * (int64_t)TILE);
    merge_range<T, BLOCK, IPT, PF, !PF, BZ>(m, nnz, nnz - 1, origin, origin, rowptr,
                                            colind, val, x, y, alpha, beta, dbeg, dend,
                                            start_rows ? start_rows[L] : -1,
                                            carry_row + L, carry_val + L, sm);
}

struct SliceInfo {
    int64_t off[NUM_XCD + 1];      // slice s occupies [off[s], off[s+1]) of colind/val
    int64_t tiles[NUM_XCD];        // tiles per block in slice s
};

// Workgroup b runs slice s = b % 8 (on XCD s); rowptr_all holds 8 row-pointer
// arrays of m+1 absolute positions; colind_all holds slice-local columns.
template <typename T, int BLOCK, int IPT, bool NT>
__global__ __launch_bounds__(BLOCK) void csr_spmv_sliced_kernel(
    int64_t m, SliceInfo info, const int32_t *__restrict__ rowptr_all,
    const int32_t *__restrict__ colind_all, const T *__restrict__ val_all,
    const T *__restrict__ x, int64_t slice_w, T *__restrict__ ypart, int64_t nb,
    const int64_t *__restrict__ start_rows, int64_t *__restrict__ carry_row,
    T *__restrict__ carry_val)
{
    constexpr int TILE = BLOCK * IPT;
    __shared__ SpmvSmem<T, TILE, BLOCK / 64> sm;
    const int s = blockIdx.x % NUM_XCD;
    const int64_t lb = blockIdx.x / NUM_XCD;
    const int64_t slot = s * nb + lb;
    const int64_t off = info.off[s];
    const int64_t nnz_s = info.off[s + 1] - off;
    const int64_t total = m + nnz_s;
    const int64_t dbeg = lb * info.tiles[s] * TILE;
    if (dbeg >= total) {
        if (threadIdx.x == 0) carry_row[slot] = -1;
        return;
    }
    const int64_t dend = min(total, dbeg + info.tiles[s] * (int64_t)TILE);
    // An empty slice gathers only xs[0]; its columns may start past x's end.
    const T *xs = nnz_s > 0 ? x + s * slice_w : x;
    merge_range<T, BLOCK, IPT, true, NT, true>(m, nnz_s, info.off[NUM_XCD] - 1 - off, off, 0,
                                               rowptr_all + s * (m + 1), colind_all + off,
                                               val_all + off, xs, ypart + s * m,
                                               T(1), T(0), dbeg, dend,
                                               start_rows ? start_rows[slot] : -1, carry_row + slot,
                                               carry_val + slot, sm);
}

// Adds each run of equal-row carries (in block order) of each segment into
// y + seg*ystride.  Segment = one merge path (the whole matrix, or a slice).
template <typename T>
__global__ void spmv_carry_fixup_kernel(int64_t nb, int64_t nseg, const int64_t *__restrict__ carry_row,
                                        const T *__restrict__ carry_val, T *__restrict__ y,
                                        int64_t ystride, T alpha)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nb * nseg) return;
    const int64_t seg = t / nb, b = t % nb;
    const int64_t *cr = carry_row + seg * nb;
    const T *cv = carry_val + seg * nb;
    const int64_t r = cr[b];
    if (r < 0) return;
    if (b > 0 && cr[b - 1] == r) return;
    T s = cv[b];
    for (int64_t u = b + 1; u < nb && cr[u] == r; ++u) s += cv[u];
    atomicAdd(&y[seg * ystride + r], alpha * s);
}

template <typename T>
__global__ void slice_reduce_kernel(int64_t m, const T *__restrict__ ypart, T *__restrict__ y,
                                    T alpha, T beta, int beta_zero)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= m) return;
    T s = __builtin_nontemporal_load(ypart + i);
#pragma unroll
    for (int k = 1; k < NUM_XCD; ++k) s += __builtin_nontemporal_load(ypart + k * m + i);
    const T r = alpha * s;
    y[i] = beta_zero ? r : r + beta * y[i];
}

// Start row of each block's first tile: plain (nseg = 1) or per slice.
__global__ void merge_start_kernel(int64_t m, int64_t nnz, int32_t origin,
                                   const int32_t *__restrict__ rowptr, int64_t items_per_block,
                                   int64_t nblocks, int64_t *__restrict__ start_rows)
{
    const int64_t b = blockIdx.x;
    if (b >= nblocks) return;
    const int64_t r = wave_merge_search(rowptr, origin, m, nnz, b * items_per_block);
    if (__lane_id() == 0) start_rows[b] = r;
}

__global__ void sliced_start_kernel(int64_t m, SliceInfo info, const int32_t *__restrict__ rowptr_all,
                                    int64_t nb, int64_t tile, int64_t *__restrict__ start_rows)
{
    const int s = blockIdx.x % NUM_XCD;
    const int64_t lb = blockIdx.x / NUM_XCD;
    const int64_t nnz_s = info.off[s + 1] - info.off[s];
    const int64_t d = lb * info.tiles[s] * tile;
    int64_t r = -1;
    if (d < m + nnz_s)
        r = wave_merge_search(rowptr_all + s * (m + 1), info.off[s], m, nnz_s, d);
    if (__lane_id() == 0) start_rows[s * nb + lb] = r;
}

// ---- sliced layout build: a stable partition of the entries by column slice.
//
// Slice s of the layout holds, in their original (row-major) order, the
// entries whose column lies in [s*w, (s+1)*w).  So the position of entry p is
// off[s] + (entries of slice s before p), and slice s's row pointer for row i
// is off[s] + (entries of slice s before rowptr[i]).  Both are prefix counts
// over the entry array, computed entry-parallel in SB_E-entry blocks, so the
// build costs the same whatever the row lengths (a row-parallel walk waits on
// the longest row, 100k entries in a power-law pattern).  Positions are always
// a permutation of [0, nnz), whatever rowptr holds.
constexpr int SB_THREADS = 256, SB_IPT = 8, SB_E = SB_THREADS * SB_IPT;
constexpr int SB_CKPT = 32;   // prefix checkpoint every SB_CKPT entries

__device__ __forceinline__ int slice_of(int64_t c, int64_t w)
{
    const int64_t s = c / w;          // c < 0 only on invalid input
    return s < 0 ? 0 : (s >= NUM_XCD ? NUM_XCD - 1 : (int)s);
}

// Eight 16-bit counters packed in four words: slice s in word s/2, half s%2.
struct Packed8 {
    uint32_t w[4];
};

__device__ __forceinline__ uint32_t packed_get(const Packed8 &p, int s)
{
    const uint32_t v = (s >> 1) == 0 ? p.w[0] : (s >> 1) == 1 ? p.w[1] : (s >> 1) == 2 ? p.w[2] : p.w[3];
    return (v >> (16 * (s & 1))) & 0xffffu;
}

__device__ __forceinline__ void packed_inc(Packed8 &p, int s)
{
    const uint32_t one = 1u << (16 * (s & 1));
#pragma unroll
    for (int k = 0; k < 4; ++k) p.w[k] += (s >> 1) == k ? one : 0u;
}

// bcnt[s*nblk + b] = entries of slice s in entry block b.
__global__ __launch_bounds__(SB_THREADS) void slice_block_count_kernel(int64_t nnz, int32_t origin,
                                                                       const int32_t *__restrict__ colind,
                                                                       int64_t w, int64_t nblk,
                                                                       int32_t *__restrict__ bcnt)
{
    __shared__ uint32_t wsum[SB_THREADS / 64][4];
    const int t = threadIdx.x;
    const int64_t e0 = (int64_t)blockIdx.x * SB_E;
    Packed8 c = {{0, 0, 0, 0}};
#pragma unroll
    for (int k = 0; k < SB_IPT; ++k) {
        const int64_t p = e0 + k * SB_THREADS + t;
        if (p < nnz) packed_inc(c, slice_of((int64_t)colind[p] - origin, w));
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) c.w[k] += __shfl_xor(c.w[k], off, 64);
    if (__lane_id() == 0)
#pragma unroll
        for (int k = 0; k < 4; ++k) wsum[t >> 6][k] = c.w[k];
    __syncthreads();
    if (t < NUM_XCD) {
        uint32_t v = 0;
#pragma unroll
        for (int q = 0; q < SB_THREADS / 64; ++q) v += (wsum[q][t >> 1] >> (16 * (t & 1))) & 0xffffu;
        bcnt[t * nblk + blockIdx.x] = (int32_t)v;
    }
}

// With bstart = the exclusive scan of bcnt (slice-major, so bstart[s*nblk+b]
// = off[s] + slice-s entries of blocks before b): places entry block b's
// entries and writes the prefix checkpoints ckpt[g*8 + s] = slice s's
// position for the entries before g*SB_CKPT.
template <typename T>
__global__ __launch_bounds__(SB_THREADS) void slice_place_kernel(
    int64_t nnz, int32_t origin, const int32_t *__restrict__ colind, const T *__restrict__ val, int64_t w,
    int64_t nblk, const int32_t *__restrict__ bstart, int32_t *__restrict__ ckpt,
    int32_t *__restrict__ colind_all, T *__restrict__ val_all, int32_t *__restrict__ perm)
{
    __shared__ uint8_t sl[SB_E];
    __shared__ int32_t qloc[SB_E];
    __shared__ uint32_t wsum[SB_THREADS / 64][4];
    __shared__ int32_t base[NUM_XCD];
    const int t = threadIdx.x, lane = __lane_id(), wave = t >> 6;
    const int64_t e0 = (int64_t)blockIdx.x * SB_E;
    if (t < NUM_XCD) base[t] = bstart[t * nblk + blockIdx.x];
    int32_t c[SB_IPT];
#pragma unroll
    for (int k = 0; k < SB_IPT; ++k) {
        const int64_t p = e0 + k * SB_THREADS + t;
        c[k] = p < nnz ? colind[p] - origin : 0;
        sl[k * SB_THREADS + t] = p < nnz ? (uint8_t)slice_of(c[k], w) : (uint8_t)NUM_XCD;
    }
    __syncthreads();
    // Thread t owns entries t*SB_IPT .. t*SB_IPT+7 of the block (in order).
    uint8_t mine[SB_IPT];
    Packed8 own = {{0, 0, 0, 0}};
#pragma unroll
    for (int j = 0; j < SB_IPT; ++j) {
        mine[j] = sl[t * SB_IPT + j];
        if (mine[j] < NUM_XCD) packed_inc(own, mine[j]);
    }
    Packed8 inc = own;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t v = __shfl_up(inc.w[k], off, 64);
            if (lane >= off) inc.w[k] += v;
        }
    if (lane == 63)
#pragma unroll
        for (int k = 0; k < 4; ++k) wsum[wave][k] = inc.w[k];
    __syncthreads();
    Packed8 pre;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        pre.w[k] = inc.w[k] - own.w[k];
        for (int q = 0; q < wave; ++q) pre.w[k] += wsum[q][k];
    }
#pragma unroll
    for (int j = 0; j < SB_IPT; ++j) {
        const int jj = t * SB_IPT + j;
        const int64_t e = e0 + jj;
        if (jj % SB_CKPT == 0 && e < nnz) {
            const int64_t g = e / SB_CKPT;
#pragma unroll
            for (int s = 0; s < NUM_XCD; ++s) ckpt[g * NUM_XCD + s] = base[s] + (int32_t)packed_get(pre, s);
        }
        if (mine[j] < NUM_XCD) {
            qloc[jj] = base[mine[j]] + (int32_t)packed_get(pre, mine[j]);
            packed_inc(pre, mine[j]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < SB_IPT; ++k) {
        const int jj = k * SB_THREADS + t;
        const int64_t p = e0 + jj;
        if (p < nnz) {
            const int32_t q = qloc[jj];
            colind_all[q] = (int32_t)(c[k] - (int64_t)sl[jj] * w);
            val_all[q] = val[p];
            perm[q] = (int32_t)p;
        }
    }
}

// rowptr_all[s*(m+1) + i] = slice s's position for the entries before row i:
// the checkpoint below rowptr[i] plus at most SB_CKPT-1 entries counted.
__global__ void slice_rowptr_kernel(int64_t m, int64_t nnz, int32_t origin, const int32_t *__restrict__ rowptr,
                                    const int32_t *__restrict__ colind, int64_t w, int64_t nblk,
                                    const int32_t *__restrict__ bstart, const int32_t *__restrict__ ckpt,
                                    int32_t *__restrict__ rowptr_all)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i > m) return;
    int64_t e = (int64_t)rowptr[i] - origin;
    e = e < 0 ? 0 : (e > nnz ? nnz : e);
    int32_t v[NUM_XCD];
    if (e == nnz) {
        // Past the last entry: every slice's end, off[s+1].
#pragma unroll
        for (int s = 0; s < NUM_XCD; ++s) v[s] = s + 1 < NUM_XCD ? bstart[(s + 1) * nblk] : (int32_t)nnz;
    } else {
        const int64_t g = e / SB_CKPT;
#pragma unroll
        for (int s = 0; s < NUM_XCD; ++s) v[s] = ckpt[g * NUM_XCD + s];
        for (int64_t k = g * SB_CKPT; k < e; ++k) {
            const int sk = slice_of((int64_t)colind[k] - origin, w);
#pragma unroll
            for (int s = 0; s < NUM_XCD; ++s) v[s] += s == sk ? 1 : 0;
        }
    }
#pragma unroll
    for (int s = 0; s < NUM_XCD; ++s) rowptr_all[s * (m + 1) + i] = v[s];
}

template <typename T>
__global__ void gather_values_kernel(int64_t nnz, const int32_t *__restrict__ perm,
                                     const T *__restrict__ src, T *__restrict__ dst)
{
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q < nnz) dst[q] = src[perm[q]];
}

struct SpmvGrid {
    int64_t tiles_per_block = 1;
    int64_t nblocks = 0;
    bool pf = false;      // prefetching plain kernel
};

// Items per thread (tile = 256 * ipt merge items): JLUST_HIP_SPMV_IPT in
// {4, 8}, default 8.
int spmv_ipt()
{
    static const int v = [] {
        const char *e = getenv("JLUST_HIP_SPMV_IPT");
        const int x = e ? atoi(e) : 8;
        return x == 4 ? 4 : 8;
    }();
    return v;
}

#define JLUST_SPMV_IPT_DISPATCH(ipt, F) ((ipt) == 4 ? F(4) : F(8))

// Merge-kernel variant: plain (row ends, then col/val, then x, per tile),
// plain with register prefetch, or column-sliced (prefetching).
enum SpmvKind { SPMV_PLAIN = 0, SPMV_PLAIN_PF = 1, SPMV_SLICED = 2 };

// JLUST_HIP_SPMV_PF=1 selects the prefetching plain kernel (default off).
bool spmv_plain_pf()
{
    static const bool v = [] {
        const char *e = getenv("JLUST_HIP_SPMV_PF");
        return e && e[0] == '1';
    }();
    return v;
}

template <typename T, int IPT, int KIND>
int spmv_occupancy_ipt(int dev, int *occ_out)
{
    static int occ_cache[64] = {};
    int &occ = occ_cache[dev & 63];
    if (occ == 0) {
        int nb = 0;
        if (KIND == SPMV_SLICED)
            JLUST_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, csr_spmv_sliced_kernel<T, SPMV_BLOCK, IPT, false>, SPMV_BLOCK, 0));
        else {
            // The grid is sized before beta is known: the smaller occupancy of
            // the beta == 0 and beta != 0 instances.
            int nb2 = 0;
            JLUST_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb, csr_spmv_merge_kernel<T, SPMV_BLOCK, IPT, KIND == SPMV_PLAIN_PF, true>,
                SPMV_BLOCK, 0));
            JLUST_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &nb2, csr_spmv_merge_kernel<T, SPMV_BLOCK, IPT, KIND == SPMV_PLAIN_PF, false>,
                SPMV_BLOCK, 0));
            nb = nb2 < nb ? nb2 : nb;
        }
        occ = nb > 0 ? nb : 1;
    }
    *occ_out = occ;
    return JLUST_STATUS_SUCCESS;
}

template <typename T>
int spmv_occupancy(int dev, int ipt, int kind, int *occ_out)
{
#define F(I)                                                                         \
    (kind == SPMV_SLICED     ? spmv_occupancy_ipt<T, I, SPMV_SLICED>(dev, occ_out)    \
     : kind == SPMV_PLAIN_PF ? spmv_occupancy_ipt<T, I, SPMV_PLAIN_PF>(dev, occ_out)  \
                             : spmv_occupancy_ipt<T, I, SPMV_PLAIN>(dev, occ_out))
    return JLUST_SPMV_IPT_DISPATCH(ipt, F);
#undef F
}

template <typename T>
int spmv_grid(int64_t m, int64_t nnz, int ipt, SpmvGrid *g)
{
    const int64_t TILE = (int64_t)SPMV_BLOCK * ipt;
    int dev = 0, occ = 1;
    if (int st = require_device(&dev)) return st;
    // The prefetching kernel's clamped loads need at least one nonzero.
    g->pf = spmv_plain_pf() && nnz > 0;
    if (int st = spmv_occupancy<T>(dev, ipt, g->pf ? SPMV_PLAIN_PF : SPMV_PLAIN, &occ)) return st;
    int64_t target = (int64_t)occ * device_info(dev).cu_count;
    if (target < 1) target = 1;
    const int64_t ntiles = (m + nnz + TILE - 1) / TILE;
    // Rounded up, so that nblocks <= target: every block is resident at once
    // and no block runs as a tail after the others.
    g->tiles_per_block = (ntiles + target - 1) / target;
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
                const SpmvGrid &g, int ipt, const int64_t *start_rows, int64_t *carry_row,
                T *carry_val, hipStream_t stream)
{
    // Whole XCD groups: logical blocks past g.nblocks return at once.
    const unsigned launch = (unsigned)((g.nblocks + NUM_XCD - 1) / NUM_XCD * NUM_XCD);
#define H(I, P, B)                                                                                \
    hipLaunchKernelGGL((csr_spmv_merge_kernel<T, SPMV_BLOCK, I, P, B>), dim3(launch),              \
                       dim3(SPMV_BLOCK), 0, stream, m, nnz, origin, rowptr, colind, val, x, y,    \
                       alpha, beta, g.tiles_per_block, start_rows, carry_row, carry_val)
#define G(I, P) do { if (beta == T(0)) H(I, P, true); else H(I, P, false); } while (0)
#define F(I) do { if (g.pf) G(I, true); else G(I, false); } while (0)
    if (ipt == 4) F(4);
    else F(8);
#undef F
#undef G
#undef H
    if (int st = check_launch("csr_spmv_merge_kernel")) return st;
    // A single block ends on the last row end, so it never leaves a carry.
    if (g.nblocks > 1) {
        hipLaunchKernelGGL((spmv_carry_fixup_kernel<T>), dim3((unsigned)((g.nblocks + 255) / 256)),
                           dim3(256), 0, stream, g.nblocks, (int64_t)1, carry_row, carry_val, y,
                           (int64_t)0, alpha);
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
    const int ipt = spmv_ipt();
    if (int st = spmv_grid<T>(m, nnz, ipt, &g)) return st;
    void *ws = nullptr;
    const size_t rows_bytes = align_up(sizeof(int64_t) * (size_t)g.nblocks, 256);
    if (int st = scratch(stream, rows_bytes + sizeof(T) * (size_t)g.nblocks, &ws)) return st;
    int64_t *carry_row = (int64_t *)ws;
    T *carry_val = (T *)((char *)ws + rows_bytes);
    return spmv_launch<T>(m, nnz, origin, rowptr, colind, val, alpha, x, beta, y, g, ipt, nullptr,
                          carry_row, carry_val, (hipStream_t)stream);
}

// Vector kernel for plans of short, even rows: LPR lanes per row, each lane
// striding the row by LPR,
// partial sums combined with xor-shuffles.  No LDS, no barriers, no carries:
// every wave holds 64/LPR rows, so a small matrix still puts many waves in
// flight (the merge kernel spends one 2048-item tile per block there).  All
// waves of such a matrix are resident at once, so the time is one wave's
// chain of dependent loads: both row pointers are loaded together, and each
// step issues VEC_U of the lane's entries at once (indices clamped into the
// row, products of the clamped copies dropped by a select), so a row of
// 4*LPR entries costs one rowptr -> colind -> x chain rather than four.
constexpr int VEC_U = 4;

// UNI: every row holds exactly ulen entries (rowptr[i] = origin + i*ulen, checked
// when the plan was made), so the row bounds are computed instead of loaded and
// the column/value loads are the first memory access.
template <typename T, int LPR, bool BZ, bool UNI>
__global__ __launch_bounds__(256) void csr_spmv_vector_kernel(int64_t m, int32_t origin,
                                                              const int32_t *__restrict__ rowptr,
                                                              const int32_t *__restrict__ colind,
                                                              const T *__restrict__ val, const T *__restrict__ x,
                                                              T *__restrict__ y, T alpha, T beta,
                                                              int32_t ulen)
{
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = t / LPR;
    const int sub = (int)(t % LPR);
    const int64_t r = row < m ? row : m - 1;            // clamped: loads stay in bounds
    int64_t lo, hi;
    if constexpr (UNI) {
        lo = r * ulen;
        hi = row < m ? lo + ulen : lo;
    } else {
        int32_t rp0 = rowptr[r], rp1 = rowptr[r + 1];
        // Both values are needed here, so both loads are issued before the first
        // wait (otherwise the second sinks under the row < m branch below).
        __asm__ volatile("" : "+v"(rp0), "+v"(rp1));
        lo = (int64_t)rp0 - origin;
        hi = row < m ? (int64_t)rp1 - origin : lo;
    }
    T acc = T(0);
    for (int64_t p0 = lo + sub; p0 < hi; p0 += VEC_U * LPR) {
        int32_t c[VEC_U];
        T v[VEC_U], xv[VEC_U];
#pragma unroll
        for (int u = 0; u < VEC_U; ++u) {
            const int64_t p = min(p0 + u * LPR, hi - 1);
            c[u] = colind[p];
            v[u] = val[p];
        }
#pragma unroll
        for (int u = 0; u < VEC_U; ++u) xv[u] = x[c[u] - origin];
#pragma unroll
        for (int u = 0; u < VEC_U; ++u) {
            const T a = acc + v[u] * xv[u];
            acc = p0 + u * LPR < hi ? a : acc;
        }
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, LPR);
    if (sub == 0 && row < m) y[row] = BZ ? alpha * acc : alpha * acc + beta * y[row];
}

// out[0] = max row length: a grid-stride maximum per thread, reduced per
// block in LDS, one atomicMax per block.
__global__ __launch_bounds__(256) void row_len_max_kernel(int64_t m, const int32_t *__restrict__ rowptr,
                                                          int32_t *__restrict__ out)
{
    __shared__ int32_t s_w[4];
    int32_t len = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < m; i += (int64_t)gridDim.x * 256)
        len = max(len, rowptr[i + 1] - rowptr[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) len = max(len, __shfl_xor(len, off, 64));
    if (__lane_id() == 0) s_w[threadIdx.x >> 6] = len;
    __syncthreads();
    if (threadIdx.x == 0) {
        const int32_t b = max(max(s_w[0], s_w[1]), max(s_w[2], s_w[3]));
        if (b > 0) atomicMax(out, b);
    }
}

// Lanes per row of the vector kernel for a plan (0 = merge kernel): the
// smallest power of two >= 2 giving a lane about 4 entries of an average row,
// when rows average at most 64 entries and the longest needs at most 16 steps
// per lane.  JLUST_HIP_SPMV_VECTOR=0 disables it, =L forces L lanes per row.
// Synchronises `s`.
// flag[0] = 1 if some row pointer differs from origin + i*len.
__global__ __launch_bounds__(256) void row_uniform_kernel(int64_t m, int32_t origin, int32_t len,
                                                          const int32_t *__restrict__ rowptr,
                                                          int32_t *__restrict__ flag)
{
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i <= m; i += (int64_t)gridDim.x * 256)
        if ((int64_t)rowptr[i] != origin + i * len) flag[0] = 1;
}

// Lanes per row of the vector kernel (0: rows too long for it) and, in
// *ulen_out, the common row length when every row has the same one (else 0).
int vector_lanes(int64_t m, int64_t nnz, int32_t origin, const int32_t *rowptr, hipStream_t s,
                 int *lpr_out, int32_t *ulen_out)
{
    *lpr_out = 0;
    *ulen_out = 0;
    const char *e = getenv("JLUST_HIP_SPMV_VECTOR");
    if ((e && e[0] == '0') || m <= 0) return JLUST_STATUS_SUCCESS;
    const double avg = (double)nnz / (double)m;
    if (avg > 64.0) return JLUST_STATUS_SUCCESS;
    int lpr = 2;                                 // about 4 entries per lane on average
    while (lpr < 64 && 4 * lpr < avg) lpr <<= 1;
    const int forced = e ? atoi(e) : 0;          // JLUST_HIP_SPMV_VECTOR=L: L lanes per row
    if (forced >= 2 && forced <= 64 && (forced & (forced - 1)) == 0) lpr = forced;
    void *ws = nullptr;
    if (int st = scratch(s, 2 * sizeof(int32_t), &ws)) return st;
    auto *mx = (int32_t *)ws;                    // [0] longest row, [1] non-uniform flag
    JLUST_HIP_TRY(hipMemsetAsync(mx, 0, 2 * sizeof(int32_t), s));
    const int64_t nblk = min((int64_t)1024, (m + 255) / 256);
    hipLaunchKernelGGL(row_len_max_kernel, dim3((unsigned)nblk), dim3(256), 0, s, m, rowptr, mx);
    if (int st = check_launch("row_len_max_kernel")) return st;
    const bool may_be_uniform = nnz % m == 0 && nnz / m <= INT32_MAX;
    if (may_be_uniform) {
        hipLaunchKernelGGL(row_uniform_kernel, dim3((unsigned)nblk), dim3(256), 0, s, m, origin,
                           (int32_t)(nnz / m), rowptr, mx + 1);
        if (int st = check_launch("row_uniform_kernel")) return st;
    }
    int32_t h[2] = {0, 1};
    JLUST_HIP_TRY(hipMemcpyAsync(h, mx, sizeof(h), hipMemcpyDeviceToHost, s));
    JLUST_HIP_TRY(hipStreamSynchronize(s));
    if (h[0] <= 16 * lpr) {                      // the longest row: at most 16 steps per lane
        *lpr_out = lpr;
        if (may_be_uniform && h[1] == 0) *ulen_out = (int32_t)(nnz / m);
    }
    return JLUST_STATUS_SUCCESS;
}

// Counts the entries whose column lies within +-w of their row's diagonal
// position r*n/m, on every LOC_SAMPLE-th chunk of LOC_CHUNK consecutive
// entries: each thread walks one chunk from the row found by binary search;
// count[0] gets the local entries, count[1] the entries examined (one atomic
// each per wave).  The test is a 90 % threshold, so a fixed 1-in-8 sample of
// chunks spread over the whole matrix decides it at an eighth of the cost.
constexpr int LOC_CHUNK = 64;
constexpr int LOC_SAMPLE = 8;

__global__ __launch_bounds__(256) void locality_kernel(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                                       const int32_t *__restrict__ rowptr,
                                                       const int32_t *__restrict__ colind, int64_t w,
                                                       unsigned long long *__restrict__ count)
{
    const int64_t k0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * (LOC_CHUNK * LOC_SAMPLE);
    unsigned long long local = 0, seen = 0;
    if (k0 < nnz) {
        int64_t lo = 0, hi = m;          // rowptr[lo] <= k0 < rowptr[hi] (relative to origin)
        while (hi - lo > 1) {
            const int64_t mid = (lo + hi) >> 1;
            if ((int64_t)rowptr[mid] - origin <= k0) lo = mid;
            else hi = mid;
        }
        int64_t r = lo;
        int64_t rend = (int64_t)rowptr[r + 1] - origin;
        const int64_t k1 = min(nnz, k0 + LOC_CHUNK);
        seen = (unsigned long long)(k1 - k0);
        for (int64_t k = k0; k < k1; ++k) {
            while (k >= rend && r < m - 1) {
                ++r;
                rend = (int64_t)rowptr[r + 1] - origin;
            }
            const int64_t d = r * n / m;
            const int64_t c = (int64_t)colind[k] - origin;
            local += (c >= d - w && c <= d + w) ? 1u : 0u;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        local += __shfl_xor(local, off, 64);
        seen += __shfl_xor(seen, off, 64);
    }
    if (__lane_id() == 0 && seen) {
        atomicAdd(&count[0], local);
        atomicAdd(&count[1], seen);
    }
}

// True when at least 90% of the entries gather from within half an XCD L2
// of x around their row's diagonal position: the rows one XCD runs (an
// eighth of the merge path, XCD-major) then share one L2-sized window of x,
// and slicing would only add its reduction pass.  Synchronises `s`.
template <typename T>
int mostly_local(int64_t m, int64_t n, int64_t nnz, int32_t origin, const int32_t *rowptr,
                 const int32_t *colind, hipStream_t s, bool *out)
{
    *out = false;
    if (m <= 0 || nnz <= 0) return JLUST_STATUS_SUCCESS;
    void *ws = nullptr;
    if (int st = scratch(s, 2 * sizeof(unsigned long long), &ws)) return st;
    auto *cnt = (unsigned long long *)ws;
    JLUST_HIP_TRY(hipMemsetAsync(cnt, 0, 2 * sizeof(*cnt), s));
    const int64_t threads = (nnz + LOC_CHUNK * LOC_SAMPLE - 1) / (LOC_CHUNK * LOC_SAMPLE);
    const int64_t w = (int64_t)(SLICE_MIN_X_BYTES / sizeof(T) / 2);
    hipLaunchKernelGGL(locality_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, m, n, nnz,
                       origin, rowptr, colind, w, cnt);
    if (int st = check_launch("locality_kernel")) return st;
    unsigned long long h[2] = {0, 0};
    JLUST_HIP_TRY(hipMemcpyAsync(h, cnt, sizeof(h), hipMemcpyDeviceToHost, s));
    JLUST_HIP_TRY(hipStreamSynchronize(s));
    *out = (double)h[0] >= 0.9 * (double)h[1];
    return JLUST_STATUS_SUCCESS;
}

// Slice or not: JLUST_HIP_SPMV_SLICE=0 never, =1 always, unset = when x is
// larger than one XCD's L2, rows are long enough, and the gathers are not
// mostly local.  Slices carry every row 8 times (8 merge paths of m row ends
// plus an 8 x m partial-sum reduction, ~45-50 ps per row on MI355X) and save
// ~9 ps per nonzero gathering from a 32 MB x, ~5 ps from an 8 MB x (random
// columns, 4M x 4M and 4M x 1M matrices): the break-even mean row length is
// ~5-6 and ~9 entries, so slicing needs nnz >= L * m with L by x's size.
enum Layout { LAYOUT_ROWS = 0, LAYOUT_SLICED = 1, LAYOUT_BINNED = 2 };

// The LDS-binned layout costs a fixed time (its bin pass is a chain of one
// step per column slice: ~85 us with 256 slices, ~35 us with the 31-123 wide
// slices of an x of 4-16 MB) plus ~3.5-5 ns per 1000 entries; scattered
// gathers of an x beyond the L2 cost the row-order kernels ~16 ns per 1000
// entries at 32 MB, ~11 ns at 8 MB and ~6 ns at 4 MB.  Measured crossovers
// (f64, random columns): 7M entries for x >= 24 MB, 6M for x >= 6 MB, 12M
// above 2 MB.
constexpr size_t BINNED_MIN_X_BYTES = (size_t)2 << 20;

int64_t binned_min_nnz(size_t xbytes)
{
    return xbytes >= ((size_t)24 << 20) ? 7000000 : xbytes >= ((size_t)6 << 20) ? 6000000 : 12000000;
}

// The layout of a prepared plan.  JLUST_HIP_SPMV_SLICE: 0 = row order, 1 =
// XCD column slices (n >= 8), 2 = LDS bins where they fit.  Default: row
// order while x fits the L2 or the columns are mostly local; otherwise LDS
// bins above binned_min_nnz entries (where they fit), else XCD slices from
// min_len entries per row once x exceeds one XCD's L2.
template <typename T>
int choose_layout(int value_type, int64_t m, int64_t n, int64_t nnz, int32_t origin,
                  const int32_t *rowptr, const int32_t *colind, hipStream_t s, int *out)
{
    const char *e = getenv("JLUST_HIP_SPMV_SLICE");
    *out = LAYOUT_ROWS;
    if (m <= 0 || nnz <= 0) return JLUST_STATUS_SUCCESS;   // the sliced kernel needs a nonzero
    if (e && e[0] == '0') return JLUST_STATUS_SUCCESS;
    if (e && e[0] == '1') {
        if (n >= NUM_XCD) *out = LAYOUT_SLICED;
        return JLUST_STATUS_SUCCESS;
    }
    if (e && e[0] == '2') {
        if (binned_fits(value_type, m, n, nnz)) *out = LAYOUT_BINNED;
        return JLUST_STATUS_SUCCESS;
    }
    const size_t xbytes = (size_t)n * sizeof(T);
    if (xbytes <= BINNED_MIN_X_BYTES) return JLUST_STATUS_SUCCESS;
    const bool bins = nnz >= binned_min_nnz(xbytes) && binned_fits(value_type, m, n, nnz);
    const int64_t min_len = xbytes >= ((size_t)24 << 20) ? 6 : xbytes >= ((size_t)6 << 20) ? 10 : 14;
    const bool slices = xbytes > SLICE_MIN_X_BYTES && nnz >= min_len * m;
    if (!bins && !slices) return JLUST_STATUS_SUCCESS;
    bool local = false;
    if (int st = mostly_local<T>(m, n, nnz, origin, rowptr, colind, s, &local)) return st;
    if (!local) *out = bins ? LAYOUT_BINNED : LAYOUT_SLICED;
    return JLUST_STATUS_SUCCESS;
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
    int device;
    int ipt;         // items per thread of the merge tiles
    void *mem;       // everything below lives in this allocation
    // unsliced
    jlust::SpmvGrid grid;
    int64_t *start_rows;
    int64_t *carry_row;
    void *carry_val;
    int vec_lpr = 0;   // > 0: vector kernel with this many lanes per row
    int32_t vec_ulen = 0;  // > 0: every row holds this many entries (bounds computed)
    // sliced
    bool sliced;
    int64_t slice_w;
    int64_t nb;                      // blocks per slice
    jlust::SliceInfo info;
    int32_t *rowptr_all;
    int32_t *colind_all;
    void *val_all;
    int32_t *perm;
    void *ypart;
    // COO plans (coo_plan.hip): the row-ordered CSR the plan runs on is owned
    // in coo_mem; coo_perm (null when the entries were already in row order)
    // maps its entries to the caller's, and coo_val holds the values in that
    // order.
    void *coo_mem = nullptr;
    const int32_t *coo_perm = nullptr;
    void *coo_val = nullptr;
    // LDS-binned layout (spmv_binned.hip), or null.
    jlust::BinnedLayout *binned = nullptr;
    int64_t bytes = 0;               // device memory held by the plan
};

namespace jlust {
int spmv_plan_adopt_coo(jlust_spmv_plan_t plan, void *mem, const int32_t *perm, void *val_copy, size_t bytes)
{
    plan->bytes += (int64_t)bytes;
    plan->coo_mem = mem;
    plan->coo_perm = perm;
    plan->coo_val = val_copy;
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust

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

// ------------------------------------------------- allocation-free SpMV call

// Carry slots of jlust_hip_csr_spmv_f64_i32_noalloc: carry rows (int64) in
// the first half, carry values (double) in the second.  The plain merge grid
// has one block per resident slot (occupancy x CUs: at most 2048 blocks of
// 256 threads on 256 CUs), so 4096 slots cover it with room to spare.  Every
// block of a launch writes its own slot before the fix-up kernel reads it,
// so nothing needs clearing between calls.  The array is never named in
// host code below except to take its device address.
constexpr int64_t NOALLOC_MAX_BLOCKS = 4096;
constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)NOALLOC_MAX_BLOCKS * (sizeof(int64_t) + sizeof(double));
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_noalloc_mu;
void *g_noalloc_ptr[NOALLOC_MAX_DEVICES];   // device address of `scratch` on each device

// The device address of this device's copy of `scratch`, looked up once per
// device (with that device current) by hipGetSymbolAddress.
int noalloc_scratch(int dev, void **out)
{
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "csr_spmv_noalloc: device %d beyond the %d supported",
                    dev, NOALLOC_MAX_DEVICES);
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(JLUST_STATUS_HIP_ERROR, "hipGetSymbolAddress(scratch) returned null");
        g_noalloc_ptr[dev] = p;
    }
    *out = g_noalloc_ptr[dev];
    return JLUST_STATUS_SUCCESS;
}
}  // namespace

extern "C" int jlust_hip_csr_spmv_f64_i32_noalloc(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                                  const int32_t *rowptr, const int32_t *colind,
                                                  const double *val, double alpha, const double *x,
                                                  double beta, double *y, jlust_stream_t stream)
{
    clear_error();
    if (int st = check_spmv_args(m, n, nnz, origin, rowptr, colind, val, x, y)) return st;
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    void *base = nullptr;
    if (int st = noalloc_scratch(dev, &base)) return st;
    if (m == 0) return JLUST_STATUS_SUCCESS;
    SpmvGrid g;
    const int ipt = spmv_ipt();
    if (int st = spmv_grid<double>(m, nnz, ipt, &g)) return st;
    if (g.nblocks > NOALLOC_MAX_BLOCKS)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "csr_spmv_noalloc: the launch needs %lld carry slots, the static scratch holds %lld",
                    (long long)g.nblocks, (long long)NOALLOC_MAX_BLOCKS);
    int64_t *carry_row = (int64_t *)base;
    double *carry_val = (double *)((char *)base + sizeof(int64_t) * NOALLOC_MAX_BLOCKS);
    return spmv_launch<double>(m, nnz, origin, rowptr, colind, val, alpha, x, beta, y, g, ipt, nullptr,
                               carry_row, carry_val, (hipStream_t)stream);
}

// The byte limit of a plan's copied layout (JLUST_HIP_PLAN_MAX_BYTES; 0 or
// unset: none), read at each plan_create.
static int64_t plan_max_bytes()
{
    const char *e = getenv("JLUST_HIP_PLAN_MAX_BYTES");
    return e ? (int64_t)strtoll(e, nullptr, 10) : 0;
}

// After an allocation that failed with out of memory: the runtime's sticky
// last error and this thread's message are cleared before another layout is
// tried (a later check_launch reads hipGetLastError).
static void fallback_clear()
{
    (void)hipGetLastError();
    clear_error();
}

// Temporaries of plan_build_sliced: block counts and checkpoints.
static size_t sliced_build_temp_bytes(int64_t nnz)
{
    const int64_t nblk = (nnz + SB_E - 1) / SB_E, nck = (nnz + SB_CKPT - 1) / SB_CKPT;
    return align_up(sizeof(int32_t) * NUM_XCD * (size_t)nblk, 256) + sizeof(int32_t) * NUM_XCD * (size_t)nck;
}

template <typename T>
static int plan_build_sliced(jlust_spmv_plan *p, jlust_stream_t stream)
{
    hipStream_t s = (hipStream_t)stream;
    const int64_t m = p->m, nnz = p->nnz;
    const int64_t nblk = (nnz + SB_E - 1) / SB_E;   // nnz > 0 on the sliced path
    const int64_t nck = (nnz + SB_CKPT - 1) / SB_CKPT;
    // Temporary: block counts (scanned in place to block starts) and checkpoints.
    const size_t sz_b = align_up(sizeof(int32_t) * NUM_XCD * (size_t)nblk, 256);
    void *tmp = nullptr;
    JLUST_HIP_TRY(hipMalloc(&tmp, sz_b + sizeof(int32_t) * NUM_XCD * (size_t)nck));
    int32_t *bstart = (int32_t *)tmp;
    int32_t *ckpt = (int32_t *)((char *)tmp + sz_b);
    int st = JLUST_STATUS_SUCCESS;
    hipLaunchKernelGGL(slice_block_count_kernel, dim3((unsigned)nblk), dim3(SB_THREADS), 0, s, nnz, p->origin,
                       p->colind, p->slice_w, nblk, bstart);
    st = check_launch("slice_block_count_kernel");
    if (!st) st = exclusive_scan_i32(bstart, bstart, NUM_XCD * nblk, stream);
    if (!st) {
        hipLaunchKernelGGL((slice_place_kernel<T>), dim3((unsigned)nblk), dim3(SB_THREADS), 0, s, nnz, p->origin,
                           p->colind, (const T *)p->val, p->slice_w, nblk, bstart, ckpt, p->colind_all,
                           (T *)p->val_all, p->perm);
        st = check_launch("slice_place_kernel");
    }
    if (!st) {
        hipLaunchKernelGGL(slice_rowptr_kernel, dim3((unsigned)((m + 1 + 255) / 256)), dim3(256), 0, s, m, nnz,
                           p->origin, p->rowptr, p->colind, p->slice_w, nblk, bstart, ckpt, p->rowptr_all);
        st = check_launch("slice_rowptr_kernel");
    }
    // Slice offsets off[s] = the first block's start in each slice.
    int32_t firsts[NUM_XCD];
    for (int k = 0; k < NUM_XCD && !st; ++k) {
        const hipError_t e = hipMemcpyAsync(&firsts[k], bstart + k * nblk, sizeof(int32_t),
                                            hipMemcpyDeviceToHost, s);
        if (e != hipSuccess) st = hip_fail(e, "hipMemcpyAsync(slice offsets)");
    }
    const hipError_t es = hipStreamSynchronize(s);
    (void)hipFree(tmp);
    if (st) return st;
    if (es != hipSuccess) return hip_fail(es, "hipStreamSynchronize(sliced plan build)");
    for (int k = 0; k < NUM_XCD; ++k) p->info.off[k] = firsts[k];
    p->info.off[NUM_XCD] = nnz;
    const int64_t TILE = (int64_t)SPMV_BLOCK * p->ipt;
    int64_t maxb = 1;
    for (int k = 0; k < NUM_XCD; ++k) {
        const int64_t ntiles = (m + p->info.off[k + 1] - p->info.off[k] + TILE - 1) / TILE;
        p->info.tiles[k] = ntiles;   // provisional: blocks needed at one tile each
        if (ntiles > maxb) maxb = ntiles;
    }
    int occ = 1;
    if (int st = spmv_occupancy<T>(p->device, p->ipt, SPMV_SLICED, &occ)) return st;
    int64_t target = (int64_t)occ * device_info(p->device).cu_count / NUM_XCD;
    if (target < 1) target = 1;
    // Rounded up, so that nb <= target (one resident wave of blocks).
    int64_t tpb = (maxb + target - 1) / target;
    if (tpb < 1) tpb = 1;
    p->nb = (maxb + tpb - 1) / tpb;
    for (int k = 0; k < NUM_XCD; ++k) {
        const int64_t ntiles = p->info.tiles[k];
        int64_t t = (ntiles + p->nb - 1) / p->nb;
        p->info.tiles[k] = t < 1 ? 1 : t;
    }
    return JLUST_STATUS_SUCCESS;
}

static int csr_spmv_plan_create_body(int64_t m, int64_t n, int64_t nnz, int32_t origin,
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
    const size_t tsz = value_type == 0 ? sizeof(double) : sizeof(float);
    auto *p = new jlust_spmv_plan();
    p->m = m;
    p->n = n;
    p->nnz = nnz;
    p->origin = origin;
    p->value_type = value_type;
    p->rowptr = rowptr;
    p->colind = colind;
    p->val = val;
    p->device = dev;
    p->ipt = spmv_ipt();
    hipStream_t s = (hipStream_t)stream;
    // (The sliced kernel's clamped prefetch needs at least one nonzero.)
    int layout = LAYOUT_ROWS;
    int st = value_type == 0
                 ? choose_layout<double>(value_type, m, n, nnz, origin, rowptr, colind, s, &layout)
                 : choose_layout<float>(value_type, m, n, nnz, origin, rowptr, colind, s, &layout);
    if (st) {
        delete p;
        return st;
    }
    // Layouts that copy the matrix (binned, sliced) fall back to the merge or
    // vector kernels on the caller's arrays when they cannot be allocated:
    // hipMalloc out of memory, or the layout with its build temporaries above
    // JLUST_HIP_PLAN_MAX_BYTES.
    const int64_t cap = plan_max_bytes();
    if (layout == LAYOUT_BINNED) {
        st = binned_build(&p->binned, value_type, m, n, nnz, origin, rowptr, colind, val, cap, s);
        if (!st) {
            p->bytes = binned_bytes(p->binned);
            *plan_out = p;
            return JLUST_STATUS_SUCCESS;
        }
        if (st != JLUST_STATUS_OUT_OF_MEMORY) {
            delete p;
            return st;
        }
        fallback_clear();
        layout = LAYOUT_ROWS;
        st = JLUST_STATUS_SUCCESS;
    }
    p->sliced = layout == LAYOUT_SLICED;
    if (p->sliced) {
        p->slice_w = (n + NUM_XCD - 1) / NUM_XCD;
        // Upper bound of blocks per slice: one tile each.
        const int64_t tile = (int64_t)SPMV_BLOCK * p->ipt;
        const int64_t nb_max = (m + nnz + tile - 1) / tile + 1;
        const size_t sz_rp = align_up(sizeof(int32_t) * NUM_XCD * (size_t)(m + 1), 256);
        const size_t sz_ci = align_up(sizeof(int32_t) * (size_t)(nnz > 0 ? nnz : 1), 256);
        const size_t sz_v = align_up(tsz * (size_t)(nnz > 0 ? nnz : 1), 256);
        const size_t sz_y = align_up(tsz * NUM_XCD * (size_t)m, 256);
        const size_t sz_sr = align_up(sizeof(int64_t) * NUM_XCD * (size_t)nb_max, 256);
        const size_t sz_cv = align_up(tsz * NUM_XCD * (size_t)nb_max, 256);
        const size_t total = sz_rp + 2 * sz_ci + sz_v + sz_y + 2 * sz_sr + sz_cv;
        if (cap > 0 && (int64_t)(total + sliced_build_temp_bytes(nnz)) > cap) {
            st = fail(JLUST_STATUS_OUT_OF_MEMORY, "sliced spmv layout: %lld bytes above JLUST_HIP_PLAN_MAX_BYTES",
                      (long long)total);
        } else {
            const hipError_t e = hipMalloc(&p->mem, total);
            if (e != hipSuccess) {
                p->mem = nullptr;
                st = hip_fail(e, "hipMalloc(sliced spmv plan)");
            }
        }
        if (!st) {
            char *b = (char *)p->mem;
            p->rowptr_all = (int32_t *)b;  b += sz_rp;
            p->colind_all = (int32_t *)b;  b += sz_ci;
            p->perm = (int32_t *)b;        b += sz_ci;
            p->val_all = b;                b += sz_v;
            p->ypart = b;                  b += sz_y;
            p->start_rows = (int64_t *)b;  b += sz_sr;
            p->carry_row = (int64_t *)b;   b += sz_sr;
            p->carry_val = b;
            p->bytes = (int64_t)total;
            st = value_type == 0 ? plan_build_sliced<double>(p, stream) : plan_build_sliced<float>(p, stream);
            if (!st && p->nb > nb_max) st = fail(JLUST_STATUS_HIP_ERROR, "spmv plan: block count overflow");
            if (!st) {
                hipLaunchKernelGGL(sliced_start_kernel, dim3((unsigned)(NUM_XCD * p->nb)), dim3(64), 0, s,
                                   m, p->info, p->rowptr_all, p->nb, (int64_t)SPMV_BLOCK * p->ipt,
                                   p->start_rows);
                st = check_launch("sliced_start_kernel");
            }
        }
        if (st == JLUST_STATUS_OUT_OF_MEMORY) {
            (void)hipStreamSynchronize(s);
            if (p->mem) (void)hipFree(p->mem);
            p->mem = nullptr;
            p->bytes = 0;
            p->sliced = false;
            fallback_clear();
            st = JLUST_STATUS_SUCCESS;
        }
    }
    if (!st && !p->sliced) {
        if (m > 0) {
            st = value_type == 0 ? spmv_grid<double>(m, nnz, p->ipt, &p->grid)
                                 : spmv_grid<float>(m, nnz, p->ipt, &p->grid);
            if (!st) st = vector_lanes(m, nnz, origin, rowptr, s, &p->vec_lpr, &p->vec_ulen);
            if (st) { delete p; return st; }
        }
        const size_t nb = (size_t)(p->grid.nblocks > 0 ? p->grid.nblocks : 1);
        const size_t sz_rows = align_up(sizeof(int64_t) * nb, 256);
        hipError_t e = hipMalloc(&p->mem, 2 * sz_rows + tsz * nb);
        if (e != hipSuccess) { delete p; return hip_fail(e, "hipMalloc(spmv plan)"); }
        p->bytes = (int64_t)(2 * sz_rows + tsz * nb);
        p->start_rows = (int64_t *)p->mem;
        p->carry_row = (int64_t *)((char *)p->mem + sz_rows);
        p->carry_val = (char *)p->mem + 2 * sz_rows;
        if (m > 0 && p->vec_lpr == 0) {
            hipLaunchKernelGGL(merge_start_kernel, dim3((unsigned)p->grid.nblocks), dim3(64), 0, s, m,
                               nnz, origin, rowptr,
                               p->grid.tiles_per_block * (int64_t)(SPMV_BLOCK * p->ipt),
                               p->grid.nblocks, p->start_rows);
            st = check_launch("merge_start_kernel");
        }
    }
    if (st) {
        (void)hipStreamSynchronize(s);
        if (p->mem) (void)hipFree(p->mem);
        delete p;
        return st;
    }
    *plan_out = p;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_csr_spmv_plan_create(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                              int value_type, const int32_t *rowptr,
                                              const int32_t *colind, const void *val,
                                              jlust_stream_t stream, jlust_spmv_plan_t *plan_out)
{
    return jlust::host_guard("csr_spmv_plan_create", [&] {
        return csr_spmv_plan_create_body(m, n, nnz, origin, value_type, rowptr, colind, val, stream,
                                         plan_out);
    });
}

namespace jlust {
// Makes the plan read the values `val` (same pattern as the plan's), in stream
// order on s: merge and vector plans only take the pointer; a COO plan whose
// entries were reordered gathers them into its row-ordered copy first; the
// sliced and binned layouts gather them into their own slice-major copy.  A
// later execute on s (or anything ordered after s) sees them.
int plan_refresh(jlust_spmv_plan_t plan, const void *val, hipStream_t s)
{
    if (plan->coo_perm && plan->nnz > 0) {
        // COO entries in the caller's order -> the plan's row order.
        const unsigned grid = (unsigned)((plan->nnz + 255) / 256);
        if (plan->value_type == 0)
            hipLaunchKernelGGL((gather_values_kernel<double>), dim3(grid), dim3(256), 0, s, plan->nnz,
                               plan->coo_perm, (const double *)val, (double *)plan->coo_val);
        else
            hipLaunchKernelGGL((gather_values_kernel<float>), dim3(grid), dim3(256), 0, s, plan->nnz,
                               plan->coo_perm, (const float *)val, (float *)plan->coo_val);
        if (int st = check_launch("gather_values_kernel")) return st;
        val = plan->coo_val;
    }
    plan->val = val;
    if (plan->binned)
        if (int st = binned_update(plan->binned, val, s)) return st;
    if (plan->sliced && plan->nnz > 0) {
        const unsigned grid = (unsigned)((plan->nnz + 255) / 256);
        if (plan->value_type == 0)
            hipLaunchKernelGGL((gather_values_kernel<double>), dim3(grid), dim3(256), 0, s, plan->nnz,
                               plan->perm, (const double *)val, (double *)plan->val_all);
        else
            hipLaunchKernelGGL((gather_values_kernel<float>), dim3(grid), dim3(256), 0, s, plan->nnz,
                               plan->perm, (const float *)val, (float *)plan->val_all);
        if (int st = check_launch("gather_values_kernel")) return st;
    }
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust

extern "C" int jlust_hip_csr_spmv_plan_update_values(jlust_spmv_plan_t plan, const void *val,
                                                     jlust_stream_t stream)
{
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_update_values: null plan");
    if (bad_ptr(val, plan->nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_update_values: null values");
    // Stream-ordered, like a descriptor swap followed by work on the stream:
    // plans that copy the values (COO order, sliced and binned layouts) gather
    // them on `stream`; nothing waits on the host or on other streams.
    if (plan->coo_perm || plan->binned || plan->sliced) {
        int dev = 0;
        if (int st = require_device(&dev)) return st;
        if (dev != plan->device)
            return fail(JLUST_STATUS_INVALID_ARGUMENT,
                        "spmv_plan_update_values: plan belongs to device %d, current device is %d",
                        plan->device, dev);
    }
    return plan_refresh(plan, val, (hipStream_t)stream);
}

namespace jlust {
template <typename T>
int vector_launch(const jlust_spmv_plan_t p, int lpr, T alpha, const T *x, T beta, T *y, hipStream_t s)
{
    const int64_t threads = p->m * lpr;
    const dim3 grid((unsigned)((threads + 255) / 256));
    const T *val = (const T *)p->val;
#define VK(L, Z, U)                                                                                 \
    hipLaunchKernelGGL((csr_spmv_vector_kernel<T, L, Z, U>), grid, dim3(256), 0, s, p->m, p->origin,   \
                       p->rowptr, p->colind, val, x, y, alpha, beta, p->vec_ulen)
#define VZ(L, U) do { if (beta == T(0)) VK(L, true, U); else VK(L, false, U); } while (0)
#define V(L) do { if (p->vec_ulen > 0) VZ(L, true); else VZ(L, false); } while (0)
    switch (lpr) {
    case 2: V(2); break;
    case 4: V(4); break;
    case 8: V(8); break;
    case 16: V(16); break;
    case 32: V(32); break;
    default: V(64); break;
    }
#undef V
#undef VZ
#undef VK
    return check_launch("csr_spmv_vector_kernel");
}
}  // namespace jlust

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
    hipStream_t s = (hipStream_t)stream;
    if (plan->binned) {
        if constexpr (sizeof(T) == 8)
            return binned_execute_f64(plan->binned, alpha, x, beta, y, s);
        else
            return binned_execute_f32(plan->binned, alpha, x, beta, y, s);
    }
    if (!plan->sliced && plan->vec_lpr > 0)
        return vector_launch<T>(plan, plan->vec_lpr, alpha, x, beta, y, s);
    if (!plan->sliced)
        return spmv_launch<T>(plan->m, plan->nnz, plan->origin, plan->rowptr, plan->colind,
                              (const T *)plan->val, alpha, x, beta, y, plan->grid, plan->ipt,
                              plan->start_rows, plan->carry_row, (T *)plan->carry_val, s);
    const int64_t m = plan->m;
    T *ypart = (T *)plan->ypart;
    static const bool nt = [] {
        const char *e = getenv("JLUST_HIP_SPMV_SLICED_NT");
        return e && e[0] == '1';
    }();
#define G(I, N)                                                                                  \
    hipLaunchKernelGGL((csr_spmv_sliced_kernel<T, SPMV_BLOCK, I, N>),                            \
                       dim3((unsigned)(NUM_XCD * plan->nb)), dim3(SPMV_BLOCK), 0, s, m, plan->info, \
                       plan->rowptr_all, plan->colind_all, (const T *)plan->val_all, x,         \
                       plan->slice_w, ypart, plan->nb, plan->start_rows, plan->carry_row,       \
                       (T *)plan->carry_val)
#define F(I) do { if (nt) G(I, true); else G(I, false); } while (0)
    if (plan->ipt == 4) F(4);
    else F(8);
#undef F
#undef G
    if (int st = check_launch("csr_spmv_sliced_kernel")) return st;
    hipLaunchKernelGGL((spmv_carry_fixup_kernel<T>),
                       dim3((unsigned)((NUM_XCD * plan->nb + 255) / 256)), dim3(256), 0, s, plan->nb,
                       (int64_t)NUM_XCD, plan->carry_row, (const T *)plan->carry_val, ypart, m, T(1));
    if (int st = check_launch("spmv_carry_fixup_kernel")) return st;
    hipLaunchKernelGGL((slice_reduce_kernel<T>), dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, m,
                       (const T *)ypart, y, alpha, beta, (int)(beta == T(0)));
    return check_launch("slice_reduce_kernel");
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

template <typename T>
static int plan_execute_values(jlust_spmv_plan_t plan, int want_type, const T *val, T alpha, const T *x,
                               T beta, T *y, jlust_stream_t stream)
{
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_execute_values: null plan");
    if (plan->value_type != want_type)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE,
                    "spmv_plan_execute_values: plan was created for %s values",
                    plan->value_type == 0 ? "Float64" : "Float32");
    if (bad_ptr(val, plan->nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_execute_values: null values");
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    if (dev != plan->device)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "spmv_plan_execute_values: plan belongs to device %d, current device is %d",
                    plan->device, dev);
    if (int st = plan_refresh(plan, val, (hipStream_t)stream)) return st;
    return plan_execute<T>(plan, want_type, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_csr_spmv_plan_execute_values_f64(jlust_spmv_plan_t plan, const double *val,
                                                          double alpha, const double *x, double beta,
                                                          double *y, jlust_stream_t stream)
{
    return plan_execute_values<double>(plan, 0, val, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_csr_spmv_plan_execute_values_f32(jlust_spmv_plan_t plan, const float *val,
                                                          float alpha, const float *x, float beta,
                                                          float *y, jlust_stream_t stream)
{
    return plan_execute_values<float>(plan, 1, val, alpha, x, beta, y, stream);
}

// A plan execution recorded once as a HIP graph and replayed: the capture
// runs on a private stream in thread-local mode (other threads' work is not
// affected), and the executable graph is launched on the caller's stream.
struct jlust_spmv_graph {
    hipGraphExec_t exec;
    int device;
};

template <typename T>
static int plan_capture(jlust_spmv_plan_t plan, int want_type, T alpha, const T *x, T beta, T *y,
                        jlust_spmv_graph_t *out)
{
    clear_error();
    if (!out) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_capture: null output");
    *out = nullptr;
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_capture: null plan");
    if (plan->m == 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_capture: a plan with no rows launches nothing");
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    if (dev != plan->device)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "spmv_plan_capture: plan belongs to device %d, current device is %d", plan->device, dev);
    hipStream_t cs = nullptr;
    JLUST_HIP_TRY(hipStreamCreateWithFlags(&cs, hipStreamNonBlocking));
    hipError_t e = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
        (void)hipStreamDestroy(cs);
        return hip_fail(e, "hipStreamBeginCapture");
    }
    const int st = plan_execute<T>(plan, want_type, alpha, x, beta, y, cs);
    hipGraph_t g = nullptr;
    e = hipStreamEndCapture(cs, &g);
    (void)hipStreamDestroy(cs);
    if (st != JLUST_STATUS_SUCCESS || e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return st != JLUST_STATUS_SUCCESS ? st : hip_fail(e, "hipStreamEndCapture");
    }
    hipGraphExec_t ex = nullptr;
    e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    auto *h = new (std::nothrow) jlust_spmv_graph{ex, dev};
    if (!h) {
        (void)hipGraphExecDestroy(ex);
        return fail(JLUST_STATUS_OUT_OF_MEMORY, "spmv_plan_capture: host allocation failed");
    }
    *out = h;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_csr_spmv_plan_capture_f64(jlust_spmv_plan_t plan, double alpha, const double *x,
                                                   double beta, double *y, jlust_spmv_graph_t *graph_out)
{
    return plan_capture<double>(plan, 0, alpha, x, beta, y, graph_out);
}

extern "C" int jlust_hip_csr_spmv_plan_capture_f32(jlust_spmv_plan_t plan, float alpha, const float *x,
                                                   float beta, float *y, jlust_spmv_graph_t *graph_out)
{
    return plan_capture<float>(plan, 1, alpha, x, beta, y, graph_out);
}

extern "C" int jlust_hip_spmv_graph_launch(jlust_spmv_graph_t graph, jlust_stream_t stream)
{
    clear_error();
    if (!graph) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_graph_launch: null graph");
    hipStream_t s = (hipStream_t)stream;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    JLUST_HIP_TRY(hipStreamIsCapturing(s, &cap));
    if (cap != hipStreamCaptureStatusNone)
        return fail(JLUST_STATUS_STREAM_CAPTURING,
                    "spmv_graph_launch: the stream is being captured; execute the plan so that the "
                    "capture records its kernels");
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    if (dev != graph->device)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "spmv_graph_launch: graph belongs to device %d, current device is %d", graph->device, dev);
    JLUST_HIP_TRY(hipGraphLaunch(graph->exec, s));
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_spmv_graph_destroy(jlust_spmv_graph_t graph)
{
    clear_error();
    if (!graph) return JLUST_STATUS_SUCCESS;
    // Launches already queued finish first: the device is drained before the
    // executable graph goes away.
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != graph->device) e = hipSetDevice(graph->device);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    const hipError_t d = hipGraphExecDestroy(graph->exec);
    if (cur != graph->device) (void)hipSetDevice(cur);
    delete graph;
    if (e != hipSuccess) return hip_fail(e, "spmv_graph_destroy: hipDeviceSynchronize");
    if (d != hipSuccess) return hip_fail(d, "hipGraphExecDestroy");
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_csr_spmv_plan_info(jlust_spmv_plan_t plan, int32_t *kernel, int32_t *lanes_per_row,
                                            int64_t *device_bytes)
{
    clear_error();
    if (!plan || !kernel) return fail(JLUST_STATUS_INVALID_ARGUMENT, "spmv_plan_info: null argument");
    *kernel = plan->binned ? JLUST_SPMV_BINNED
              : plan->sliced ? JLUST_SPMV_SLICED
              : plan->vec_lpr > 0 ? JLUST_SPMV_VECTOR : JLUST_SPMV_MERGE;
    if (lanes_per_row) *lanes_per_row = plan->vec_lpr;
    if (device_bytes) *device_bytes = plan->bytes;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_csr_spmv_plan_destroy(jlust_spmv_plan_t plan)
{
    clear_error();
    if (!plan) return JLUST_STATUS_SUCCESS;
    hipError_t e = plan->mem ? hipFree(plan->mem) : hipSuccess;
    hipError_t e2 = plan->coo_mem ? hipFree(plan->coo_mem) : hipSuccess;
    binned_destroy(plan->binned);
    if (e == hipSuccess) e = e2;
    delete plan;
    if (e != hipSuccess) return hip_fail(e, "hipFree(plan)");
    return JLUST_STATUS_SUCCESS;
}

namespace jlust {
int preload_spmv()
{
    JLUST_PRELOAD_KERNEL(spmv_carry_fixup_kernel<double>);
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
