// convert.hip -- bit-exact sparse format conversions on the GPU.
//
// Restates JLUST's convert_format (src/convert.jl:302-388) for the hot-path
// formats CSR, CSC, COO, DCSR and BSR (src/named_formats.jl:24-27,106-128):
//   1. every stored entry is visited in storage order (TensorDecomposer,
//      convert.jl:5-122) and explicit zeros are dropped (convert.jl:316);
//   2. entries are keyed by their coordinates in the target's level order
//      (dim2lvl) and sorted stably unless the target is the identity
//      ordering and the source is ordered identity (convert.jl:331-349);
//   3. the target's buffers are composed (TensorComposer, convert.jl:124-299):
//      on a unique level, adjacent entries with equal coordinates form one
//      segment and only the first value of a segment is kept; Dense levels
//      of a block are zero-filled;
//   4. the result keeps the source's index origin (convert.jl:363-377).
// Pipeline on the device: per-entry coordinates (segment ids by scatter +
// max-scan), zero-drop compaction, stable LSD radix sort (rocPRIM) of packed
// level keys with source positions as values, adjacent-key dedup, then the
// target's pos/crd/val from the sorted keys.  Integer work only; values are
// moved as bits.
//
// Also: sparse_to_dense (ext/KernelAbstractionsExt/ops/conversion.jl:47-65)
// and the index shift of materialize's origin change (CUDAExt.jl:199-220).
#include <cstring>

#include <hip/hip_runtime.h>
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include "common.hpp"

namespace jlust {
namespace {

constexpr int CV_BLOCK = 256;

unsigned cv_grid(int64_t n) { return (unsigned)((n + CV_BLOCK - 1) / CV_BLOCK); }

int bits_for(int64_t n)             // bits to hold values in [0, n)
{
    int b = 0;
    while (b < 63 && ((int64_t)1 << b) < n) ++b;
    return b;
}

// Level layout of a target format: the key of an entry is
//   major << (minor_bits + inner_bits) | minor << inner_bits | inner,
// with (major, minor) = (row, col) for CSR/COO/DCSR, (col, row) for CSC and
// (block row, block col) for BSR, whose `inner` is the position inside the
// block in storage order (row-major: ii*b2 + jj, column-major: jj*b1 + ii).
struct KeyLayout {
    int fmt = 0;
    int b1 = 1, b2 = 1, row_major = 1;
    int minor_bits = 0, inner_bits = 0, total_bits = 0;
    int64_t major_dim = 0, minor_dim = 0;
};

__device__ __forceinline__ uint64_t make_key(const KeyLayout &L, int64_t row, int64_t col)
{
    uint64_t major, minor, inner = 0;
    if (L.fmt == JLUST_FORMAT_CSC) {
        major = (uint64_t)col;
        minor = (uint64_t)row;
    } else if (L.fmt == JLUST_FORMAT_BSR) {
        major = (uint64_t)(row / L.b1);
        minor = (uint64_t)(col / L.b2);
        const int64_t ii = row % L.b1, jj = col % L.b2;
        inner = (uint64_t)(L.row_major ? ii * L.b2 + jj : jj * L.b1 + ii);
    } else {
        major = (uint64_t)row;
        minor = (uint64_t)col;
    }
    return (major << (L.minor_bits + L.inner_bits)) | (minor << L.inner_bits) | inner;
}

__device__ __forceinline__ int64_t key_major(const KeyLayout &L, uint64_t k)
{
    return (int64_t)(k >> (L.minor_bits + L.inner_bits));
}
__device__ __forceinline__ int64_t key_minor(const KeyLayout &L, uint64_t k)
{
    return (int64_t)((k >> L.inner_bits) & ((1ull << L.minor_bits) - 1));
}
__device__ __forceinline__ int64_t key_inner(const KeyLayout &L, uint64_t k)
{
    return (int64_t)(k & ((1ull << L.inner_bits) - 1));
}
// Key without the inner part: identifies a BSR block.
__device__ __forceinline__ uint64_t key_block(const KeyLayout &L, uint64_t k)
{
    return k >> L.inner_bits;
}

// ------------------------------------------------------------- kernels

// mark[ptr[s] - origin] = s for every nonempty segment s < nseg (positions
// below len); with mark zero-initialised, an inclusive max-scan then gives the
// segment of every position.
__global__ void seg_mark_kernel(const int32_t *__restrict__ ptr, int64_t nseg, int32_t origin,
                                int64_t len, int32_t *__restrict__ mark)
{
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const int64_t a = (int64_t)ptr[s] - origin, b = (int64_t)ptr[s + 1] - origin;
    if (b > a && a >= 0 && a < len) mark[a] = (int32_t)s;
}

// Per stored value p: its (row, col), a keep flag (value != 0) and its key;
// *dropped (if given) counts the values not kept, one atomic per wave that
// drops any.
template <typename T>
__global__ void decompose_kernel(jlust_sparse src, const int32_t *__restrict__ seg, KeyLayout L,
                                 uint64_t *__restrict__ keys, int32_t *__restrict__ keep,
                                 int32_t *__restrict__ bad, int32_t *__restrict__ dropped)
{
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= src.nnz) return;
    const int32_t o = src.origin;
    int64_t row = 0, col = 0;
    switch (src.format) {
    case JLUST_FORMAT_CSR: row = seg[p]; col = (int64_t)src.crd2[p] - o; break;
    case JLUST_FORMAT_CSC: col = seg[p]; row = (int64_t)src.crd2[p] - o; break;
    case JLUST_FORMAT_COO: row = (int64_t)src.crd1[p] - o; col = (int64_t)src.crd2[p] - o; break;
    case JLUST_FORMAT_DCSR: row = (int64_t)src.crd1[seg[p]] - o; col = (int64_t)src.crd2[p] - o; break;
    default: {                                   // BSR: seg holds the block row of each block
        const int64_t bs = (int64_t)src.b1 * src.b2;
        const int64_t q = p / bs, e = p % bs;
        const int64_t ii = src.row_major_blocks ? e / src.b2 : e % src.b1;
        const int64_t jj = src.row_major_blocks ? e % src.b2 : e / src.b1;
        row = (int64_t)seg[q] * src.b1 + ii;
        col = ((int64_t)src.crd2[q] - o) * src.b2 + jj;
    }
    }
    const bool inb = row >= 0 && row < src.m && col >= 0 && col < src.n;
    if (!inb) bad[0] = 1;
    const T v = static_cast<const T *>(src.val)[p];
    const bool kp = inb && v != T(0);           // -0.0 == 0 is dropped, NaN kept
    keep[p] = kp ? 1 : 0;
    keys[p] = inb ? make_key(L, row, col) : 0;
    if (dropped) {
        const uint64_t d = __ballot(!kp);
        if (d && __lane_id() == (int)__builtin_ctzll(__ballot(1))) atomicAdd(dropped, (int32_t)__popcll(d));
    }
}

__global__ void iota_kernel(int64_t n, int32_t *__restrict__ p)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = (int32_t)i;
}

// out[idx[i]] = in[i] for flagged i, idx = exclusive scan of the flags.
__global__ void compact_kernel(int64_t n, const int32_t *__restrict__ flag,
                               const int32_t *__restrict__ idx, const uint64_t *__restrict__ kin,
                               const int32_t *__restrict__ pin, uint64_t *__restrict__ kout,
                               int32_t *__restrict__ pout)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n || !flag[i]) return;
    kout[idx[i]] = kin[i];
    pout[idx[i]] = pin ? pin[i] : (int32_t)i;
}

// head[i] = 1 where key (or, with block_only, its block) differs from i-1;
// *repeats (if given) counts the others, one atomic per wave that has any.
__global__ void head_kernel(int64_t n, const uint64_t *__restrict__ k, KeyLayout L, int block_only,
                            int32_t *__restrict__ head, int32_t *__restrict__ repeats)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    bool h = i == 0;
    if (!h) h = block_only ? key_block(L, k[i]) != key_block(L, k[i - 1]) : k[i] != k[i - 1];
    head[i] = h ? 1 : 0;
    if (repeats) {
        const uint64_t r = __ballot(!h);
        if (r && __lane_id() == (int)__builtin_ctzll(__ballot(1))) atomicAdd(repeats, (int32_t)__popcll(r));
    }
}

// Sets bad[0] when the major coordinate decreases (an unsorted "ordered" source).
__global__ void major_order_kernel(int64_t n, const uint64_t *__restrict__ k, KeyLayout L,
                                   int32_t *__restrict__ bad)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0 || i >= n) return;
    if (key_major(L, k[i]) < key_major(L, k[i - 1])) bad[0] = 1;
}

// ptr[r] = origin + first i with major(key[i]) >= r, for r in [0, nmajor].
// `major` (if given) holds per-item majors instead of keys.
__global__ void lower_bound_ptr_kernel(int64_t n, const uint64_t *__restrict__ k,
                                       const int32_t *__restrict__ major, KeyLayout L,
                                       int64_t nmajor, int32_t origin, int32_t *__restrict__ ptr)
{
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r > nmajor) return;
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        const int64_t mj = major ? (int64_t)major[mid] : key_major(L, k[mid]);
        if (mj < r) lo = mid + 1;
        else hi = mid;
    }
    ptr[r] = (int32_t)(lo + origin);
}

// Entry arrays of CSR/CSC/COO/DCSR targets (pos null: entry i is stored value i).
template <typename T>
__global__ void fill_entries_kernel(int64_t n, const uint64_t *__restrict__ k,
                                    const int32_t *__restrict__ pos, KeyLayout L, int32_t origin,
                                    const T *__restrict__ sval, int32_t *__restrict__ major_out,
                                    int32_t *__restrict__ minor_out, T *__restrict__ val_out)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (major_out) major_out[i] = (int32_t)(key_major(L, k[i]) + origin);
    minor_out[i] = (int32_t)(key_minor(L, k[i]) + origin);
    val_out[i] = sval[pos ? pos[i] : i];
}

// DCSR: at run heads of the row, crd1[run] = row + origin and pos2[run] = i + origin.
__global__ void fill_runs_kernel(int64_t n, const uint64_t *__restrict__ k,
                                 const int32_t *__restrict__ head, const int32_t *__restrict__ run,
                                 KeyLayout L, int32_t origin, int64_t nruns,
                                 int32_t *__restrict__ crd1, int32_t *__restrict__ pos2,
                                 int32_t *__restrict__ pos1)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i == 0) {
        pos2[nruns] = (int32_t)(n + origin);
        if (pos1) {
            pos1[0] = origin;
            pos1[1] = (int32_t)(nruns + origin);
        }
    }
    if (i >= n || !head[i]) return;
    crd1[run[i]] = (int32_t)(key_major(L, k[i]) + origin);
    pos2[run[i]] = (int32_t)(i + origin);
}

// BSR target: block b = run[i] of entry i; at block heads the block column
// and block row; every entry's value into its block slot (pos as above).
template <typename T>
__global__ void fill_bsr_kernel(int64_t n, const uint64_t *__restrict__ k,
                                const int32_t *__restrict__ pos, const int32_t *__restrict__ head,
                                const int32_t *__restrict__ run, KeyLayout L, int32_t origin,
                                const T *__restrict__ sval, int32_t *__restrict__ bcol,
                                int32_t *__restrict__ brow, T *__restrict__ val_out)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t b = run[i];
    if (head[i]) {
        bcol[b] = (int32_t)(key_minor(L, k[i]) + origin);
        brow[b] = (int32_t)key_major(L, k[i]);
    }
    val_out[b * L.b1 * L.b2 + key_inner(L, k[i])] = sval[pos ? pos[i] : i];
}

template <typename T>
__global__ void zero_kernel(int64_t n, T *__restrict__ p)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = T(0);
}

__global__ void pair_kernel(int32_t *__restrict__ p, int32_t a, int32_t b)
{
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        p[0] = a;
        p[1] = b;
    }
}

// dense[row + col*ld] = value of stored entry i (keys in CSR layout).
template <typename T>
__global__ void to_dense_kernel(int64_t n, const uint64_t *__restrict__ k, KeyLayout L,
                                const T *__restrict__ sval, T *__restrict__ dense, int64_t ld)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t row = key_major(L, k[i]), col = key_minor(L, k[i]);
    dense[row + col * ld] = sval[i];
}

__global__ void shift_kernel(int64_t n, int32_t *__restrict__ dst, const int32_t *__restrict__ src,
                             int32_t delta)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i] + delta;
}

// ----------------------------------------------------------------- host

int check_format(int fmt) { return fmt >= JLUST_FORMAT_CSR && fmt <= JLUST_FORMAT_BSR; }

bool src_ordered_identity(int fmt)
{
    return fmt == JLUST_FORMAT_CSR || fmt == JLUST_FORMAT_COO || fmt == JLUST_FORMAT_DCSR;
}
bool dst_identity(int fmt)
{
    return fmt == JLUST_FORMAT_CSR || fmt == JLUST_FORMAT_COO || fmt == JLUST_FORMAT_DCSR;
}

int check_sparse(const jlust_sparse *a, const char *what)
{
    if (!a) return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: null descriptor", what);
    if (!check_format(a->format))
        return fail(JLUST_STATUS_UNSUPPORTED_FORMAT, "%s: unknown format %d", what, a->format);
    if (int st = check_origin(a->origin)) return st;
    if (a->m < 0 || a->n < 0 || a->nnz < 0 || a->nouter < 0 || a->m > INT32_MAX ||
        a->n > INT32_MAX || a->nnz > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: extents outside the Int32 range", what);
    if (a->format == JLUST_FORMAT_BSR) {
        if (a->b1 <= 0 || a->b2 <= 0 || (int64_t)a->b1 * a->b2 > 65536 || a->m % a->b1 ||
            a->n % a->b2)
            return fail(JLUST_STATUS_INVALID_ARGUMENT, "%s: BSR block size %d x %d does not tile %lld x %lld",
                        what, a->b1, a->b2, (long long)a->m, (long long)a->n);
    }
    return JLUST_STATUS_SUCCESS;
}

KeyLayout layout_for(int fmt, int64_t m, int64_t n, int b1, int b2, int row_major)
{
    KeyLayout L;
    L.fmt = fmt;
    if (fmt == JLUST_FORMAT_CSC) {
        L.major_dim = n;
        L.minor_dim = m;
    } else if (fmt == JLUST_FORMAT_BSR) {
        L.b1 = b1;
        L.b2 = b2;
        L.row_major = row_major;
        L.major_dim = m / b1;
        L.minor_dim = n / b2;
        L.inner_bits = bits_for((int64_t)b1 * b2);
    } else {
        L.major_dim = m;
        L.minor_dim = n;
    }
    L.minor_bits = bits_for(L.minor_dim);
    L.total_bits = bits_for(L.major_dim) + L.minor_bits + L.inner_bits;
    return L;
}

// Segment id per position for CSR/CSC/DCSR (per value) and BSR (per block).
int segments(const jlust_sparse *s, int32_t *seg, int64_t &len, void *&tmp, size_t &tmp_bytes,
             hipStream_t st)
{
    int64_t nseg = 0;
    len = s->nnz;
    switch (s->format) {
    case JLUST_FORMAT_CSR: nseg = s->m; break;
    case JLUST_FORMAT_CSC: nseg = s->n; break;
    case JLUST_FORMAT_DCSR: nseg = s->nouter; break;
    case JLUST_FORMAT_BSR:
        nseg = s->m / s->b1;
        len = s->nouter;
        break;
    default: return JLUST_STATUS_SUCCESS;
    }
    if (len == 0) return JLUST_STATUS_SUCCESS;
    JLUST_HIP_TRY(hipMemsetAsync(seg, 0, sizeof(int32_t) * (size_t)len, st));
    if (nseg > 0) {
        hipLaunchKernelGGL(seg_mark_kernel, dim3(cv_grid(nseg)), dim3(CV_BLOCK), 0, st, s->pos2, nseg,
                           s->origin, len, seg);
        if (int e = check_launch("seg_mark_kernel")) return e;
    }
    size_t need = 0;
    JLUST_HIP_TRY(rocprim::inclusive_scan(nullptr, need, seg, seg, (size_t)len,
                                          rocprim::maximum<int32_t>(), st));
    if (need > tmp_bytes) {
        if (tmp) JLUST_HIP_TRY(hipFree(tmp));
        tmp = nullptr;
        JLUST_HIP_TRY(hipMalloc(&tmp, need));
        tmp_bytes = need;
    }
    JLUST_HIP_TRY(rocprim::inclusive_scan(tmp, need, seg, seg, (size_t)len,
                                          rocprim::maximum<int32_t>(), st));
    return JLUST_STATUS_SUCCESS;
}

}  // namespace
}  // namespace jlust

using namespace jlust;

struct jlust_convert {
    KeyLayout L;
    int32_t dst_format = 0, origin = 0, value_type = 0;
    int64_t m = 0, n = 0;
    int64_t count = 0;          // entries after drop + dedup
    int64_t nruns = 0;          // DCSR rows / BSR blocks
    const void *src_val = nullptr;
    void *mem = nullptr;        // the analysis workspace: keys, pos, head and run point into it
    uint64_t *keys = nullptr;
    int32_t *pos = nullptr, *head = nullptr, *run = nullptr;   // pos null: the identity
};

namespace {

struct Workspace {
    void *p = nullptr;
    ~Workspace() { if (p) (void)hipFree(p); }
};

template <typename T>
int analyze(const jlust_sparse *src, jlust_convert *h, hipStream_t st)
{
    const int64_t N = src->nnz;
    KeyLayout &L = h->L;
    if (N == 0) return JLUST_STATUS_SUCCESS;
    // Workspace: seg (per value or block), keys x2, pos x2, flags, scan.
    Workspace ws, tmpw;
    size_t tmp_bytes = 0;
    const size_t n = (size_t)N;
    const size_t nseg_len = (size_t)(src->format == JLUST_FORMAT_BSR ? src->nouter : N) + 1;
    const size_t bytes = 8 * n * 2 + 4 * n * 4 + 4 * nseg_len + 64;
    JLUST_HIP_TRY(hipMalloc(&ws.p, bytes));
    char *b = (char *)ws.p;
    uint64_t *k0 = (uint64_t *)b;     b += 8 * n;
    uint64_t *k1 = (uint64_t *)b;     b += 8 * n;
    int32_t *p0 = (int32_t *)b;       b += 4 * n;
    int32_t *p1 = (int32_t *)b;       b += 4 * n;
    int32_t *flag = (int32_t *)b;     b += 4 * n;
    int32_t *idx = (int32_t *)b;      b += 4 * n;
    int32_t *seg = (int32_t *)b;      b += 4 * nseg_len;
    int32_t *bad = (int32_t *)b;      // bad[0]: a coordinate out of range; bad[1]: values dropped
    JLUST_HIP_TRY(hipMemsetAsync(bad, 0, 2 * sizeof(int32_t), st));

    int64_t seglen = 0;
    if (int e = segments(src, seg, seglen, tmpw.p, tmp_bytes, st)) return e;
    hipLaunchKernelGGL((decompose_kernel<T>), dim3(cv_grid(N)), dim3(CV_BLOCK), 0, st, *src, seg, L, k0,
                       flag, bad, bad + 1);
    if (int e = check_launch("decompose_kernel")) return e;

    auto ensure = [&](size_t need) -> int {
        if (need > tmp_bytes) {
            if (tmpw.p) JLUST_HIP_TRY(hipFree(tmpw.p));
            tmpw.p = nullptr;
            JLUST_HIP_TRY(hipMalloc(&tmpw.p, need));
            tmp_bytes = need;
        }
        return JLUST_STATUS_SUCCESS;
    };
    // count of flagged items (exclusive scan + last flag), read back.
    auto count_flags = [&](int64_t len, int64_t *out) -> int {
        size_t need = 0;
        JLUST_HIP_TRY(rocprim::exclusive_scan(nullptr, need, flag, idx, 0, (size_t)len,
                                              rocprim::plus<int32_t>(), st));
        if (int e = ensure(need)) return e;
        JLUST_HIP_TRY(rocprim::exclusive_scan(tmpw.p, need, flag, idx, 0, (size_t)len,
                                              rocprim::plus<int32_t>(), st));
        int32_t last[2] = {0, 0};
        JLUST_HIP_TRY(hipMemcpyAsync(&last[0], idx + len - 1, 4, hipMemcpyDeviceToHost, st));
        JLUST_HIP_TRY(hipMemcpyAsync(&last[1], flag + len - 1, 4, hipMemcpyDeviceToHost, st));
        JLUST_HIP_TRY(hipStreamSynchronize(st));
        *out = (int64_t)last[0] + last[1];
        return JLUST_STATUS_SUCCESS;
    };

    // 1. drop explicit zeros (stable).  With none dropped the keys stay in
    // place and an entry's position is its index (pc null).
    int32_t flags_h[2] = {0, 0};
    JLUST_HIP_TRY(hipMemcpyAsync(flags_h, bad, sizeof(flags_h), hipMemcpyDeviceToHost, st));
    JLUST_HIP_TRY(hipStreamSynchronize(st));
    if (flags_h[0])
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "convert: a stored coordinate lies outside the %lld x %lld extents",
                    (long long)src->m, (long long)src->n);
    uint64_t *kc = k0;
    int32_t *pc = nullptr;
    int64_t K = N;
    if (flags_h[1] > 0) {
        if (int e = count_flags(N, &K)) return e;
        hipLaunchKernelGGL(compact_kernel, dim3(cv_grid(N)), dim3(CV_BLOCK), 0, st, N, flag, idx, k0,
                           (const int32_t *)nullptr, k1, p1);
        if (int e = check_launch("compact_kernel")) return e;
        kc = k1;
        pc = p1;
    }
    if (K == 0) return JLUST_STATUS_SUCCESS;

    // 2. sort by level coordinates unless target and source share the
    // identity ordering (convert.jl:331-349).
    const bool sort = !(dst_identity(h->dst_format) && src_ordered_identity(src->format));
    if (sort) {
        if (!pc) {                                  // the positions to carry: 0..K-1
            hipLaunchKernelGGL(iota_kernel, dim3(cv_grid(K)), dim3(CV_BLOCK), 0, st, K, p1);
            if (int e = check_launch("iota_kernel")) return e;
            pc = p1;
        }
        uint64_t *ko = kc == k0 ? k1 : k0;
        // A source whose segments run in the order of the target's minor
        // coordinate (CSR rows to a CSC target, CSC columns to a row-major
        // one) holds equal majors in ascending minor order already, so the
        // stable sort need only order the major bits.
        const bool major_only = (src->format == JLUST_FORMAT_CSR && h->dst_format == JLUST_FORMAT_CSC) ||
                                (src->format == JLUST_FORMAT_CSC && dst_identity(h->dst_format));
        const int end_bit = L.total_bits > 0 ? L.total_bits : 1;
        const int begin_bit = major_only && L.minor_bits + L.inner_bits < end_bit ? L.minor_bits + L.inner_bits : 0;
        size_t need = 0;
        JLUST_HIP_TRY(rocprim::radix_sort_pairs(nullptr, need, kc, ko, pc, p0, (size_t)K, begin_bit, end_bit, st));
        if (int e = ensure(need)) return e;
        JLUST_HIP_TRY(rocprim::radix_sort_pairs(tmpw.p, need, kc, ko, pc, p0, (size_t)K, begin_bit, end_bit, st));
        kc = ko;
        pc = p0;
    } else if (h->dst_format == JLUST_FORMAT_CSR) {
        // CSR's Dense row level needs non-decreasing rows; the reference
        // asserts it (convert.jl:254).  COO and DCSR targets keep any order.
        JLUST_HIP_TRY(hipMemsetAsync(bad, 0, sizeof(int32_t), st));
        hipLaunchKernelGGL(major_order_kernel, dim3(cv_grid(K)), dim3(CV_BLOCK), 0, st, K, kc, L, bad);
        if (int e = check_launch("major_order_kernel")) return e;
        int32_t badh = 0;
        JLUST_HIP_TRY(hipMemcpyAsync(&badh, bad, 4, hipMemcpyDeviceToHost, st));
        JLUST_HIP_TRY(hipStreamSynchronize(st));
        if (badh)
            return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                        "convert: the source's rows are not in non-decreasing order");
    }

    // 3. merge adjacent equal coordinates on unique levels (keep the first);
    // nothing to do when no key repeats.
    int64_t C = K;
    if (h->dst_format != JLUST_FORMAT_COO) {
        JLUST_HIP_TRY(hipMemsetAsync(bad + 1, 0, sizeof(int32_t), st));
        hipLaunchKernelGGL(head_kernel, dim3(cv_grid(K)), dim3(CV_BLOCK), 0, st, K, kc, L, 0, flag, bad + 1);
        if (int e = check_launch("head_kernel")) return e;
        int32_t repeats = 0;
        JLUST_HIP_TRY(hipMemcpyAsync(&repeats, bad + 1, sizeof(int32_t), hipMemcpyDeviceToHost, st));
        JLUST_HIP_TRY(hipStreamSynchronize(st));
        if (repeats > 0) {
            if (int e = count_flags(K, &C)) return e;
            uint64_t *ko = kc == k1 ? k0 : k1;
            int32_t *po = pc == p1 ? p0 : p1;       // pc null: positions are indices
            hipLaunchKernelGGL(compact_kernel, dim3(cv_grid(K)), dim3(CV_BLOCK), 0, st, K, flag, idx, kc, pc,
                               ko, po);
            if (int e = check_launch("compact_kernel")) return e;
            kc = ko;
            pc = po;
        }
    }

    // 4. the handle keeps the workspace: keys, positions, and (DCSR rows /
    // BSR blocks) run heads and ids in the flag and index arrays, free now.
    const size_t c = (size_t)C;
    h->mem = ws.p;
    ws.p = nullptr;
    h->keys = kc;
    h->pos = pc;
    h->head = flag;
    h->run = idx;
    h->count = C;
    if (h->dst_format == JLUST_FORMAT_DCSR || h->dst_format == JLUST_FORMAT_BSR) {
        KeyLayout Lr = L;
        if (h->dst_format == JLUST_FORMAT_DCSR) {   // runs of equal row: compare majors only
            Lr.inner_bits = L.minor_bits + L.inner_bits;
            Lr.minor_bits = 0;
        }
        hipLaunchKernelGGL(head_kernel, dim3(cv_grid(C)), dim3(CV_BLOCK), 0, st, C, h->keys, Lr, 1,
                           h->head, nullptr);
        if (int e = check_launch("head_kernel")) return e;
        size_t need = 0;
        JLUST_HIP_TRY(rocprim::inclusive_scan(nullptr, need, h->head, h->run, c, rocprim::plus<int32_t>(), st));
        if (int e = ensure(need)) return e;
        JLUST_HIP_TRY(rocprim::inclusive_scan(tmpw.p, need, h->head, h->run, c, rocprim::plus<int32_t>(), st));
        int32_t nr = 0;
        JLUST_HIP_TRY(hipMemcpyAsync(&nr, h->run + C - 1, 4, hipMemcpyDeviceToHost, st));
        JLUST_HIP_TRY(hipStreamSynchronize(st));
        h->nruns = nr;
        // run ids 0-based
        hipLaunchKernelGGL(shift_kernel, dim3(cv_grid(C)), dim3(CV_BLOCK), 0, st, C, h->run, h->run, -1);
        if (int e = check_launch("shift_kernel")) return e;
    }
    JLUST_HIP_TRY(hipStreamSynchronize(st));
    return JLUST_STATUS_SUCCESS;
}

template <typename T>
int fill(const jlust_convert *h, const jlust_sparse *d, hipStream_t st)
{
    const KeyLayout &L = h->L;
    const int64_t C = h->count;
    const int32_t o = h->origin;
    const T *sval = (const T *)h->src_val;
    switch (h->dst_format) {
    case JLUST_FORMAT_CSR:
    case JLUST_FORMAT_CSC:
        hipLaunchKernelGGL(lower_bound_ptr_kernel, dim3(cv_grid(L.major_dim + 1)), dim3(CV_BLOCK), 0, st, C,
                           h->keys, (const int32_t *)nullptr, L, L.major_dim, o, d->pos2);
        if (int e = check_launch("lower_bound_ptr_kernel")) return e;
        if (C > 0) {
            hipLaunchKernelGGL((fill_entries_kernel<T>), dim3(cv_grid(C)), dim3(CV_BLOCK), 0, st, C, h->keys,
                               h->pos, L, o, sval, (int32_t *)nullptr, d->crd2, (T *)d->val);
            if (int e = check_launch("fill_entries_kernel")) return e;
        }
        break;
    case JLUST_FORMAT_COO:
        if (d->pos1) {
            hipLaunchKernelGGL(pair_kernel, dim3(1), dim3(64), 0, st, d->pos1, o, (int32_t)(C + o));
            if (int e = check_launch("pair_kernel")) return e;
        }
        if (C > 0) {
            hipLaunchKernelGGL((fill_entries_kernel<T>), dim3(cv_grid(C)), dim3(CV_BLOCK), 0, st, C, h->keys,
                               h->pos, L, o, sval, d->crd1, d->crd2, (T *)d->val);
            if (int e = check_launch("fill_entries_kernel")) return e;
        }
        break;
    case JLUST_FORMAT_DCSR:
        hipLaunchKernelGGL(fill_runs_kernel, dim3(cv_grid(C > 0 ? C : 1)), dim3(CV_BLOCK), 0, st, C, h->keys,
                           h->head, h->run, L, o, h->nruns, d->crd1, d->pos2, d->pos1);
        if (int e = check_launch("fill_runs_kernel")) return e;
        if (C > 0) {
            hipLaunchKernelGGL((fill_entries_kernel<T>), dim3(cv_grid(C)), dim3(CV_BLOCK), 0, st, C, h->keys,
                               h->pos, L, o, sval, (int32_t *)nullptr, d->crd2, (T *)d->val);
            if (int e = check_launch("fill_entries_kernel")) return e;
        }
        break;
    default: {                                       // BSR
        const int64_t nb = h->nruns;
        const int64_t nv = nb * L.b1 * L.b2;
        int32_t *brow = nullptr;
        if (nb > 0) {
            JLUST_HIP_TRY(hipMallocAsync((void **)&brow, 4 * (size_t)nb, st));
            hipLaunchKernelGGL((zero_kernel<T>), dim3(cv_grid(nv)), dim3(CV_BLOCK), 0, st, nv, (T *)d->val);
            if (int e = check_launch("zero_kernel")) return e;
            hipLaunchKernelGGL((fill_bsr_kernel<T>), dim3(cv_grid(C)), dim3(CV_BLOCK), 0, st, C, h->keys, h->pos,
                               h->head, h->run, L, o, sval, d->crd2, brow, (T *)d->val);
            if (int e = check_launch("fill_bsr_kernel")) return e;
        }
        hipLaunchKernelGGL(lower_bound_ptr_kernel, dim3(cv_grid(L.major_dim + 1)), dim3(CV_BLOCK), 0, st, nb,
                           (const uint64_t *)nullptr, brow, L, L.major_dim, o, d->pos2);
        if (int e = check_launch("lower_bound_ptr_kernel")) return e;
        if (brow) JLUST_HIP_TRY(hipFreeAsync(brow, st));
    }
    }
    return JLUST_STATUS_SUCCESS;
}

int dst_check(const jlust_convert *h, const jlust_sparse *d)
{
    if (!d) return fail(JLUST_STATUS_INVALID_ARGUMENT, "convert_fill: null descriptor");
    const KeyLayout &L = h->L;
    if (d->format != h->dst_format || d->origin != h->origin || d->m != h->m || d->n != h->n)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "convert_fill: descriptor does not match the analysed conversion");
    if (h->dst_format == JLUST_FORMAT_BSR &&
        (d->b1 != L.b1 || d->b2 != L.b2 || (d->row_major_blocks != 0) != (L.row_major != 0)))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "convert_fill: BSR block layout differs from analyse");
    const int64_t want = h->dst_format == JLUST_FORMAT_BSR ? h->nruns * L.b1 * L.b2 : h->count;
    if (d->nnz != want)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "convert_fill: nnz %lld, analyse reported %lld",
                    (long long)d->nnz, (long long)want);
    bool bad = bad_ptr(d->val, want);
    switch (h->dst_format) {
    case JLUST_FORMAT_CSR:
    case JLUST_FORMAT_CSC: bad = bad || !d->pos2 || bad_ptr(d->crd2, want); break;
    case JLUST_FORMAT_COO: bad = bad || bad_ptr(d->crd1, want) || bad_ptr(d->crd2, want); break;
    case JLUST_FORMAT_DCSR: bad = bad || !d->pos2 || bad_ptr(d->crd1, h->nruns) || bad_ptr(d->crd2, want); break;
    default: bad = bad || !d->pos2 || bad_ptr(d->crd2, h->nruns);
    }
    if (bad) return fail(JLUST_STATUS_INVALID_ARGUMENT, "convert_fill: null device pointer");
    return JLUST_STATUS_SUCCESS;
}

bool src_ptrs_ok(const jlust_sparse *s)
{
    const int64_t nz = s->nnz;
    switch (s->format) {
    case JLUST_FORMAT_CSR: return (s->m == 0 || s->pos2) && !bad_ptr(s->crd2, nz) && !bad_ptr(s->val, nz);
    case JLUST_FORMAT_CSC: return (s->n == 0 || s->pos2) && !bad_ptr(s->crd2, nz) && !bad_ptr(s->val, nz);
    case JLUST_FORMAT_COO: return !bad_ptr(s->crd1, nz) && !bad_ptr(s->crd2, nz) && !bad_ptr(s->val, nz);
    case JLUST_FORMAT_DCSR:
        return (s->nouter == 0 || (s->pos2 && s->crd1)) && !bad_ptr(s->crd2, nz) && !bad_ptr(s->val, nz);
    default:
        return (s->m == 0 || s->pos2) && !bad_ptr(s->crd2, s->nouter) && !bad_ptr(s->val, nz) &&
               s->nnz == s->nouter * s->b1 * s->b2;
    }
}

}  // namespace

extern "C" int jlust_hip_convert_analyze(const jlust_sparse *src, int32_t dst_format, int32_t dst_b1,
                                         int32_t dst_b2, int32_t dst_row_major_blocks, int value_type,
                                         jlust_stream_t stream, jlust_convert_t *out, int64_t *dst_nnz,
                                         int64_t *dst_nouter)
{
    clear_error();
    if (!out || !dst_nnz || !dst_nouter)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "convert_analyze: null output pointer");
    *out = nullptr;
    if (int st = check_sparse(src, "convert_analyze")) return st;
    if (!check_format(dst_format))
        return fail(JLUST_STATUS_UNSUPPORTED_FORMAT, "convert_analyze: unknown target format %d", dst_format);
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "convert_analyze: value_type %d", value_type);
    if (!src_ptrs_ok(src)) return fail(JLUST_STATUS_INVALID_ARGUMENT, "convert_analyze: null or inconsistent source buffers");
    if (dst_format == JLUST_FORMAT_BSR &&
        (dst_b1 <= 0 || dst_b2 <= 0 || (int64_t)dst_b1 * dst_b2 > 65536 || src->m % dst_b1 || src->n % dst_b2))
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "convert_analyze: BSR block size %d x %d does not tile %lld x %lld", dst_b1, dst_b2,
                    (long long)src->m, (long long)src->n);
    if (int st = require_device(nullptr)) return st;
    auto *h = new jlust_convert();
    h->dst_format = dst_format;
    h->origin = src->origin;
    h->value_type = value_type;
    h->m = src->m;
    h->n = src->n;
    h->src_val = src->val;
    h->L = layout_for(dst_format, src->m, src->n, dst_b1, dst_b2, dst_row_major_blocks);
    if (h->L.total_bits > 64) {
        delete h;
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "convert_analyze: coordinates need more than 64 key bits");
    }
    const int st = value_type == 0 ? analyze<double>(src, h, (hipStream_t)stream)
                                   : analyze<float>(src, h, (hipStream_t)stream);
    if (st) {
        if (h->mem) (void)hipFree(h->mem);
        delete h;
        return st;
    }
    *dst_nnz = dst_format == JLUST_FORMAT_BSR ? h->nruns * dst_b1 * dst_b2 : h->count;
    *dst_nouter = (dst_format == JLUST_FORMAT_DCSR || dst_format == JLUST_FORMAT_BSR) ? h->nruns : 0;
    *out = h;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_convert_fill(jlust_convert_t h, const jlust_sparse *dst, jlust_stream_t stream)
{
    clear_error();
    if (!h) return fail(JLUST_STATUS_INVALID_ARGUMENT, "convert_fill: null handle");
    if (int st = dst_check(h, dst)) return st;
    if (int st = require_device(nullptr)) return st;
    return h->value_type == 0 ? fill<double>(h, dst, (hipStream_t)stream)
                              : fill<float>(h, dst, (hipStream_t)stream);
}

extern "C" int jlust_hip_convert_destroy(jlust_convert_t h)
{
    clear_error();
    if (!h) return JLUST_STATUS_SUCCESS;
    hipError_t e = h->mem ? hipFree(h->mem) : hipSuccess;
    delete h;
    if (e != hipSuccess) return hip_fail(e, "hipFree(convert)");
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_sparse_to_dense(const jlust_sparse *src, int value_type, void *dense, int64_t ld,
                                         jlust_stream_t stream)
{
    clear_error();
    if (int st = check_sparse(src, "sparse_to_dense")) return st;
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "sparse_to_dense: value_type %d", value_type);
    if (ld < (src->m > 0 ? src->m : 1))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "sparse_to_dense: ld %lld < m %lld", (long long)ld,
                    (long long)src->m);
    if (!src_ptrs_ok(src) || bad_ptr(dense, src->m * src->n))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "sparse_to_dense: null device pointer");
    if (int st = require_device(nullptr)) return st;
    hipStream_t s = (hipStream_t)stream;
    const size_t tsz = value_type == 0 ? 8 : 4;
    if (src->m > 0 && src->n > 0)
        JLUST_HIP_TRY(hipMemset2DAsync(dense, (size_t)ld * tsz, 0, (size_t)src->m * tsz, (size_t)src->n, s));
    // Every stored entry is scattered (explicit zeros write 0; duplicates of
    // one coordinate are not defined, as in the reference).
    const int64_t N = src->nnz;
    if (N == 0) return JLUST_STATUS_SUCCESS;
    const KeyLayout L = layout_for(JLUST_FORMAT_CSR, src->m, src->n, 1, 1, 1);
    Workspace ws, tmpw;
    size_t tmp_bytes = 0;
    const size_t nseg_len = (size_t)(src->format == JLUST_FORMAT_BSR ? src->nouter : N) + 1;
    JLUST_HIP_TRY(hipMalloc(&ws.p, 8 * (size_t)N + 4 * (size_t)N + 4 * nseg_len + 64));
    char *b = (char *)ws.p;
    uint64_t *k = (uint64_t *)b;        b += 8 * (size_t)N;
    int32_t *keep = (int32_t *)b;       b += 4 * (size_t)N;
    int32_t *seg = (int32_t *)b;        b += 4 * nseg_len;
    int32_t *bad = (int32_t *)b;
    JLUST_HIP_TRY(hipMemsetAsync(bad, 0, 4, s));
    int64_t seglen = 0;
    if (int st = segments(src, seg, seglen, tmpw.p, tmp_bytes, s)) return st;
    if (value_type == 0)
        hipLaunchKernelGGL((decompose_kernel<double>), dim3(cv_grid(N)), dim3(CV_BLOCK), 0, s, *src, seg, L, k,
                           keep, bad, nullptr);
    else
        hipLaunchKernelGGL((decompose_kernel<float>), dim3(cv_grid(N)), dim3(CV_BLOCK), 0, s, *src, seg, L, k,
                           keep, bad, nullptr);
    if (int st = check_launch("decompose_kernel")) return st;
    int32_t badh = 0;
    JLUST_HIP_TRY(hipMemcpyAsync(&badh, bad, 4, hipMemcpyDeviceToHost, s));
    JLUST_HIP_TRY(hipStreamSynchronize(s));
    if (badh)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "sparse_to_dense: a stored coordinate lies outside the %lld x %lld extents",
                    (long long)src->m, (long long)src->n);
    if (value_type == 0)
        hipLaunchKernelGGL((to_dense_kernel<double>), dim3(cv_grid(N)), dim3(CV_BLOCK), 0, s, N, k, L,
                           (const double *)src->val, (double *)dense, ld);
    else
        hipLaunchKernelGGL((to_dense_kernel<float>), dim3(cv_grid(N)), dim3(CV_BLOCK), 0, s, N, k, L,
                           (const float *)src->val, (float *)dense, ld);
    if (int st = check_launch("to_dense_kernel")) return st;
    JLUST_HIP_TRY(hipStreamSynchronize(s));
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_shift_index(int32_t *dst, const int32_t *src, int64_t len, int32_t delta,
                                     jlust_stream_t stream)
{
    clear_error();
    if (len < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "shift_index: negative length");
    if (bad_ptr(dst, len) || bad_ptr(src, len))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "shift_index: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (len == 0) return JLUST_STATUS_SUCCESS;
    hipLaunchKernelGGL(shift_kernel, dim3(cv_grid(len)), dim3(CV_BLOCK), 0, (hipStream_t)stream, len, dst,
                       src, delta);
    return check_launch("shift_kernel");
}

namespace jlust {
// The unit's device code plus the rocPRIM instantiations a conversion runs
// (64-bit key sort, int32 scans), each launched once on 64 elements.
int preload_convert(hipStream_t s)
{
    JLUST_PRELOAD_KERNEL(compact_kernel);
    constexpr size_t n = 64;
    size_t need_sort = 0, need_max = 0, need_ex = 0, need_in = 0;
    uint64_t *kn = nullptr;
    int32_t *vn = nullptr;
    JLUST_HIP_TRY(rocprim::radix_sort_pairs(nullptr, need_sort, kn, kn, vn, vn, n, 0, 64, s));
    JLUST_HIP_TRY(rocprim::inclusive_scan(nullptr, need_max, vn, vn, n, rocprim::maximum<int32_t>(), s));
    JLUST_HIP_TRY(rocprim::exclusive_scan(nullptr, need_ex, vn, vn, 0, n, rocprim::plus<int32_t>(), s));
    JLUST_HIP_TRY(rocprim::inclusive_scan(nullptr, need_in, vn, vn, n, rocprim::plus<int32_t>(), s));
    const size_t need = std::max(std::max(need_sort, need_max), std::max(need_ex, need_in));
    void *buf = nullptr;
    JLUST_HIP_TRY(hipMalloc(&buf, 2 * n * 8 + 2 * n * 4 + (need + 255) / 256 * 256));
    char *b = (char *)buf;
    uint64_t *k0 = (uint64_t *)b, *k1 = (uint64_t *)(b + n * 8);
    int32_t *v0 = (int32_t *)(b + 2 * n * 8), *v1 = (int32_t *)(b + 2 * n * 8 + n * 4);
    void *tmp = b + 2 * n * 8 + 2 * n * 4;
    hipError_t e = hipMemsetAsync(buf, 0, 2 * n * 8 + 2 * n * 4, s);
    size_t t = need;
    if (e == hipSuccess) e = rocprim::radix_sort_pairs(tmp, t, k0, k1, v0, v1, n, 0, 64, s);
    t = need;
    if (e == hipSuccess) e = rocprim::inclusive_scan(tmp, t, v0, v1, n, rocprim::maximum<int32_t>(), s);
    t = need;
    if (e == hipSuccess) e = rocprim::exclusive_scan(tmp, t, v0, v1, 0, n, rocprim::plus<int32_t>(), s);
    t = need;
    if (e == hipSuccess) e = rocprim::inclusive_scan(tmp, t, v0, v1, n, rocprim::plus<int32_t>(), s);
    const hipError_t e2 = hipStreamSynchronize(s);
    (void)hipFree(buf);
    if (e != hipSuccess) return hip_fail(e, "preload_convert");
    if (e2 != hipSuccess) return hip_fail(e2, "preload_convert");
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
