// spmv_binned.hpp -- the LDS-binned CSR SpMV layout of a prepared plan
// (spmv_binned.hip), used by spmv.hip's plans.
#pragma once

#include "common.hpp"

namespace jlust {

struct BinnedLayout {
    int64_t m = 0, n = 0, nnz = 0;
    int value_type = 0;      // 0 f64, 1 f32
    int32_t S = 0, B = 0;    // column slices, row bins
    int32_t W = 0, H = 0;    // columns per slice, rows per bin
    int32_t G = 1;           // workgroups per slice in the slice pass
    int32_t nch = 0;         // chunks per slice (G * waves per workgroup)
    int64_t P = 0;           // partial sums (one per (row, slice) pair with entries)
    int32_t maxrun = 0;      // longest run (partials of one slice in one bin)
    void *mem = nullptr;     // one allocation holds everything below
    void *sval = nullptr;    // values in slice-major (slice, bin, row, k) order
    uint16_t *scol = nullptr;  // slice-local column | (last entry of a partial) << 15
    uint16_t *loff = nullptr;  // sval[e] = val[bst[b] + k * chunk + loff[e]]: entry e of bin b sits
                               // at offset loff[e] of the bin's refresh chunk k
    int32_t *cst = nullptr;    // [S*nch + 1] entry start of each chunk
    int32_t *cpi = nullptr;    // [S*nch] index of the chunk's first partial
    int32_t *pr = nullptr;     // [S*B + 1] first partial of run (slice c, bin b) at c*B + b
    int32_t *est = nullptr;    // [S*B + 1] first entry of run (slice c, bin b) at c*B + b
    // Value refresh by chunks of a bin's CSR entries held in LDS (BN_LDS bytes):
    int32_t nrch = 0;          // chunks
    int32_t *rch = nullptr;    // [2*nrch] (bin, chunk index within the bin) of each chunk
    int32_t *bst = nullptr;    // [B + 1] first CSR entry of each bin
    int32_t *rtb = nullptr;    // [B + 1] first row of each bin in rtab
    int32_t *rtab = nullptr;   // [(nrch + B) * S]: row rtb[b] + k, column c = first entry of run
                               // (c, b) taken from CSR entries bst[b] + k * chunk or later
    uint16_t *prow = nullptr;  // [P + 1] bin-local row of each partial
    void *pval = nullptr;      // [P + 1] partial sums, rewritten by every execute
    int64_t bytes = 0;         // size of mem
};

// Whether a matrix of this shape fits the binned layout (slice count, bin
// count and positions within the layout's index widths).
bool binned_fits(int value_type, int64_t m, int64_t n, int64_t nnz);

// Builds the layout of an m x n CSR matrix with nnz >= 1 entries, on the
// stream, and waits for it.  val is read once; update refreshes it.
int binned_build(BinnedLayout **out, int value_type, int64_t m, int64_t n, int64_t nnz,
                 int32_t origin, const int32_t *rowptr, const int32_t *colind, const void *val,
                 int64_t max_bytes, hipStream_t s);

// Device bytes the layout holds (its one allocation).
int64_t binned_bytes(const BinnedLayout *L);

// sval = val[perm] for new values with the same pattern (stream-ordered).
int binned_update(BinnedLayout *L, const void *val, hipStream_t s);

// y = alpha * A x + beta * y (beta == 0: y is only written).
int binned_execute_f64(const BinnedLayout *L, double alpha, const double *x, double beta, double *y,
                       hipStream_t s);
int binned_execute_f32(const BinnedLayout *L, float alpha, const float *x, float beta, float *y,
                       hipStream_t s);

void binned_destroy(BinnedLayout *L);

}  // namespace jlust
