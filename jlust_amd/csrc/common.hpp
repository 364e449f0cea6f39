// common.hpp -- internals shared by the libjlust_hip.so translation units:
// status/error plumbing for the C ABI, argument checks, per-(device, stream)
// scratch buffers, device properties and wave64 helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <new>
#include <string>

#include "../../include/jlust_hip.h"

namespace jlust {

// ----------------------------------------------------------------- errors

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Maps a failed HIP call onto JLUST_STATUS_HIP_ERROR / OUT_OF_MEMORY.
int hip_fail(hipError_t e, const char *what);

// Runs f() and turns a host allocation failure (std::bad_alloc from the
// library's host-side tables) into JLUST_STATUS_OUT_OF_MEMORY, so that no C++
// exception crosses the C ABI.  The guarded code makes its host allocations
// before its device ones, so such a failure leaks no device memory.
template <typename F>
int host_guard(const char *what, F &&f)
{
    try {
        return f();
    } catch (const std::bad_alloc &) {
        return fail(JLUST_STATUS_OUT_OF_MEMORY, "%s: out of host memory", what);
    }
}

#define JLUST_HIP_TRY(expr)                                      \
    do {                                                         \
        hipError_t _e = (expr);                                  \
        if (_e != hipSuccess) return ::jlust::hip_fail(_e, #expr); \
    } while (0)

// Checks that a GPU is present and current; JLUST_STATUS_NO_DEVICE otherwise.
int require_device(int *device_out);

// Checks a kernel launch (hipGetLastError) and turns failures into a status.
int check_launch(const char *kernel);

// ------------------------------------------------------------- arguments

inline bool bad_ptr(const void *p, int64_t count) { return count > 0 && p == nullptr; }

int check_origin(int32_t origin);

// ---------------------------------------------------------------- devices

struct DeviceInfo {
    int cu_count = 0;          // compute units
    int wave_size = 64;
    size_t lds_per_block = 0;  // bytes
    char arch[64] = {0};
};
const DeviceInfo &device_info(int device);

// ---------------------------------------------------------------- scratch

// Returns a device buffer of at least `bytes` owned by the library and
// private to (current device, stream).  It grows on demand; an outgrown
// buffer is kept until process exit, since queued work or a captured graph
// may still read it.
int scratch(jlust_stream_t stream, size_t bytes, void **out);

// out[i] = sum(in[0..i)) over n int32 counts (in == out allowed); stream-ordered.
// Uses the stream's scratch buffer for chunk sums.
int exclusive_scan_i32(const int32_t *in, int32_t *out, int64_t n, jlust_stream_t stream);
// The first bytes of the stream's scratch buffer that exclusive_scan_i32 over
// n counts uses; a caller keeping data of its own in that buffer across the
// scan places it after them.
size_t exclusive_scan_scratch_bytes(int64_t n);

constexpr int NUM_XCD = 8;   // MI355X: workgroup b runs on XCD b % 8

// Hands a COO plan's owned buffers to a CSR SpMV plan (spmv.hip): mem is
// freed with the plan; perm/val_copy (or null) reorder new values on
// update_values.
int spmv_plan_adopt_coo(jlust_spmv_plan_t plan, void *mem, const int32_t *perm, void *val_copy, size_t bytes);

// Row order of m x n COO entries (coo_plan.hip): rowptr[m+1] (origin-based)
// of the entries in row order and, unless the rows were already
// non-decreasing (*sorted set, perm and cols_out untouched), perm[q] = the
// caller's position of row-ordered entry q (a stable sort) and cols_out[q] =
// its column.  Buffers are the caller's (perm and cols_out nnz entries); a
// row outside [origin, m + origin) is NONCANONICAL_STORAGE.  Synchronises s.
int coo_row_order(int64_t m, int64_t nnz, int32_t origin, const int32_t *rows, const int32_t *cols,
                  int32_t *rowptr, int32_t *perm, int32_t *cols_out, bool *sorted, hipStream_t s);

// Checks a position array (coo_csc.hip): pos[0] == origin, pos[nouter] ==
// nnz + origin, non-decreasing; NONCANONICAL_STORAGE otherwise.  Synchronises s.
int check_pos(const char *who, int64_t nouter, int64_t nnz, int32_t origin, const int32_t *pos, hipStream_t s);

// crd_out[p] = the outer coordinate of entry p (outer[s], or s + origin when
// outer is null) after check_pos of pos (coo_csc.hip).
int expand_pos(int64_t nouter, int64_t nnz, int32_t origin, const int32_t *pos, const int32_t *outer,
               int32_t *crd_out, hipStream_t s);

// Row order of COO (idx1 = rows, idx2 = cols) or CSC (idx1 = colptr, idx2 =
// rowind) entries (coo_csc.hip): rowptr[m+1]; perm/cols written and
// *reordered = 1 unless the source order already is the row order.
int row_order(int32_t format, int64_t m, int64_t n, int64_t nnz, int32_t origin, const int32_t *idx1,
              const int32_t *idx2, int32_t *rowptr, int32_t *perm, int32_t *cols, int32_t *reordered,
              hipStream_t s);

// dst[i] = src[perm[i]] for i < nnz (value_type 0 = f64, 1 = f32), on s.
int perm_gather(int value_type, int64_t nnz, const int32_t *perm, const void *src, void *dst, hipStream_t s);

// Hands a COO/CSC SpMM plan's owned row order to a CSR SpMM plan (spmm.hip):
// mem is freed with the plan; perm/val_copy (or null) reorder new values on
// update_values.
int spmm_plan_adopt_reorder(jlust_spmm_plan_t plan, void *mem, const int32_t *perm, void *val_copy);

// ---------------------------------------------------------------- preload

// The runtime loads a translation unit's device code on the first launch of
// one of its kernels (tens of milliseconds for the larger ones).  Each unit
// defines preload_<unit>(), which asks for the attributes of one of its
// kernels -- enough to make the runtime load that code object now -- and, in
// the units that sort with rocPRIM, runs one tiny sort on the stream, since
// rocPRIM's kernels are loaded at their first launch.  jlust_hip_preload()
// calls them all.
int preload_spmv();
int preload_binned(hipStream_t s);
int preload_coo_plan(hipStream_t s);
int preload_convert(hipStream_t s);
int preload_spmm();
int preload_sddmm();
int preload_bsr();
int preload_coo_spmv();
int preload_coo_csc();
int preload_assemble();
int preload_dcsr();
int preload_fn();
int preload_periodic();
int preload_scan();

#define JLUST_PRELOAD_KERNEL(KERNEL)                                                        \
    do {                                                                                    \
        hipFuncAttributes attr_;                                                            \
        const hipError_t e_ = hipFuncGetAttributes(&attr_, reinterpret_cast<const void *>(KERNEL)); \
        if (e_ != hipSuccess) return ::jlust::hip_fail(e_, "preload " #KERNEL);             \
    } while (0)

// ------------------------------------------------------------ device code

__device__ __forceinline__ int lane_id() { return __lane_id(); }

template <typename T>
__device__ __forceinline__ T ld_nt(const T *p) { return __builtin_nontemporal_load(p); }

}  // namespace jlust
