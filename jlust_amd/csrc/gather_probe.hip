// gather_probe.hip -- measurement probe for bench.py (not part of the operator
// library; built into libjlust_probe.so).
//
// Random 8-byte gather throughput: out[t] = sum_u src[base + idx[u*nthreads + t]]
// for u < 8, with idx uniform random below `range`.  With xcd_slice != 0,
// workgroup b gathers only from slice b % 8 of src (base = (b % 8) * range),
// the access pattern of the column-sliced SpMV plan, so each XCD's gathers
// stay inside its own L2.  The ceiling it measures bounds any kernel whose
// time is set by random gathers from an operand of that size.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int PROBE_U = 8;

__global__ __launch_bounds__(256) void gather_probe_kernel(const double *__restrict__ src,
                                                           const uint32_t *__restrict__ idx,
                                                           double *__restrict__ out,
                                                           int64_t nthreads, int xcd_slice,
                                                           uint32_t range)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nthreads) return;
    const uint64_t base = xcd_slice ? (uint64_t)(blockIdx.x % 8) * range : 0;
    uint32_t id[PROBE_U];
#pragma unroll
    for (int u = 0; u < PROBE_U; ++u) id[u] = __builtin_nontemporal_load(idx + t + u * nthreads);
    double s = 0;
#pragma unroll
    for (int u = 0; u < PROBE_U; ++u) s += src[base + id[u]];
    out[t] = s;
}

}  // namespace

// idx holds 8*nthreads values below `range`; src holds at least range
// (xcd_slice == 0) or 8*range (xcd_slice != 0) elements; out holds nthreads.
// Returns 0, or 1 on invalid arguments, 2 on a launch error.
extern "C" int jlust_probe_gather_f64(const double *src, int64_t src_len, const uint32_t *idx,
                                      double *out, int64_t nthreads, int xcd_slice,
                                      uint32_t range, void *stream)
{
    if (!src || !idx || !out || nthreads <= 0 || range == 0) return 1;
    if ((uint64_t)range * (xcd_slice ? 8u : 1u) > (uint64_t)src_len) return 1;
    const unsigned grid = (unsigned)((nthreads + 255) / 256);
    hipLaunchKernelGGL(gather_probe_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, idx,
                       out, nthreads, xcd_slice, range);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}
