// gather_probe.hip -- measurement probes for bench.py (not part of the operator
// library; built into libjlust_probe.so).
//
// 1. Random 8-byte gather throughput: out[t] = sum_u src[base + idx[u*nthreads + t]]
// for u < 8, with idx uniform random below `range`.  With xcd_slice != 0,
// workgroup b gathers only from slice b % 8 of src (base = (b % 8) * range),
// the access pattern of the column-sliced SpMV plan, so each XCD's gathers
// stay inside its own L2.  The ceiling it measures bounds any kernel whose
// time is set by random gathers from an operand of that size.
//
// 2. Sustained fp32 matrix-core rate: every wave runs `iters` rounds of
// PROBE_CHAINS independent v_mfma_f32_16x16x4_f32 accumulation chains (2048
// flops each) on register operands, so the figure is the MFMA pipes' own rate
// at the clock the chip holds under that load.
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

constexpr int PROBE_CHAINS = 4;

typedef float probe_floatx4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void mfma_probe_kernel(float *__restrict__ out, int64_t iters, float seed)
{
    const int lane = threadIdx.x & 63;
    const float a = seed + 0.001f * lane, b = 1.0f - 0.0005f * lane;
    probe_floatx4 acc[PROBE_CHAINS];
#pragma unroll
    for (int c = 0; c < PROBE_CHAINS; ++c) acc[c] = probe_floatx4{0.f, 0.f, 0.f, 0.f};
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < PROBE_CHAINS; ++c)
            acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[c], 0, 0, 0);
    }
    probe_floatx4 s = acc[0];
#pragma unroll
    for (int c = 1; c < PROBE_CHAINS; ++c) s += acc[c];
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s[0] + s[1] + s[2] + s[3];
}

}  // namespace

// out holds blocks*256 floats.  Flops = blocks * 4 waves * iters *
// PROBE_CHAINS * 2048.  Returns 0, 1 on invalid arguments, 2 on a launch error.
extern "C" int jlust_probe_mfma_f32(float *out, int64_t blocks, int64_t iters, void *stream)
{
    if (!out || blocks <= 0 || blocks > (1 << 20) || iters <= 0) return 1;
    hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, out,
                       iters, 0.5f);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

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
