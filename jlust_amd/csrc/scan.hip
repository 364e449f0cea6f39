// scan.hip -- device-wide exclusive prefix sum of int32 counts (in place
// allowed), used to turn per-row counts into row pointers.  Three passes:
// per-chunk sums, a single-block scan of the chunk sums, and a rescan of each
// chunk with its offset.
#include "common.hpp"

namespace jlust {
namespace {

constexpr int SCAN_BLOCK = 256;
constexpr int SCAN_IPT = 16;
constexpr int64_t SCAN_CHUNK = SCAN_BLOCK * SCAN_IPT;

// Exclusive scan of one value per thread over a block of SCAN_BLOCK threads.
__device__ int64_t block_exclusive_scan(int64_t v, int64_t *s_w, int64_t *total)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int64_t inc = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int64_t o = __shfl_up(inc, off, 64);
        if (lane >= off) inc += o;
    }
    if (lane == 63) s_w[wave] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t run = 0;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) {
            const int64_t t = s_w[w];
            s_w[w] = run;
            run += t;
        }
        s_w[blockDim.x >> 6] = run;
    }
    __syncthreads();
    const int64_t ex = inc - v + s_w[wave];
    *total = s_w[blockDim.x >> 6];
    __syncthreads();
    return ex;
}

__global__ __launch_bounds__(SCAN_BLOCK) void scan_chunk_sums(const int32_t *__restrict__ in,
                                                             int64_t n, int64_t *__restrict__ sums)
{
    __shared__ int64_t s_w[SCAN_BLOCK / 64 + 1];
    const int64_t base = (int64_t)blockIdx.x * SCAN_CHUNK;
    int64_t v = 0;
#pragma unroll
    for (int u = 0; u < SCAN_IPT; ++u) {
        const int64_t i = base + u * SCAN_BLOCK + threadIdx.x;
        if (i < n) v += in[i];
    }
    int64_t total;
    block_exclusive_scan(v, s_w, &total);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

// One block: exclusive scan of nsum chunk sums in place.
__global__ __launch_bounds__(1024) void scan_sums(int64_t *__restrict__ sums, int64_t nsum)
{
    __shared__ int64_t s_w[1024 / 64 + 1];
    const int64_t per = (nsum + 1023) / 1024;
    const int64_t lo = (int64_t)threadIdx.x * per;
    const int64_t hi = min(nsum, lo + per);
    int64_t v = 0;
    for (int64_t i = lo; i < hi; ++i) v += sums[i];
    int64_t total;
    int64_t run = block_exclusive_scan(v, s_w, &total);
    for (int64_t i = lo; i < hi; ++i) {
        const int64_t t = sums[i];
        sums[i] = run;
        run += t;
    }
}

__global__ __launch_bounds__(SCAN_BLOCK) void scan_apply(const int32_t *in, int32_t *out, int64_t n,
                                                         const int64_t *__restrict__ offs)
{
    __shared__ int64_t s_w[SCAN_BLOCK / 64 + 1];
    const int64_t base = (int64_t)blockIdx.x * SCAN_CHUNK + (int64_t)threadIdx.x * SCAN_IPT;
    int32_t v[SCAN_IPT];
    int64_t sum = 0;
#pragma unroll
    for (int u = 0; u < SCAN_IPT; ++u) {
        v[u] = base + u < n ? in[base + u] : 0;
        sum += v[u];
    }
    int64_t total;
    int64_t run = block_exclusive_scan(sum, s_w, &total) + offs[blockIdx.x];
#pragma unroll
    for (int u = 0; u < SCAN_IPT; ++u) {
        if (base + u < n) out[base + u] = (int32_t)run;
        run += v[u];
    }
}

}  // namespace

size_t exclusive_scan_scratch_bytes(int64_t n)
{
    return n <= 0 ? 0 : sizeof(int64_t) * (size_t)((n + SCAN_CHUNK - 1) / SCAN_CHUNK);
}

int exclusive_scan_i32(const int32_t *in, int32_t *out, int64_t n, jlust_stream_t stream)
{
    if (n <= 0) return JLUST_STATUS_SUCCESS;
    const int64_t nchunks = (n + SCAN_CHUNK - 1) / SCAN_CHUNK;
    void *ws = nullptr;
    if (int st = scratch(stream, sizeof(int64_t) * (size_t)nchunks, &ws)) return st;
    int64_t *sums = (int64_t *)ws;
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(scan_chunk_sums, dim3((unsigned)nchunks), dim3(SCAN_BLOCK), 0, s, in, n, sums);
    if (int st = check_launch("scan_chunk_sums")) return st;
    hipLaunchKernelGGL(scan_sums, dim3(1), dim3(1024), 0, s, sums, nchunks);
    if (int st = check_launch("scan_sums")) return st;
    hipLaunchKernelGGL(scan_apply, dim3((unsigned)nchunks), dim3(SCAN_BLOCK), 0, s, in, out, n, sums);
    return check_launch("scan_apply");
}

}  // namespace jlust

namespace jlust {
int preload_scan()
{
    JLUST_PRELOAD_KERNEL(scan_chunk_sums);
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
