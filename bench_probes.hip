// bench_probes.hip -- measurement probes for bench.py (not part of the operator
// library or the C ABI; bench.py builds them into bench_probes.so on demand).
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
//
// 3. Random whole-row gathers: each wave sums rows src[idx[p], 0:row] (row =
// 64 or 128 floats) for a run of indices, ROWS_U rows in flight per wave,
// the lanes covering the row with 4- or 8-byte vector loads -- the access
// pattern of the SpMM kernel's gathers from the row-major copy of B (256-byte
// rows) and of the SDDMM kernel's gathers of B's columns (512-byte rows),
// without their arithmetic or outputs.  Its time bounds any kernel that
// makes those gathers.  3b: the same with 16-byte lanes, several rows per
// wave instruction.
//
// 4. Streaming write and read of a buffer (16-byte lanes, grid-stride), for
// the question whether data written by one kernel is read back by the next
// from the MALL faster than from HBM.
//
// 5. The parts of a uniform-row CSR SpMV step (rows of exactly `ulen`
// entries, 4 lanes per row, 4 entries per lane at a time: the shape of the
// library's vector kernel at config 1): mode 0 multiplies by x[col], the
// random gathers; mode 1 by x[row], a coalesced read of the same bytes;
// mode 2 by the column index itself, no x; mode 3 writes y only.  The
// differences between the modes split the step into its gathers, its stream
// of A and its launch.
#include <hip/hip_runtime.h>

#include <cstdint>

typedef int probe_int32x4 __attribute__((ext_vector_type(4)));

__device__ double probe_buffer_load_f64(probe_int32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.f64");

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

// Buffer resource over p (wave-uniform): base in dwords 0-1, no stride,
// num_records 0xffffffff bytes, gfx9 data format in dword 3.
__device__ __forceinline__ probe_int32x4 probe_resource(const void *p)
{
    const uint64_t a = (uint64_t)p;
    probe_int32x4 r;
    r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffff));
    r.z = -1;
    r.w = 0x00020000;
    return r;
}

// 1b. The gathers of 1. (whole source) as buffer loads carrying cache-policy
// bits CPOL (bit 0 sc0, bit 1 nt, bit 4 sc1): which form moves an 8-byte
// gather from the L2 fastest.
template <int CPOL>
__global__ __launch_bounds__(256) void gather_cpol_kernel(const double *__restrict__ src,
                                                          const uint32_t *__restrict__ idx,
                                                          double *__restrict__ out, int64_t nthreads)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nthreads) return;
    const probe_int32x4 rsrc = probe_resource(src);
    uint32_t id[PROBE_U];
#pragma unroll
    for (int u = 0; u < PROBE_U; ++u) id[u] = __builtin_nontemporal_load(idx + t + u * nthreads);
    double s = 0;
#pragma unroll
    for (int u = 0; u < PROBE_U; ++u) s += probe_buffer_load_f64(rsrc, (int)(id[u] * 8u), 0, CPOL);
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

constexpr int ROWS_U = 8;

// Gathers `count` rows; wave w takes indices [w*per_wave, (w+1)*per_wave).
template <int VEC>
__global__ __launch_bounds__(256) void rows_probe_kernel(const float *__restrict__ src, int64_t row,
                                                         const uint32_t *__restrict__ idx, int64_t count,
                                                         int64_t per_wave, float *__restrict__ out)
{
    typedef float vec_t __attribute__((ext_vector_type(VEC)));
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t p0 = wave * per_wave;
    const int64_t p1 = p0 + per_wave < count ? p0 + per_wave : count;
    vec_t acc = {};
    for (int64_t p = p0; p < p1; p += ROWS_U) {
        vec_t v[ROWS_U];
#pragma unroll
        for (int u = 0; u < ROWS_U; ++u) {
            const int64_t q = p + u < p1 ? p + u : p1 - 1;
            const uint64_t r = idx[q];
            v[u] = *reinterpret_cast<const vec_t *>(src + r * row + lane * VEC);
        }
#pragma unroll
        for (int u = 0; u < ROWS_U; ++u) acc += v[u];
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) s += acc[e];
    if (p0 < count) out[wave * 64 + lane] = s;
}

// 3b. The same gathers with 16-byte lanes: LPR lanes cover a row (16 for
// 256-byte rows, 32 for 512-byte rows), so one wave instruction reads 64/LPR
// rows and ROWS_U instructions keep ROWS_U * 64/LPR rows in flight per wave.
template <int LPR>
__global__ __launch_bounds__(256) void rows_wide_probe_kernel(const float *__restrict__ src, int64_t row,
                                                              const uint32_t *__restrict__ idx, int64_t count,
                                                              int64_t per_wave, float *__restrict__ out)
{
    typedef float vec_t __attribute__((ext_vector_type(4)));
    constexpr int RPI = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane / LPR, l = lane % LPR;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t p0 = wave * per_wave;
    const int64_t p1 = p0 + per_wave < count ? p0 + per_wave : count;
    vec_t acc = {};
    for (int64_t p = p0; p < p1; p += ROWS_U * RPI) {
        vec_t v[ROWS_U];
#pragma unroll
        for (int u = 0; u < ROWS_U; ++u) {
            const int64_t q0 = p + u * RPI + sub;
            const int64_t q = q0 < p1 ? q0 : p1 - 1;
            const uint64_t r = idx[q];
            v[u] = *reinterpret_cast<const vec_t *>(src + r * row + l * 4);
        }
#pragma unroll
        for (int u = 0; u < ROWS_U; ++u) acc += v[u];
    }
    if (p0 < count) out[wave * 64 + lane] = acc[0] + acc[1] + acc[2] + acc[3];
}

typedef double probe_double2 __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(256) void write_probe_kernel(probe_double2 *__restrict__ dst, int64_t n, double v)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = probe_double2{v, v + 1.0};
}

__global__ __launch_bounds__(256) void read_probe_kernel(const probe_double2 *__restrict__ src, int64_t n,
                                                         double *__restrict__ out)
{
    double s = 0.0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const probe_double2 v = __builtin_nontemporal_load(src + i);
        s += v.x + v.y;
    }
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

template <int MODE>
__global__ __launch_bounds__(256) void spmv_parts_kernel(int64_t m, int32_t ulen, int32_t origin,
                                                         const int32_t *__restrict__ colind,
                                                         const double *__restrict__ val,
                                                         const double *__restrict__ x, double *__restrict__ y)
{
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = t >> 2;
    const int sub = (int)(t & 3);
    const int64_t r = row < m ? row : m - 1;
    const int64_t lo = r * ulen, hi = row < m ? lo + ulen : lo;
    double acc = 0.0;
    if (MODE != 3) {
        for (int64_t p0 = lo + sub; p0 < hi; p0 += 16) {
            int32_t c[4];
            double v[4], xv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t p = min(p0 + 4 * u, hi - 1);
                c[u] = colind[p];
                v[u] = val[p];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
                xv[u] = MODE == 0 ? x[c[u] - origin] : MODE == 1 ? x[r] : (double)c[u];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const double a = acc + v[u] * xv[u];
                acc = p0 + 4 * u < hi ? a : acc;
            }
        }
    }
    acc += __shfl_xor(acc, 1, 4);
    acc += __shfl_xor(acc, 2, 4);
    if (sub == 0 && row < m) y[row] = acc;
}

// src holds nrows x row floats (row-major, 16-byte aligned), idx holds count
// row indices below nrows, out holds 64 * waves floats with waves =
// ceil(count / per_wave); row is 64 (4-byte lanes) or 128 (8-byte lanes).
// Returns 0, 1 on invalid arguments, 2 on a launch error.
extern "C" int jlust_probe_rows_f32(const float *src, int64_t nrows, int64_t row, const uint32_t *idx,
                                    int64_t count, int64_t per_wave, float *out, void *stream)
{
    if (!src || !idx || !out || nrows <= 0 || count <= 0 || per_wave <= 0) return 1;
    if (row != 64 && row != 128) return 1;
    const int64_t waves = (count + per_wave - 1) / per_wave;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    if (row == 64)
        hipLaunchKernelGGL(rows_probe_kernel<1>, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, row, idx,
                           count, per_wave, out);
    else
        hipLaunchKernelGGL(rows_probe_kernel<2>, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, row, idx,
                           count, per_wave, out);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// As jlust_probe_rows_f32, with 16-byte lanes (rows_wide_probe_kernel).
extern "C" int jlust_probe_rows_wide_f32(const float *src, int64_t nrows, int64_t row, const uint32_t *idx,
                                         int64_t count, int64_t per_wave, float *out, void *stream)
{
    if (!src || !idx || !out || nrows <= 0 || count <= 0 || per_wave <= 0) return 1;
    if (row != 64 && row != 128) return 1;
    const int64_t waves = (count + per_wave - 1) / per_wave;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    if (row == 64)
        hipLaunchKernelGGL(rows_wide_probe_kernel<16>, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, row,
                           idx, count, per_wave, out);
    else
        hipLaunchKernelGGL(rows_wide_probe_kernel<32>, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, row,
                           idx, count, per_wave, out);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Streaming write (dst) or nontemporal read (src, partial sums into out:
// grid*256 doubles) of nbytes (a multiple of 16) with a grid of `grid`
// 256-thread workgroups.  Returns 0, 1 on invalid arguments, 2 on a launch error.
extern "C" int jlust_probe_stream(void *buf, int64_t nbytes, int write, int64_t grid, double *out, void *stream)
{
    if (!buf || nbytes <= 0 || nbytes % 16 || grid <= 0 || grid > (1 << 20) || (!write && !out)) return 1;
    if (write)
        hipLaunchKernelGGL(write_probe_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                           (probe_double2 *)buf, nbytes / 16, 1.0);
    else
        hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                           (const probe_double2 *)buf, nbytes / 16, out);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

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

// The gathers of jlust_probe_gather_f64 (whole source) as buffer loads with
// cache-policy bits cpol: 0, 1 (sc0), 2 (nt), 3 (sc0 nt), 16 (sc1) or 17
// (sc0 sc1).  idx holds 8*nthreads values below range <= src_len, and
// src_len * 8 < 2^31.  Returns 0, 1 on invalid arguments, 2 on a launch error.
extern "C" int jlust_probe_gather_cpol_f64(const double *src, int64_t src_len, const uint32_t *idx,
                                           double *out, int64_t nthreads, uint32_t range, int cpol,
                                           void *stream)
{
    if (!src || !idx || !out || nthreads <= 0 || range == 0 || range > (uint64_t)src_len) return 1;
    if (src_len * 8 >= ((int64_t)1 << 31)) return 1;
    const unsigned grid = (unsigned)((nthreads + 255) / 256);
    const hipStream_t st = (hipStream_t)stream;
#define PROBE_CPOL(C) hipLaunchKernelGGL(gather_cpol_kernel<C>, dim3(grid), dim3(256), 0, st, src, idx, out, nthreads)
    switch (cpol) {
    case 0: PROBE_CPOL(0); break;
    case 1: PROBE_CPOL(1); break;
    case 2: PROBE_CPOL(2); break;
    case 3: PROBE_CPOL(3); break;
    case 16: PROBE_CPOL(16); break;
    case 17: PROBE_CPOL(17); break;
    default: return 1;
    }
#undef PROBE_CPOL
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// The parts of a uniform-row SpMV step (probe 5), launched `reps` times back
// to back from here (a launch from Python costs more host time than these
// kernels take): colind/val hold m*ulen entries with columns in
// [origin, origin + n), x holds n values (mode 0) or m (mode 1), y holds m.
// Returns 0, 1 on invalid arguments, 2 on a launch error.
extern "C" int jlust_probe_spmv_parts_f64(int64_t m, int64_t n, int32_t ulen, int32_t origin,
                                          const int32_t *colind, const double *val, const double *x,
                                          double *y, int mode, int reps, void *stream)
{
    if (m <= 0 || n <= 0 || ulen <= 0 || m * ulen > ((int64_t)1 << 31) || !colind || !val || !x || !y ||
        reps < 1)
        return 1;
    if (mode == 1 && n < m) return 1;
    const unsigned grid = (unsigned)((m * 4 + 255) / 256);
    const hipStream_t st = (hipStream_t)stream;
    for (int r = 0; r < reps; ++r) {
        switch (mode) {
        case 0: hipLaunchKernelGGL(spmv_parts_kernel<0>, dim3(grid), dim3(256), 0, st, m, ulen, origin, colind, val, x, y); break;
        case 1: hipLaunchKernelGGL(spmv_parts_kernel<1>, dim3(grid), dim3(256), 0, st, m, ulen, origin, colind, val, x, y); break;
        case 2: hipLaunchKernelGGL(spmv_parts_kernel<2>, dim3(grid), dim3(256), 0, st, m, ulen, origin, colind, val, x, y); break;
        case 3: hipLaunchKernelGGL(spmv_parts_kernel<3>, dim3(grid), dim3(256), 0, st, m, ulen, origin, colind, val, x, y); break;
        default: return 1;
        }
    }
    return hipGetLastError() == hipSuccess ? 0 : 2;
}
