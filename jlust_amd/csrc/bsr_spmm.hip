// bsr_spmm.hip -- BSR (16 x 16 blocks) SpMM C = alpha*A*B + beta*C on the
// gfx950 fp32 matrix cores (v_mfma_f32_16x16x4_f32).
//
// JLUST's BSR layout: Formats.BSRRight/BSRLeft (src/named_formats.jl:106-128),
// block-row pointers and block-column indices at level 2, values block-major,
// row-major inside a block for BSRRight (ext/CUDAExt/CUDAExt.jl:144-156).
// The reference sends BSR SpMM to execute(::EmitterBackend, ::Op{:SpMM})
// (KernelAbstractionsExt.jl:35-37), which does not compute it; this kernel
// implements the definition C[16R+r, c] = alpha*sum_q sum_s V_q[r][s] *
// B[16*bcol_q + s, c] + beta*C.
//
// One workgroup owns one block-row; its 4 waves split each 256-column pass
// into 4 x 64 columns (V is read from HBM once, the other waves hit L1).  A 16 x 16 block times a 16 x 16 slab of B is four MFMA 16x16x4
// steps.  The contraction index is split as s = 4*g + step (g = lane / 16),
// so every lane needs 4 consecutive s of its row (A) and of its column (B):
//   A operand: lane (i = lane % 16, g) holds V_q[i][4g .. 4g+3]  (one float4
//              of a row-major block);
//   B operand: lane (j = lane % 16, g) holds B[16*bcol + 4g .. +3, c0 + j]
//              (one float4 of a column-major B column);
//   result:    lane (j, g) holds C rows 16R + 4g .. +3 of column c0 + j, so
//              the epilogue is one float4 load/store per 16-column tile.
// Block-rows are mapped XCD-major: the 8 XCDs each take one contiguous band
// of block-rows, so the +-bandwidth window of B a band reuses stays in that
// XCD's L2.
#include "common.hpp"

#include <cstdlib>
#include <memory>
#include <type_traits>

// Raw buffer intrinsics (MUBUF with a 128-bit resource in SGPRs), bound to
// the LLVM intrinsics by name; declared at file scope, since a declaration
// with internal linkage would have to be defined.
typedef __attribute__((address_space(3))) void bsr_lds_void;
typedef int bsr_int32x4 __attribute__((ext_vector_type(4)));
typedef float bsr_floatx4 __attribute__((ext_vector_type(4)));
__device__ void raw_buffer_load_lds(bsr_int32x4 rsrc, bsr_lds_void *lds, int size, int voffset, int soffset,
                                    int offset, int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");
__device__ void raw_buffer_store_v4f32(bsr_floatx4 data, bsr_int32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.store.v4f32");
__device__ bsr_floatx4 raw_buffer_load_v4f32(bsr_int32x4 rsrc, int voffset, int soffset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4f32");

namespace jlust {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int BSR_BS = 16;
constexpr int BSR_WAVES = 4;                 // waves per workgroup (one block-row)
constexpr int BSR_WTILES = 4;                // 16-column tiles per wave per pass
constexpr int BSR_PASS = 16 * BSR_WTILES * BSR_WAVES;   // 256 columns per pass

// VEC: B, C 16-byte aligned with ld % 4 == 0 (float4 access).
template <bool ROW_MAJOR, bool VEC>
__global__ __launch_bounds__(64 * BSR_WAVES) void bsr16_spmm_mfma_kernel(
    int64_t mb, int32_t origin, const int32_t *__restrict__ browptr,
    const int32_t *__restrict__ bcolind, const float *__restrict__ val, int64_t k, float alpha,
    const float *__restrict__ B, int64_t ldb, float beta, int beta_zero, float *__restrict__ C,
    int64_t ldc)
{
    // XCD-major remap of the workgroup index (grid padded to a multiple of 8):
    // XCD x takes block-rows [x*per_xcd, (x+1)*per_xcd).
    const int64_t per_xcd = (int64_t)gridDim.x / NUM_XCD;
    const int64_t R = (int64_t)(blockIdx.x % NUM_XCD) * per_xcd + blockIdx.x / NUM_XCD;
    if (R >= mb) return;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i = lane & 15;       // block row (A operand) / column in tile (B, C)
    const int g = lane >> 4;       // group of 4 in the contraction / C row group
    const int64_t q0 = (int64_t)browptr[R] - origin;
    const int64_t q1 = (int64_t)browptr[R + 1] - origin;
    const int64_t crow = R * BSR_BS + 4 * g;

    for (int64_t pass = 0; pass < k; pass += BSR_PASS) {
        const int64_t c0 = pass + (int64_t)wave * 16 * BSR_WTILES;   // this wave's first column
        if (c0 >= k) continue;
        floatx4 acc[BSR_WTILES];
#pragma unroll
        for (int t = 0; t < BSR_WTILES; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};

        for (int64_t q = q0; q < q1; ++q) {
            const int64_t brow = ((int64_t)bcolind[q] - origin) * BSR_BS + 4 * g;
            const float *vb = val + q * (BSR_BS * BSR_BS);
            floatx4 a;
            if (ROW_MAJOR) {
                a = *reinterpret_cast<const floatx4 *>(vb + i * BSR_BS + 4 * g);
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) a[u] = vb[(4 * g + u) * BSR_BS + i];
            }
            floatx4 b[BSR_WTILES];
#pragma unroll
            for (int t = 0; t < BSR_WTILES; ++t) {
                const int64_t col = c0 + 16 * t + i;
                if (col < k) {
                    const float *src = B + brow + col * ldb;
                    if (VEC) {
                        b[t] = *reinterpret_cast<const floatx4 *>(src);
                    } else {
#pragma unroll
                        for (int u = 0; u < 4; ++u) b[t][u] = src[u];
                    }
                } else {
                    b[t] = floatx4{0.f, 0.f, 0.f, 0.f};
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int t = 0; t < BSR_WTILES; ++t)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], b[t][u], acc[t], 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < BSR_WTILES; ++t) {
            const int64_t col = c0 + 16 * t + i;
            if (col >= k) continue;
            float *dst = C + crow + col * ldc;
            floatx4 out = acc[t] * alpha;
            if (!beta_zero) {
                floatx4 old;
                if (VEC) old = *reinterpret_cast<const floatx4 *>(dst);
                else
#pragma unroll
                    for (int u = 0; u < 4; ++u) old[u] = dst[u];
                out += beta * old;
            }
            if (VEC) {
                *reinterpret_cast<floatx4 *>(dst) = out;
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) dst[u] = out[u];
            }
        }
    }
}

// Float64 blocks: the same tiling on the fp64 matrix cores
// (v_mfma_f64_16x16x4_f64).  Each step takes one double of A and one of B per
// lane (A row lane % 16, B column lane % 16, contraction index lane / 16, as
// in the fp32 step) and accumulates a 16 x 16 double tile held as four
// doubles per lane; but where the fp32 step leaves rows 4g .. 4g+3 in lane
// (j, g), the fp64 step leaves rows g, g+4, g+8, g+12 (register v: row
// g + 4v; checked on gfx950 with a one-wave probe).  Lane (i, g) therefore
// feeds A's row p(i) = 4 (i % 4) + i / 4: the step's output row g + 4v is
// then A's row 4g + v, and lane (j, g) holds rows 16R + 4g .. +3 of column
// c0 + j as in the fp32 kernel, one contiguous double4 of C.  The
// contraction split s = 4g + step is the fp32 kernel's, so lane (i, g) needs
// V_q[p(i)][4g .. 4g+3] and B[16*bcol + 4g .. +3, c0 + i], 32 contiguous
// bytes each.  VEC: values, B and C 32-byte aligned and ldb, ldc multiples
// of 4 (double4 access); otherwise element loads and stores.
typedef double doublex4 __attribute__((ext_vector_type(4)));

template <bool ROW_MAJOR, bool VEC>
__global__ __launch_bounds__(64 * BSR_WAVES) void bsr16_spmm_f64_kernel(
    int64_t mb, int32_t origin, const int32_t *__restrict__ browptr,
    const int32_t *__restrict__ bcolind, const double *__restrict__ val, int64_t k, double alpha,
    const double *__restrict__ B, int64_t ldb, double beta, int beta_zero, double *__restrict__ C,
    int64_t ldc)
{
    const int64_t per_xcd = (int64_t)gridDim.x / NUM_XCD;
    const int64_t R = (int64_t)(blockIdx.x % NUM_XCD) * per_xcd + blockIdx.x / NUM_XCD;
    if (R >= mb) return;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int i = lane & 15;
    const int g = lane >> 4;
    const int ar = 4 * (i & 3) + (i >> 2);     // the A row this lane feeds
    const int64_t q0 = (int64_t)browptr[R] - origin;
    const int64_t q1 = (int64_t)browptr[R + 1] - origin;
    const int64_t crow = R * BSR_BS + 4 * g;
    const doublex4 zero = {0.0, 0.0, 0.0, 0.0};

    for (int64_t pass = 0; pass < k; pass += BSR_PASS) {
        const int64_t c0 = pass + (int64_t)wave * 16 * BSR_WTILES;
        if (c0 >= k) continue;
        doublex4 acc[BSR_WTILES];
#pragma unroll
        for (int t = 0; t < BSR_WTILES; ++t) acc[t] = zero;

        for (int64_t q = q0; q < q1; ++q) {
            const int64_t brow = ((int64_t)bcolind[q] - origin) * BSR_BS + 4 * g;
            const double *vb = val + q * (BSR_BS * BSR_BS);
            doublex4 a;
            if (ROW_MAJOR && VEC) {
                a = *reinterpret_cast<const doublex4 *>(vb + ar * BSR_BS + 4 * g);
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    a[u] = ROW_MAJOR ? vb[ar * BSR_BS + 4 * g + u] : vb[(4 * g + u) * BSR_BS + ar];
            }
            doublex4 b[BSR_WTILES];
#pragma unroll
            for (int t = 0; t < BSR_WTILES; ++t) {
                const int64_t col = c0 + 16 * t + i;
                if (col < k) {
                    const double *src = B + brow + col * ldb;
                    if (VEC) {
                        b[t] = *reinterpret_cast<const doublex4 *>(src);
                    } else {
#pragma unroll
                        for (int u = 0; u < 4; ++u) b[t][u] = src[u];
                    }
                } else {
                    b[t] = zero;
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int t = 0; t < BSR_WTILES; ++t)
                    acc[t] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[u], b[t][u], acc[t], 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < BSR_WTILES; ++t) {
            const int64_t col = c0 + 16 * t + i;
            if (col >= k) continue;
            double *dst = C + crow + col * ldc;
            doublex4 out = acc[t] * alpha;
            if (!beta_zero) {
                doublex4 old;
                if (VEC) old = *reinterpret_cast<const doublex4 *>(dst);
                else
#pragma unroll
                    for (int u = 0; u < 4; ++u) old[u] = dst[u];
                out += beta * old;
            }
            if (VEC) {
                *reinterpret_cast<doublex4 *>(dst) = out;
            } else {
#pragma unroll
                for (int u = 0; u < 4; ++u) dst[u] = out[u];
            }
        }
    }
}

// Row-wave kernel (row-major blocks, B and C float4-aligned).  One wave owns
// one block-row.  Column-major B with a large ldb puts every column in its own
// memory page, so loading B in the MFMA operand layout (16 columns per
// instruction) costs 16 address translations per load.  Here each 16-column
// tile of B is loaded down the columns instead -- lane l covers block
// sq = l/8 of the chunk, rows 4*(l%4) .. +3, column 2t + (l/4)%2 of load t,
// so each quad of lanes reads one whole 64-byte column segment (the address
// unit handles a quad per step when its 64 bytes are contiguous) and one
// load touches 2 columns -- and is transposed into the MFMA layout through a
// per-wave LDS area.  Load t lands at t*BSR_LSTRIDE + 16*slot bytes, slot =
// 8*block + 2*(row group) + column; the 32-byte pad per load puts column i of
// an MFMA operand read at bank 4*i (mod 64), so its 16 lanes hit distinct
// banks.  The chunk's A operands (up to BSR_QCHUNK blocks) stay in
// registers for all of k; the next tile's B is loaded while the current
// tile's MFMAs run.
constexpr int BSR_QCHUNK = 8;
constexpr int BSR_LSTRIDE = 1024 + 32;

template <bool BZ>
__global__ __launch_bounds__(256) void bsr16_spmm_rowwave_kernel(
    int64_t mb, int32_t origin, const int32_t *__restrict__ browptr,
    const int32_t *__restrict__ bcolind, const float *__restrict__ val, int64_t k, float alpha,
    const float *__restrict__ B, int64_t ldb, float beta, float *__restrict__ C, int64_t ldc)
{
    __shared__ __align__(16) char lds[4][BSR_QCHUNK * BSR_LSTRIDE];
    // XCD-major remap (grid padded to a multiple of 8): XCD x takes a
    // contiguous band of block-rows, so the B rows the band shares stay in
    // that XCD's L2.
    const int64_t per_xcd = (int64_t)gridDim.x / NUM_XCD;
    const int64_t wg = (int64_t)(blockIdx.x % NUM_XCD) * per_xcd + blockIdx.x / NUM_XCD;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int64_t R = wg * 4 + wave;
    if (R >= mb) return;                   // whole waves only; no block barrier follows

    char *ws = lds[wave];
    const int i = lane & 15;               // MFMA: A row / B, C column in the tile
    const int g = lane >> 4;               // MFMA: contraction group / C row group
    const int sq = lane >> 3;              // staging: block of the chunk
    const int srow = 4 * (lane & 3);       // a quad of lanes reads one 64-byte column segment
    const int sj = (lane >> 2) & 1;
    // LDS slot of this lane's 16 bytes in a load's area: block sq, row group
    // srow/4, column sj at (8*sq + 2*(srow/4) + sj) * 16, so that the MFMA
    // operand reads below (16 lanes, 16 columns) hit distinct banks.
    const int wslot = (8 * sq + 2 * (lane & 3) + sj) * 16;
    const int64_t crow = R * BSR_BS + 4 * g;
    const int64_t q0 = (int64_t)browptr[R] - origin;
    const int64_t q1 = (int64_t)browptr[R + 1] - origin;
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};

    if (q1 <= q0) {                        // empty block-row: C = beta*C
        for (int64_t c0 = 0; c0 < k; c0 += 16) {
            const int64_t col = c0 + i;
            if (col >= k) continue;
            floatx4 *dst = reinterpret_cast<floatx4 *>(C + crow + col * ldc);
            *dst = BZ ? zero : beta * *dst;
        }
        return;
    }
    for (int64_t qb = q0; qb < q1; qb += BSR_QCHUNK) {
        const int nq = (int)min((int64_t)BSR_QCHUNK, q1 - qb);
        const bool first = qb == q0;
        floatx4 a[BSR_QCHUNK];
#pragma unroll
        for (int qq = 0; qq < BSR_QCHUNK; ++qq)
            a[qq] = qq < nq ? *reinterpret_cast<const floatx4 *>(val + (qb + qq) * 256 + i * 16 + 4 * g)
                            : zero;
        // Staging lanes past the chunk's blocks repeat its last block (their
        // LDS slots are never read).
        const int64_t sb = (int64_t)bcolind[qb + min(sq, nq - 1)] - origin;
        const float *bsrc = B + sb * BSR_BS + srow;
        floatx4 st[8];
        auto load_tile = [&](int64_t c0) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int64_t col = min(c0 + 2 * t + sj, k - 1);
                st[t] = *reinterpret_cast<const floatx4 *>(bsrc + col * ldb);
            }
        };
        load_tile(0);
        for (int64_t c0 = 0; c0 < k; c0 += 16) {
#pragma unroll
            for (int t = 0; t < 8; ++t)
                *reinterpret_cast<floatx4 *>(ws + t * BSR_LSTRIDE + wslot) = st[t];
            if (c0 + 16 < k) load_tile(c0 + 16);
            floatx4 acc = zero;
            const char *rd = ws + (i >> 1) * BSR_LSTRIDE + (g * 2 + (i & 1)) * 16;
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
                if (qq < nq) {
                    const floatx4 b = *reinterpret_cast<const floatx4 *>(rd + qq * 128);
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[qq][u], b[u], acc, 0, 0, 0);
                }
            }
            const int64_t col = c0 + i;
            if (col < k) {
                floatx4 *dst = reinterpret_cast<floatx4 *>(C + crow + col * ldc);
                floatx4 out = alpha * acc;
                if (!first) out += *dst;
                else if (!BZ) out += beta * *dst;
                *dst = out;
            }
        }
    }
}

// Strip kernel (row-major blocks, B and C float4-aligned, byte offsets of B
// and C below 2^31).  A workgroup owns BSR_SR consecutive block-rows, one
// wave each, with the row's blocks (up to BSR_QCHUNK) held as MFMA A operands
// in registers for all of k.  For each 16-column tile the strip's window of B
// -- block-rows [J_min, J_max] of all its blocks, each of the 16 columns one
// contiguous run of (J_max - J_min + 1) * 64 bytes -- sits in LDS, copied
// there with direct global-to-LDS loads (buffer_load_dwordx4 ... lds: 64
// lanes x 16 bytes of one column per instruction, whole 128-byte lines, no
// registers).  Per tile every wave reads all of its row's B operands from the
// window into registers; after a barrier the window is free, so the next
// tile's copies are issued during this tile's MFMAs -- one copy instruction
// before each block's four MFMAs, so they issue in the MFMA chain's
// dependency stalls -- and land while the waves finish the MFMAs and store C.  One wait + barrier per tile finds the
// copies done (vmcnt(1): all but the C store just issued; an explicit
// s_barrier, since a fence would wait for everything).  The window buffer is
// single (78 KB) and the kernel fits 80 VGPRs (buffer resources keep the
// addresses of B and C in SGPRs), so two workgroups share a CU and each has
// a window in flight: one workgroup's copies alone are latency-bound at about
// half the rate of two.  Columns sit BSR_CS bytes apart (a 32-byte pad per
// column), so the 16-byte operand reads of the 64 lanes (16 columns x 4 row
// groups) meet no bank conflict; the 16-byte pad that a 16-lane count
// suggests costs 4 conflict cycles per read (measured by SQ_LDS_BANK_CONFLICT).  A strip whose rows hold more than BSR_QCHUNK blocks
// or whose window exceeds BSR_WMAX block-rows computes its rows with direct
// operand loads instead (same arithmetic).
constexpr int BSR_SR = 12;                        // block-rows (waves) per workgroup
constexpr int BSR_WMAX = BSR_SR + 64;             // window block-rows (a +-32 band)
constexpr int BSR_CS = BSR_WMAX * 64 + 32;        // LDS bytes per column of a window
constexpr int BSR_BUF = 16 * BSR_CS;              // the window buffer

typedef bsr_lds_void lds_void;
typedef bsr_int32x4 int32x4;

// A buffer resource over [p, p + 4 GB): base address, stride 0, no range
// limit, the gfx9 default format word.
__device__ __forceinline__ int32x4 buffer_resource(const void *p)
{
    const uint64_t a = (uint64_t)p;
    int32x4 r;
    r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffff));
    r.z = -1;
    r.w = 0x00020000;
    return r;
}

template <bool BZ>
__global__ __launch_bounds__(64 * BSR_SR) __attribute__((amdgpu_waves_per_eu(6))) 
void bsr16_spmm_strip_kernel(
    int64_t mb, int32_t origin, const int32_t *__restrict__ browptr,
    const int32_t *__restrict__ bcolind, const float *__restrict__ val, int64_t k, float alpha,
    const float *__restrict__ B, int64_t ldb, float beta, float *__restrict__ C, int64_t ldc)
{
    __shared__ __align__(16) char win[BSR_BUF];
    __shared__ int32_t s_jmin[BSR_SR], s_jmax[BSR_SR], s_len[BSR_SR];
    // XCD-major remap of the strip index (grid padded to a multiple of 8).
    const int64_t per_xcd = (int64_t)gridDim.x / NUM_XCD;
    const int64_t strip = (int64_t)(blockIdx.x % NUM_XCD) * per_xcd + blockIdx.x / NUM_XCD;
    const int64_t R0 = strip * BSR_SR;
    if (R0 >= mb) return;                  // whole workgroup
    // Wave-uniform values go to SGPRs (readfirstlane), which keeps the kernel
    // within the 80 VGPRs two workgroups per CU need.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int i = lane & 15;               // MFMA: A row / B, C column in the tile
    const int g = lane >> 4;               // MFMA: contraction group / C row group
    const int64_t R = R0 + wave;
    const bool live = R < mb;
    const int64_t q0 = live ? (int64_t)__builtin_amdgcn_readfirstlane(browptr[R]) - origin : 0;
    const int64_t q1 = live ? (int64_t)__builtin_amdgcn_readfirstlane(browptr[R + 1]) - origin : 0;
    const int nq = (int)(q1 - q0);
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};

    // The strip's window: smallest and largest block column of its blocks.
    {
        int32_t jmin = INT32_MAX, jmax = INT32_MIN;
        for (int64_t q = q0 + lane; q < q1; q += 64) {
            const int32_t j = bcolind[q] - origin;
            jmin = min(jmin, j);
            jmax = max(jmax, j);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            jmin = min(jmin, __shfl_xor(jmin, off, 64));
            jmax = max(jmax, __shfl_xor(jmax, off, 64));
        }
        if (lane == 0) {
            s_jmin[wave] = jmin;
            s_jmax[wave] = jmax;
            s_len[wave] = nq;
        }
    }
    __syncthreads();
    int32_t jw0 = INT32_MAX, jw1 = INT32_MIN, lmax = 0;
#pragma unroll
    for (int w = 0; w < BSR_SR; ++w) {
        jw0 = min(jw0, s_jmin[w]);
        jw1 = max(jw1, s_jmax[w]);
        lmax = max(lmax, s_len[w]);
    }
    jw0 = __builtin_amdgcn_readfirstlane(jw0);
    jw1 = __builtin_amdgcn_readfirstlane(jw1);
    lmax = __builtin_amdgcn_readfirstlane(lmax);
    const int32_t nwin = jw1 >= jw0 ? jw1 - jw0 + 1 : 0;
    const int64_t crow = R * BSR_BS + 4 * g;

    auto store_tile = [&](floatx4 acc, int64_t c0) {
        const int64_t col = c0 + i;
        if (col < k) {
            floatx4 *dst = reinterpret_cast<floatx4 *>(C + crow + col * ldc);
            floatx4 out = alpha * acc;
            if (!BZ) out += beta * *dst;
            *dst = out;
        }
    };
    if (lmax > BSR_QCHUNK || nwin > BSR_WMAX) {
        // Direct operand loads (any row length, any window).
        if (!live) return;
        for (int64_t c0 = 0; c0 < k; c0 += 16) {
            const int64_t colc = c0 + i < k ? c0 + i : k - 1;
            floatx4 acc = zero;
            for (int64_t q = q0; q < q1; ++q) {
                const floatx4 a = *reinterpret_cast<const floatx4 *>(val + q * 256 + i * 16 + 4 * g);
                const int64_t brow = ((int64_t)bcolind[q] - origin) * BSR_BS + 4 * g;
                const floatx4 b = *reinterpret_cast<const floatx4 *>(B + brow + colc * ldb);
#pragma unroll
                for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], b[u], acc, 0, 0, 0);
            }
            store_tile(acc, c0);
        }
        return;
    }

    // A operands and window-relative block rows (wave-uniform) of this row.
    floatx4 a[BSR_QCHUNK];
    int32_t jrel[BSR_QCHUNK];
#pragma unroll
    for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
        a[qq] = qq < nq ? *reinterpret_cast<const floatx4 *>(val + (q0 + qq) * 256 + i * 16 + 4 * g) : zero;
        jrel[qq] = qq < nq ? __builtin_amdgcn_readfirstlane(bcolind[q0 + qq] - origin - jw0) : 0;
    }
    // Window copy of one tile: instruction ii = (column j, part p) moves the
    // column's floats [256 p, 256 p + 256) of the window; lanes past the
    // window's end, and columns past k, are masked off.
    const int npc = (nwin * 16 + 255) / 256;     // instructions per column
    const int ninst = 16 * npc;
    const int64_t wfloats = (int64_t)nwin * 16;
    const float *bwin = B + (int64_t)jw0 * BSR_BS;
    const uint32_t col_off = (uint32_t)(i * BSR_CS + 16 * g);
    const int lane16 = lane * 16;
    const int32x4 rs_b = buffer_resource(bwin);  // B's window: lane offset in a VGPR, the rest in an SGPR
    auto copy_one = [&](int64_t c0, int ii) {
        const int j = ii / npc, p = ii % npc;
        if (c0 + j >= k) return;
        const int fu = p * 256;                        // floats, wave-uniform
        const int so = (int)((fu + (c0 + j) * ldb) * 4); // bytes, wave-uniform
        if (fu + 4 * lane < wfloats)
            raw_buffer_load_lds(rs_b, (lds_void *)(win + j * BSR_CS + p * 1024), 16, lane16, so, 0, 0);
    };
    auto copy_tile = [&](int64_t c0) {
        for (int ii = wave; ii < ninst; ii += BSR_SR) copy_one(c0, ii);
    };
    const int32x4 rs_c = buffer_resource(C);
    const int c_lane = (4 * g + i * (int)ldc) * 4;
    copy_tile(0);
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("s_barrier" ::: "memory");
    for (int64_t c0 = 0; c0 < k; c0 += 16) {
        // This tile's B operands into registers; then the window is free.
        floatx4 b[BSR_QCHUNK];
        uint32_t co = col_off;
        asm volatile("" : "+v"(co));           // the read addresses are formed per tile, not kept
#pragma unroll
        for (int qq = 0; qq < BSR_QCHUNK; ++qq) b[qq] = *reinterpret_cast<const floatx4 *>(win + co + jrel[qq] * 64);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // One copy instruction of the next tile before each block's MFMAs (the
        // branches keep the order), the rest after: the copies issue in the
        // MFMA chain's dependency stalls instead of ahead of it.
        floatx4 acc = zero;
        const bool more = c0 + 16 < k;
        int ii = wave;
#pragma unroll
        for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
            if (more && ii < ninst) {
                copy_one(c0 + 16, ii);
                ii += BSR_SR;
            }
            asm volatile("" ::: "memory");
            if (live && qq < nq) {
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[qq][u], b[qq][u], acc, 0, 0, 0);
            }
        }
        for (; more && ii < ninst; ii += BSR_SR) copy_one(c0 + 16, ii);
        asm volatile("" ::: "memory");        // every copy is issued before the store
        if (live) {
            // C's lane part (4 g + i ldc) * 4 bytes in a VGPR, the rest in an SGPR.
            if (c0 + i < k) {
                const int so_c = (int)((R * BSR_BS + c0 * ldc) * 4);
                floatx4 out = alpha * acc;
                if (!BZ) out += beta * raw_buffer_load_v4f32(rs_c, c_lane, so_c, 0);
                raw_buffer_store_v4f32(out, rs_c, c_lane, so_c, 0);
            }
            __builtin_amdgcn_s_waitcnt(0x0001);   // vmcnt(1): every copy; the C store may be in flight
        } else {
            __builtin_amdgcn_s_waitcnt(0);
        }
        asm volatile("s_barrier" ::: "memory");
    }
    __builtin_amdgcn_s_waitcnt(0);
}

// Wide strip kernel: the strip kernel's window scheme over strips of
// BSRW_SR = 24 block-rows, two per wave (rows 2w and 2w + 1 of the strip, so
// a wave's two C tiles are whole 128-byte lines per column), one workgroup
// per CU.  Under a +-32 band the B rows a strip uses are copied to LDS about
// 3.5 times per product instead of 6 times with 12-row strips; the copies
// through L1 and L2, limited by the misses a CU keeps in flight, are what
// bound the 12-row kernel.  A wave holds both rows' A operands (16 blocks)
// for all of k; per tile it reads both rows' B operands from the window, and
// after the barrier issues the next tile's copies between the blocks' MFMAs
// (two accumulator chains, one per row).  The window's column stride keeps
// the stride in 4-byte banks at 72 mod 128, which leaves the operand reads
// free of bank conflicts.
//
// The workgroups are persistent, one per CU: XCD x = blockIdx % 8 owns
// strips [lo, hi), a contiguous run, and its G workgroups take lo + w,
// lo + w + G, ..., so the strips in flight on an XCD are neighbours sharing
// B rows in its L2; a last round of r <= G / 2 strips is cut into f = G / r
// column ranges each.  With one workgroup per CU nothing covers a strip's
// set-up, so a unit of four or more tiles sets up the next unit's strip
// during its last four tiles: the rows' block ranges (tile -4), block
// columns (-3), per-wave column ranges (-2), and, in the last tile, the
// window; the last tile's copies then move the next strip's first window,
// and its A operands are loaded as this strip's last MFMAs release their
// registers.
constexpr int BSRW_WAVES = 12;                    // waves per workgroup
constexpr int BSRW_SR = 2 * BSRW_WAVES;           // block-rows per workgroup
constexpr int BSRW_WMAX = BSRW_SR + 64;           // window block-rows (a +-32 band)
constexpr int BSRW_CS = BSRW_WMAX * 64 + 288;     // LDS bytes per window column
constexpr int BSRW_BUF = 16 * BSRW_CS;            // the window buffer (94,720 B)
constexpr int BSRW_ZROW = BSRW_WMAX;              // window row of zeros (in each column's pad)
static_assert((BSRW_ZROW + 1) * 64 <= BSRW_CS && BSRW_ZROW < 256, "zero row in the pad");
#ifndef JLUST_BSRW_CPQ
#define JLUST_BSRW_CPQ 2
#endif
constexpr int BSRW_CPQ = JLUST_BSRW_CPQ;          // copies issued per block pair

template <bool BZ>
__global__ __launch_bounds__(64 * BSRW_WAVES) __attribute__((amdgpu_waves_per_eu(3)))
void bsr16_spmm_wide_strip_kernel(
    int64_t mb, int32_t origin, const int32_t *__restrict__ browptr,
    const int32_t *__restrict__ bcolind, const float *__restrict__ val, int64_t k, float alpha,
    const float *__restrict__ B, int64_t ldb, float beta, float *__restrict__ C, int64_t ldc)
{
    __shared__ __align__(16) char win[BSRW_BUF];
    __shared__ int32_t s_jmin[2][BSRW_WAVES], s_jmax[2][BSRW_WAVES], s_len[2][BSRW_WAVES];
    const int nstrips = (int)((mb + BSRW_SR - 1) / BSRW_SR);
    const int G = (int)gridDim.x / NUM_XCD;
    const int xcd = (int)blockIdx.x % NUM_XCD;
    const int wl = (int)blockIdx.x / NUM_XCD;
    const int lo = (int)((int64_t)xcd * nstrips / NUM_XCD), hi = (int)((int64_t)(xcd + 1) * nstrips / NUM_XCD);
    if (hi <= lo) return;                  // whole workgroup
    const int kk = (int)k;                 // k < 2^31 - 16 (checked by the host)
    const int ntiles = (kk + 15) / 16;
    const int rounds = (hi - lo + G - 1) / G;
    const int rlast = hi - lo - (rounds - 1) * G;          // strips in the last round, 1..G
    const int fsplit = min(2 * rlast <= G ? G / rlast : 1, ntiles);
    // Work unit it of this workgroup: strip s, tiles [t0, t1).
    auto unit = [&](int it, int &s, int &t0, int &t1) -> bool {
        if (it < rounds - 1) {
            s = lo + wl + it * G;
            t0 = 0;
            t1 = ntiles;
            return true;
        }
        if (it > rounds - 1 || wl >= rlast * fsplit) return false;
        s = lo + (rounds - 1) * G + wl / fsplit;
        const int c = wl % fsplit;
        t0 = c * ntiles / fsplit;
        t1 = (c + 1) * ntiles / fsplit;
        return true;
    };
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int i = lane & 15;               // MFMA: A row / B, C column in the tile
    const int g = lane >> 4;               // MFMA: contraction group / C row group
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    const uint32_t col_off = (uint32_t)(i * BSRW_CS + 16 * g);
    const int lane16 = lane * 16;
    const int c_lane = (4 * g + i * (int)ldc) * 4;
    const int32x4 rs_c = buffer_resource(C);
    // Window copies: a tile's window is 16 columns x 6 parts of 1024 bytes
    // (nwin <= 88 block-rows, 5,632 bytes a column), 96 instructions, 8 per
    // wave: wave w moves part w % 6 of columns 2t + w / 6, t = 0..7.  Lanes
    // past the window's end are masked off, and a part wholly past it, or a
    // column past k, is skipped.
    static_assert(16 * 6 == 8 * BSRW_WAVES && BSRW_WMAX * 64 <= 6 * 1024, "wide strip copy split");
    const int cpar = wave / 6, cpart = wave % 6;
    const uint32_t lds_base = (uint32_t)(cpar * BSRW_CS + cpart * 1024);
    const int g_base = (int)((cpart * 256 + cpar * ldb) * 4);   // bytes, wave-uniform
    auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    // The zero row of each window column, in the column's pad, which no copy
    // writes (the first unit's set-up barriers precede every read).
    if (threadIdx.x < 64)
        *reinterpret_cast<floatx4 *>(win + (threadIdx.x >> 2) * BSRW_CS + BSRW_ZROW * 64 + (threadIdx.x & 3) * 16) = zero;

    // ---- the strip being computed.
    bool live0 = false, live1 = false, windowed = false, cvalid = false, lane_ok = false;
    int Ra = 0, nq0 = 0, nq1 = 0;
    int64_t qa = 0, qb = 0;
    int32x4 rs_b = buffer_resource(B);
    uint32_t jp[4] = {0u, 0u, 0u, 0u};     // window rows of the blocks, 8 bits each
    // ---- set-up of a strip in five steps: 1-4 write the *n variables (the
    // strip being set up), 5 adopts them.
    int Ran = 0;
    bool live0n = false, live1n = false, windowedn = false, cvalidn = false, lane_okn = false;
    int32_t pa = 0, pb = 0, pc = 0, bcoln = 0, jw0n = 0;
    int qan = 0, qbn = 0, nq0n = 0, nq1n = 0;
    uint32_t jpn[4] = {0u, 0u, 0u, 0u};
    // 1: the rows' block ranges.
    auto setup1 = [&](int sn) {
        Ran = sn * BSRW_SR + 2 * wave;
        live0n = Ran < mb;
        live1n = Ran + 1 < mb;
        pa = live0n ? browptr[Ran] : 0;
        pb = live0n ? browptr[Ran + 1] : 0;
        pc = live1n ? browptr[Ran + 2] : pb;
    };
    // 2: the rows' block columns, one per lane (row 0's then row 1's), when
    // both rows are short enough to be held as operands.
    auto setup2 = [&]() {
        qan = __builtin_amdgcn_readfirstlane(pa) - origin;
        qbn = __builtin_amdgcn_readfirstlane(pb) - origin;
        const int qcn = __builtin_amdgcn_readfirstlane(pc) - origin;
        nq0n = qbn - qan;
        nq1n = qcn - qbn;
        bcoln = 0;
        if (nq0n <= BSR_QCHUNK && nq1n <= BSR_QCHUNK && lane < qcn - qan) bcoln = bcolind[qan + lane] - origin;
    };
    // 3: per wave the rows' column range and longer length.
    auto setup3 = [&](int par) {
        const bool has = nq0n <= BSR_QCHUNK && nq1n <= BSR_QCHUNK && lane < nq0n + nq1n;
        int32_t jmin = has ? bcoln : INT32_MAX, jmax = has ? bcoln : INT32_MIN;
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {    // the columns sit in lanes 0..15
            jmin = min(jmin, __shfl_xor(jmin, off, 64));
            jmax = max(jmax, __shfl_xor(jmax, off, 64));
        }
        if (lane == 0) {
            s_jmin[par][wave] = jmin;
            s_jmax[par][wave] = jmax;
            s_len[par][wave] = max(nq0n, nq1n);
        }
    };
    // 4 (after a barrier): the strip's window, the blocks' window rows and
    // this wave's copy masks.
    auto setup4 = [&](int par) {
        int32_t jw0 = INT32_MAX, jw1 = INT32_MIN, lmax = 0;
        if (lane < BSRW_WAVES) {
            jw0 = s_jmin[par][lane];
            jw1 = s_jmax[par][lane];
            lmax = s_len[par][lane];
        }
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            jw0 = min(jw0, __shfl_xor(jw0, off, 64));
            jw1 = max(jw1, __shfl_xor(jw1, off, 64));
            lmax = max(lmax, __shfl_xor(lmax, off, 64));
        }
        jw0 = __builtin_amdgcn_readfirstlane(jw0);
        jw1 = __builtin_amdgcn_readfirstlane(jw1);
        lmax = __builtin_amdgcn_readfirstlane(lmax);
        const int32_t nwin = jw1 >= jw0 ? jw1 - jw0 + 1 : 0;
        jw0n = nwin > 0 ? jw0 : 0;
        windowedn = lmax <= BSR_QCHUNK && nwin <= BSRW_WMAX;
        const int wfloats = nwin * 16;
        cvalidn = cpart * 256 < wfloats;
        lane_okn = cpart * 256 + 4 * lane < wfloats;
        // A block a row does not have reads the zero row (its A operand is
        // zero too), so every wave runs all 16 blocks' MFMAs unguarded.
#pragma unroll
        for (int x = 0; x < 4; ++x) jpn[x] = BSRW_ZROW * 0x01010101u;
        if (windowedn) {
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
                const uint32_t sh = 8 * (qq & 3);
                if (qq < nq0n)
                    jpn[qq >> 2] ^= ((uint32_t)(__builtin_amdgcn_readlane(bcoln, qq) - jw0n) ^ BSRW_ZROW) << sh;
                if (qq < nq1n)
                    jpn[2 + (qq >> 2)] ^= ((uint32_t)(__builtin_amdgcn_readlane(bcoln, nq0n + qq) - jw0n) ^ BSRW_ZROW) << sh;
            }
        }
    };
    // 5: adopt the strip set up.
    auto setup5 = [&]() {
        Ra = Ran;
        live0 = live0n;
        live1 = live1n;
        qa = qan;
        qb = qbn;
        nq0 = live0n ? nq0n : 0;
        nq1 = live1n ? nq1n : 0;
        windowed = windowedn;
        cvalid = cvalidn;
        lane_ok = lane_okn;
        rs_b = buffer_resource(B + (int64_t)jw0n * BSR_BS);
#pragma unroll
        for (int x = 0; x < 4; ++x) jp[x] = jpn[x];
    };
    auto load_a0 = [&](floatx4 &dst, int qq) {
        dst = live0n && qq < nq0n ? *reinterpret_cast<const floatx4 *>(val + ((int64_t)qan + qq) * 256 + i * 16 + 4 * g) : zero;
    };
    auto load_a1 = [&](floatx4 &dst, int qq) {
        dst = live1n && qq < nq1n ? *reinterpret_cast<const floatx4 *>(val + ((int64_t)qbn + qq) * 256 + i * 16 + 4 * g) : zero;
    };
    // Copy t (0..7) of this wave for the tile at column c0 of a window at rs.
    auto copy_t = [&](int32x4 rs, bool cv, bool lok, int c0, int t) {
        if (!cv || c0 + 2 * t + cpar >= kk) return;
        const int so = g_base + (int)((int64_t)(c0 + 2 * t) * ldb * 4);
        if (lok) raw_buffer_load_lds(rs, (lds_void *)(win + lds_base + t * 2 * BSRW_CS), 16, lane16, so, 0, 0);
    };

    floatx4 a0[BSR_QCHUNK], a1[BSR_QCHUNK];
#pragma unroll
    for (int qq = 0; qq < BSR_QCHUNK; ++qq) a0[qq] = a1[qq] = zero;
    // ready: steps 1-4, the A operand loads and the first window's copies of
    // strip s were done during the previous unit's tiles.
    bool ready = false;
    int par = 0;
    int s = 0, t0 = 0, t1 = 0, sn = 0, t0n = 0, t1n = 0;
    bool has = unit(0, s, t0, t1), hasn = false;
    for (int it = 0; has; ++it, par ^= 1, has = hasn, s = sn, t0 = t0n, t1 = t1n) {
        hasn = unit(it + 1, sn, t0n, t1n);
        const bool pre = hasn && t1 - t0 >= 4;  // steps 1-4 of strip sn run during this unit's tiles
        if (!ready) {
            setup1(s);
            setup2();
            setup3(par);
            barrier();
            setup4(par);
            if (windowedn) {
#pragma unroll
                for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
                    load_a0(a0[qq], qq);
                    load_a1(a1[qq], qq);
                }
                const int32x4 rsn = buffer_resource(B + (int64_t)jw0n * BSR_BS);
#pragma unroll
                for (int t = 0; t < 8; ++t) copy_t(rsn, cvalidn, lane_okn, t0 * 16, t);
            }
            __builtin_amdgcn_s_waitcnt(0);
            asm volatile("s_barrier" ::: "memory");
        }
        setup5();
        ready = false;

        if (!windowed) {
            // Direct operand loads (any row length, any window), row by row.
            for (int r = 0; r < 2; ++r) {
                if (!(r ? live1 : live0)) break;
                const int64_t q0 = r ? qb : qa, q1 = r ? qb + nq1 : qa + nq0;
                const int64_t crow = (int64_t)(Ra + r) * BSR_BS + 4 * g;
                for (int64_t c0 = (int64_t)t0 * 16; c0 < k && c0 < (int64_t)t1 * 16; c0 += 16) {
                    const int64_t colc = c0 + i < k ? c0 + i : k - 1;
                    floatx4 acc = zero;
                    for (int64_t q = q0; q < q1; ++q) {
                        const floatx4 a = *reinterpret_cast<const floatx4 *>(val + q * 256 + i * 16 + 4 * g);
                        const int64_t brow = ((int64_t)bcolind[q] - origin) * BSR_BS + 4 * g;
                        const floatx4 b = *reinterpret_cast<const floatx4 *>(B + brow + colc * ldb);
#pragma unroll
                        for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], b[u], acc, 0, 0, 0);
                    }
                    if (c0 + i < k) {
                        floatx4 *dst = reinterpret_cast<floatx4 *>(C + crow + (c0 + i) * ldc);
                        floatx4 out = alpha * acc;
                        if (!BZ) out += beta * *dst;
                        *dst = out;
                    }
                }
            }
            __builtin_amdgcn_s_waitcnt(0);
            asm volatile("s_barrier" ::: "memory");   // every wave is past step 5
            continue;
        }

        // One tile; the unit's last tile is a separate instance, the only one
        // that loads A operands, so that the compiler sees none in flight in
        // the other tiles and adds no wait before their MFMAs: the C stores of
        // a tile stay in flight into the next.
        auto tile = [&](int t, auto last_tag) {
            constexpr bool last = decltype(last_tag)::value;
            const int c0 = t * 16;
            floatx4 b0[BSR_QCHUNK], b1[BSR_QCHUNK];
            uint32_t co = col_off, j0 = jp[0], j1 = jp[1], j2 = jp[2], j3 = jp[3];
            asm volatile("" : "+v"(co), "+s"(j0), "+s"(j1), "+s"(j2), "+s"(j3));
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
                const uint32_t r0 = ((qq < 4 ? j0 : j1) >> (8 * (qq & 3))) & 0xffu;
                const uint32_t r1 = ((qq < 4 ? j2 : j3) >> (8 * (qq & 3))) & 0xffu;
                b0[qq] = *reinterpret_cast<const floatx4 *>(win + co + r0 * 64);
                b1[qq] = *reinterpret_cast<const floatx4 *>(win + co + r1 * 64);
            }
            barrier();                     // the window is free
            if (pre && t == t1 - 4) setup1(sn);
            if (pre && t == t1 - 3) setup2();
            if (last && pre) setup4(par ^ 1);
            asm volatile("" ::: "memory");
            // The copies of the next tile of this strip or, in the last tile,
            // of the next strip's first tile; and in the last tile the next
            // strip's A operands, each after its block's MFMAs.
            const bool nxt = last && pre && windowedn;
            const bool cv = last ? nxt && cvalidn : cvalid;
            const bool lok = last ? lane_okn : lane_ok;
            const int32x4 rsn = last ? buffer_resource(B + (int64_t)jw0n * BSR_BS) : rs_b;
            const int cn = last ? t0n * 16 : c0 + 16;
            floatx4 acc0 = zero, acc1 = zero;
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
#pragma unroll
                for (int cc = 0; cc < BSRW_CPQ; ++cc) {
                    const int tt = qq * BSRW_CPQ + cc;
                    if (tt < 8) copy_t(rsn, cv, lok, cn, tt);
                }
                asm volatile("" ::: "memory");
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[qq][u], b0[qq][u], acc0, 0, 0, 0);
                if (last && nxt) load_a0(a0[qq], qq);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[qq][u], b1[qq][u], acc1, 0, 0, 0);
                if (last && nxt) load_a1(a1[qq], qq);
            }
            asm volatile("" ::: "memory");
            if (c0 + i < kk) {
                if (live0) {
                    const int so_c = (int)(((int64_t)Ra * BSR_BS + (int64_t)c0 * ldc) * 4);
                    floatx4 out = alpha * acc0;
                    if (!BZ) out += beta * raw_buffer_load_v4f32(rs_c, c_lane, so_c, 0);
                    raw_buffer_store_v4f32(out, rs_c, c_lane, so_c, 0);
                }
                if (live1) {
                    const int so_c = (int)(((int64_t)Ra * BSR_BS + BSR_BS + (int64_t)c0 * ldc) * 4);
                    floatx4 out = alpha * acc1;
                    if (!BZ) out += beta * raw_buffer_load_v4f32(rs_c, c_lane, so_c, 0);
                    raw_buffer_store_v4f32(out, rs_c, c_lane, so_c, 0);
                }
            }
            if (pre && t == t1 - 2) setup3(par ^ 1);
            // Every copy (and A load) landed; the C stores of a tile before
            // the last may be in flight.
            if (last) __builtin_amdgcn_s_waitcnt(0);
            else if (live1) __builtin_amdgcn_s_waitcnt(0x0002);       // vmcnt(2)
            else if (live0) __builtin_amdgcn_s_waitcnt(0x0001);       // vmcnt(1)
            else __builtin_amdgcn_s_waitcnt(0);
            asm volatile("s_barrier" ::: "memory");
        };
        for (int t = t0; t < t1 - 1; ++t) tile(t, std::false_type{});
        tile(t1 - 1, std::true_type{});
        ready = pre;
    }
    __builtin_amdgcn_s_waitcnt(0);
}

// Long-row kernel: the 24-row kernel above, and strips whose rows hold 9 to
// 16 blocks.  Such a strip runs as two halves of 12 rows, one row a wave,
// the row's blocks in two groups of up to 8 that take the register slots of
// the 24-row kernel's two rows (a0: blocks 0..7, a1: 8..15); the copies,
// operand reads and MFMAs are the same, and a tile's C is the two groups'
// sums.  Each half is set up at its start.  Strips of rows of at most 8
// blocks run as in the 24-row kernel.  Taken when the rows hold more than 8
// blocks on average; a function of its own because the extra state, as a
// branch of the 24-row kernel, changed that kernel's register assignment and
// cost its 8-block strips about 3 %.
template <bool BZ>
__global__ __launch_bounds__(64 * BSRW_WAVES) __attribute__((amdgpu_waves_per_eu(3)))
void bsr16_spmm_wide_long_kernel(
    int64_t mb, int32_t origin, const int32_t *__restrict__ browptr,
    const int32_t *__restrict__ bcolind, const float *__restrict__ val, int64_t k, float alpha,
    const float *__restrict__ B, int64_t ldb, float beta, float *__restrict__ C, int64_t ldc)
{
    __shared__ __align__(16) char win[BSRW_BUF];
    __shared__ int32_t s_jmin[2][BSRW_WAVES], s_jmax[2][BSRW_WAVES], s_len[2][BSRW_WAVES];
    const int nstrips = (int)((mb + BSRW_SR - 1) / BSRW_SR);
    const int G = (int)gridDim.x / NUM_XCD;
    const int xcd = (int)blockIdx.x % NUM_XCD;
    const int wl = (int)blockIdx.x / NUM_XCD;
    const int lo = (int)((int64_t)xcd * nstrips / NUM_XCD), hi = (int)((int64_t)(xcd + 1) * nstrips / NUM_XCD);
    if (hi <= lo) return;                  // whole workgroup
    const int kk = (int)k;                 // k < 2^31 - 16 (checked by the host)
    const int ntiles = (kk + 15) / 16;
    const int rounds = (hi - lo + G - 1) / G;
    const int rlast = hi - lo - (rounds - 1) * G;          // strips in the last round, 1..G
    const int fsplit = min(2 * rlast <= G ? G / rlast : 1, ntiles);
    // Work unit it of this workgroup: strip s, tiles [t0, t1).
    auto unit = [&](int it, int &s, int &t0, int &t1) -> bool {
        if (it < rounds - 1) {
            s = lo + wl + it * G;
            t0 = 0;
            t1 = ntiles;
            return true;
        }
        if (it > rounds - 1 || wl >= rlast * fsplit) return false;
        s = lo + (rounds - 1) * G + wl / fsplit;
        const int c = wl % fsplit;
        t0 = c * ntiles / fsplit;
        t1 = (c + 1) * ntiles / fsplit;
        return true;
    };
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int i = lane & 15;               // MFMA: A row / B, C column in the tile
    const int g = lane >> 4;               // MFMA: contraction group / C row group
    const floatx4 zero = {0.f, 0.f, 0.f, 0.f};
    const uint32_t col_off = (uint32_t)(i * BSRW_CS + 16 * g);
    const int lane16 = lane * 16;
    const int c_lane = (4 * g + i * (int)ldc) * 4;
    const int32x4 rs_c = buffer_resource(C);
    // Window copies: a tile's window is 16 columns x 6 parts of 1024 bytes
    // (nwin <= 88 block-rows, 5,632 bytes a column), 96 instructions, 8 per
    // wave: wave w moves part w % 6 of columns 2t + w / 6, t = 0..7.  Lanes
    // past the window's end are masked off, and a part wholly past it, or a
    // column past k, is skipped.
    static_assert(16 * 6 == 8 * BSRW_WAVES && BSRW_WMAX * 64 <= 6 * 1024, "wide strip copy split");
    const int cpar = wave / 6, cpart = wave % 6;
    const uint32_t lds_base = (uint32_t)(cpar * BSRW_CS + cpart * 1024);
    const int g_base = (int)((cpart * 256 + cpar * ldb) * 4);   // bytes, wave-uniform
    auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    // The zero row of each window column, in the column's pad, which no copy
    // writes (the first unit's set-up barriers precede every read).
    if (threadIdx.x < 64)
        *reinterpret_cast<floatx4 *>(win + (threadIdx.x >> 2) * BSRW_CS + BSRW_ZROW * 64 + (threadIdx.x & 3) * 16) = zero;

    // ---- the strip being computed.  In long mode (longm; rows of 9 to 16
    // blocks) a wave owns one row, its blocks in two groups of up to 8 (a0:
    // blocks 0..7, a1: 8..15), and the 24 rows run as two halves of 12.
    bool live0 = false, live1 = false, windowed = false, cvalid = false, lane_ok = false, longm = false;
    int Ra = 0, nq0 = 0, nq1 = 0, lmaxs = 0;
    int64_t qa = 0, qb = 0;
    int32x4 rs_b = buffer_resource(B);
    uint32_t jp[4] = {0u, 0u, 0u, 0u};     // window rows of the blocks, 8 bits each
    // ---- set-up of a strip in five steps: 1-4 write the *n variables (the
    // strip being set up), 5 adopts them.
    int Ran = 0;
    bool live0n = false, live1n = false, windowedn = false, cvalidn = false, lane_okn = false, longn = false;
    int32_t pa = 0, pb = 0, pc = 0, bcoln = 0, jw0n = 0;
    int qan = 0, qbn = 0, nq0n = 0, nq1n = 0, lmaxn = 0;
    uint32_t jpn[4] = {0u, 0u, 0u, 0u};
    // 1: the rows' block ranges (long mode: half h's row of this wave).
    auto setup1 = [&](int sn, int h, bool lg) {
        longn = lg;
        Ran = sn * BSRW_SR + (lg ? BSRW_WAVES * h + wave : 2 * wave);
        live0n = Ran < mb;
        live1n = lg ? live0n : Ran + 1 < mb;
        pa = live0n ? browptr[Ran] : 0;
        pb = live0n ? browptr[Ran + 1] : 0;
        pc = !lg && live1n ? browptr[Ran + 2] : pb;
    };
    // 2: the two block groups' ranges [qan, qbn) and [qbn, qcn) -- the two
    // rows, or a long row's first 8 blocks and the rest -- and their block
    // columns, one per lane, when both groups are short enough to be held as
    // operands.
    auto setup2 = [&]() {
        qan = __builtin_amdgcn_readfirstlane(pa) - origin;
        const int q1 = __builtin_amdgcn_readfirstlane(pb) - origin;
        const int qcn = longn ? q1 : __builtin_amdgcn_readfirstlane(pc) - origin;
        qbn = longn ? min(qan + BSR_QCHUNK, q1) : q1;
        nq0n = qbn - qan;
        nq1n = qcn - qbn;
        bcoln = 0;
        if (nq0n <= BSR_QCHUNK && nq1n <= BSR_QCHUNK && lane < qcn - qan) bcoln = bcolind[qan + lane] - origin;
    };
    // 3: per wave the rows' column range and longer length.
    auto setup3 = [&](int par) {
        const bool has = nq0n <= BSR_QCHUNK && nq1n <= BSR_QCHUNK && lane < nq0n + nq1n;
        int32_t jmin = has ? bcoln : INT32_MAX, jmax = has ? bcoln : INT32_MIN;
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {    // the columns sit in lanes 0..15
            jmin = min(jmin, __shfl_xor(jmin, off, 64));
            jmax = max(jmax, __shfl_xor(jmax, off, 64));
        }
        if (lane == 0) {
            s_jmin[par][wave] = jmin;
            s_jmax[par][wave] = jmax;
            s_len[par][wave] = max(nq0n, nq1n);
        }
    };
    // 4 (after a barrier): the strip's window, the blocks' window rows and
    // this wave's copy masks.
    auto setup4 = [&](int par) {
        int32_t jw0 = INT32_MAX, jw1 = INT32_MIN, lmax = 0;
        if (lane < BSRW_WAVES) {
            jw0 = s_jmin[par][lane];
            jw1 = s_jmax[par][lane];
            lmax = s_len[par][lane];
        }
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            jw0 = min(jw0, __shfl_xor(jw0, off, 64));
            jw1 = max(jw1, __shfl_xor(jw1, off, 64));
            lmax = max(lmax, __shfl_xor(lmax, off, 64));
        }
        jw0 = __builtin_amdgcn_readfirstlane(jw0);
        jw1 = __builtin_amdgcn_readfirstlane(jw1);
        lmax = __builtin_amdgcn_readfirstlane(lmax);
        lmaxn = lmax;
        const int32_t nwin = jw1 >= jw0 ? jw1 - jw0 + 1 : 0;
        jw0n = nwin > 0 ? jw0 : 0;
        windowedn = lmax <= BSR_QCHUNK && nwin <= BSRW_WMAX;
        const int wfloats = nwin * 16;
        cvalidn = cpart * 256 < wfloats;
        lane_okn = cpart * 256 + 4 * lane < wfloats;
        // A block a row does not have reads the zero row (its A operand is
        // zero too), so every wave runs all 16 blocks' MFMAs unguarded.
#pragma unroll
        for (int x = 0; x < 4; ++x) jpn[x] = BSRW_ZROW * 0x01010101u;
        if (windowedn) {
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
                const uint32_t sh = 8 * (qq & 3);
                if (qq < nq0n)
                    jpn[qq >> 2] ^= ((uint32_t)(__builtin_amdgcn_readlane(bcoln, qq) - jw0n) ^ BSRW_ZROW) << sh;
                if (qq < nq1n)
                    jpn[2 + (qq >> 2)] ^= ((uint32_t)(__builtin_amdgcn_readlane(bcoln, nq0n + qq) - jw0n) ^ BSRW_ZROW) << sh;
            }
        }
    };
    // 5: adopt the strip set up.
    auto setup5 = [&]() {
        longm = longn;
        lmaxs = lmaxn;
        Ra = Ran;
        live0 = live0n;
        live1 = live1n;
        qa = qan;
        qb = qbn;
        nq0 = live0n ? nq0n : 0;
        nq1 = live1n ? nq1n : 0;
        windowed = windowedn;
        cvalid = cvalidn;
        lane_ok = lane_okn;
        rs_b = buffer_resource(B + (int64_t)jw0n * BSR_BS);
#pragma unroll
        for (int x = 0; x < 4; ++x) jp[x] = jpn[x];
    };
    auto load_a0 = [&](floatx4 &dst, int qq) {
        dst = live0n && qq < nq0n ? *reinterpret_cast<const floatx4 *>(val + ((int64_t)qan + qq) * 256 + i * 16 + 4 * g) : zero;
    };
    auto load_a1 = [&](floatx4 &dst, int qq) {
        dst = live1n && qq < nq1n ? *reinterpret_cast<const floatx4 *>(val + ((int64_t)qbn + qq) * 256 + i * 16 + 4 * g) : zero;
    };
    // Copy t (0..7) of this wave for the tile at column c0 of a window at rs.
    auto copy_t = [&](int32x4 rs, bool cv, bool lok, int c0, int t) {
        if (!cv || c0 + 2 * t + cpar >= kk) return;
        const int so = g_base + (int)((int64_t)(c0 + 2 * t) * ldb * 4);
        if (lok) raw_buffer_load_lds(rs, (lds_void *)(win + lds_base + t * 2 * BSRW_CS), 16, lane16, so, 0, 0);
    };

    floatx4 a0[BSR_QCHUNK], a1[BSR_QCHUNK];
#pragma unroll
    for (int qq = 0; qq < BSR_QCHUNK; ++qq) a0[qq] = a1[qq] = zero;
    // ready: steps 1-4, the A operand loads and the first window's copies of
    // strip s were done during the previous unit's tiles.
    bool ready = false;
    int par = 0;
    int s = 0, t0 = 0, t1 = 0, sn = 0, t0n = 0, t1n = 0;
    bool has = unit(0, s, t0, t1), hasn = false;
    for (int it = 0; has; ++it, par ^= 1, has = hasn, s = sn, t0 = t0n, t1 = t1n) {
        hasn = unit(it + 1, sn, t0n, t1n);
        // Steps 1-4 of strip sn run during this unit's tiles if it has four
        // and its strip is windowed (the direct loads and long mode run no
        // set-up stage; a unit they take leaves ready false).
        const bool pre = hasn && t1 - t0 >= 4;
        if (!ready) {
            setup1(s, 0, false);
            setup2();
            setup3(par);
            barrier();
            setup4(par);
            if (windowedn) {
#pragma unroll
                for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
                    load_a0(a0[qq], qq);
                    load_a1(a1[qq], qq);
                }
                const int32x4 rsn = buffer_resource(B + (int64_t)jw0n * BSR_BS);
#pragma unroll
                for (int t = 0; t < 8; ++t) copy_t(rsn, cvalidn, lane_okn, t0 * 16, t);
            }
            __builtin_amdgcn_s_waitcnt(0);
            asm volatile("s_barrier" ::: "memory");
        }
        setup5();
        ready = false;

        // Direct operand loads (any row length, any window), row by row.
        auto direct = [&]() {
            for (int r = 0; r < (longm ? 1 : 2); ++r) {
                if (!(r ? live1 : live0)) break;
                const int64_t q0 = r ? qb : qa, q1 = longm || r ? qb + nq1 : qa + nq0;
                const int64_t crow = (int64_t)(Ra + r) * BSR_BS + 4 * g;
                for (int64_t c0 = (int64_t)t0 * 16; c0 < k && c0 < (int64_t)t1 * 16; c0 += 16) {
                    const int64_t colc = c0 + i < k ? c0 + i : k - 1;
                    floatx4 acc = zero;
                    for (int64_t q = q0; q < q1; ++q) {
                        const floatx4 a = *reinterpret_cast<const floatx4 *>(val + q * 256 + i * 16 + 4 * g);
                        const int64_t brow = ((int64_t)bcolind[q] - origin) * BSR_BS + 4 * g;
                        const floatx4 b = *reinterpret_cast<const floatx4 *>(B + brow + colc * ldb);
#pragma unroll
                        for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], b[u], acc, 0, 0, 0);
                    }
                    if (c0 + i < k) {
                        floatx4 *dst = reinterpret_cast<floatx4 *>(C + crow + (c0 + i) * ldc);
                        floatx4 out = alpha * acc;
                        if (!BZ) out += beta * *dst;
                        *dst = out;
                    }
                }
            }
            __builtin_amdgcn_s_waitcnt(0);
            asm volatile("s_barrier" ::: "memory");   // every wave is past step 5
        };

        // One tile; the unit's last tile is a separate instance, the only one
        // that loads A operands, so that the compiler sees none in flight in
        // the other tiles and adds no wait before their MFMAs: the C stores of
        // a tile stay in flight into the next.
        auto tile = [&](int t, auto last_tag) {
            constexpr bool last = decltype(last_tag)::value;
            const int c0 = t * 16;
            floatx4 b0[BSR_QCHUNK], b1[BSR_QCHUNK];
            uint32_t co = col_off, j0 = jp[0], j1 = jp[1], j2 = jp[2], j3 = jp[3];
            asm volatile("" : "+v"(co), "+s"(j0), "+s"(j1), "+s"(j2), "+s"(j3));
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
                const uint32_t r0 = ((qq < 4 ? j0 : j1) >> (8 * (qq & 3))) & 0xffu;
                const uint32_t r1 = ((qq < 4 ? j2 : j3) >> (8 * (qq & 3))) & 0xffu;
                b0[qq] = *reinterpret_cast<const floatx4 *>(win + co + r0 * 64);
                b1[qq] = *reinterpret_cast<const floatx4 *>(win + co + r1 * 64);
            }
            barrier();                     // the window is free
            if (pre && t == t1 - 4) setup1(sn, 0, false);
            if (pre && t == t1 - 3) setup2();
            if (last && pre) setup4(par ^ 1);
            asm volatile("" ::: "memory");
            // The copies of the next tile of this strip or, in the last tile,
            // of the next strip's first tile; and in the last tile the next
            // strip's A operands, each after its block's MFMAs.
            const bool nxt = last && pre && windowedn;
            const bool cv = last ? nxt && cvalidn : cvalid;
            const bool lok = last ? lane_okn : lane_ok;
            const int32x4 rsn = last ? buffer_resource(B + (int64_t)jw0n * BSR_BS) : rs_b;
            const int cn = last ? t0n * 16 : c0 + 16;
            floatx4 acc0 = zero, acc1 = zero;
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
#pragma unroll
                for (int cc = 0; cc < BSRW_CPQ; ++cc) {
                    const int tt = qq * BSRW_CPQ + cc;
                    if (tt < 8) copy_t(rsn, cv, lok, cn, tt);
                }
                asm volatile("" ::: "memory");
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[qq][u], b0[qq][u], acc0, 0, 0, 0);
                if (last && nxt) load_a0(a0[qq], qq);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[qq][u], b1[qq][u], acc1, 0, 0, 0);
                if (last && nxt) load_a1(a1[qq], qq);
            }
            asm volatile("" ::: "memory");
            if (longm) {
                // One row: its two block groups' sums.
                if (c0 + i < kk && live0) {
                    const int so_c = (int)(((int64_t)Ra * BSR_BS + (int64_t)c0 * ldc) * 4);
                    floatx4 out = alpha * (acc0 + acc1);
                    if (!BZ) out += beta * raw_buffer_load_v4f32(rs_c, c_lane, so_c, 0);
                    raw_buffer_store_v4f32(out, rs_c, c_lane, so_c, 0);
                }
            } else if (c0 + i < kk) {
                if (live0) {
                    const int so_c = (int)(((int64_t)Ra * BSR_BS + (int64_t)c0 * ldc) * 4);
                    floatx4 out = alpha * acc0;
                    if (!BZ) out += beta * raw_buffer_load_v4f32(rs_c, c_lane, so_c, 0);
                    raw_buffer_store_v4f32(out, rs_c, c_lane, so_c, 0);
                }
                if (live1) {
                    const int so_c = (int)(((int64_t)Ra * BSR_BS + BSR_BS + (int64_t)c0 * ldc) * 4);
                    floatx4 out = alpha * acc1;
                    if (!BZ) out += beta * raw_buffer_load_v4f32(rs_c, c_lane, so_c, 0);
                    raw_buffer_store_v4f32(out, rs_c, c_lane, so_c, 0);
                }
            }
            if (pre && t == t1 - 2) setup3(par ^ 1);
            // Every copy (and A load) landed; the C stores of a tile before
            // the last may be in flight.
            if (last) __builtin_amdgcn_s_waitcnt(0);
            else if (live1 && !longm) __builtin_amdgcn_s_waitcnt(0x0002);   // vmcnt(2)
            else if (live0) __builtin_amdgcn_s_waitcnt(0x0001);             // vmcnt(1)
            else __builtin_amdgcn_s_waitcnt(0);
            asm volatile("s_barrier" ::: "memory");
        };
        // Rows of 9 to 16 blocks: the strip as two halves of 12 rows, one
        // row a wave, each set up at its start; otherwise one pass over
        // the strip set up above.  (One call site of the tile code: two
        // would double its register pressure.)
        const bool first_windowed = windowed;
        const bool lng = !windowed && lmaxs > BSR_QCHUNK && lmaxs <= 2 * BSR_QCHUNK;
        for (int h = 0; h < (lng ? 2 : 1); ++h) {
            if (lng) {
                setup1(s, h, true);
                setup2();
                setup3(par);
                barrier();
                setup4(par);
                if (windowedn) {
#pragma unroll
                    for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
                        load_a0(a0[qq], qq);
                        load_a1(a1[qq], qq);
                    }
                    const int32x4 rsn = buffer_resource(B + (int64_t)jw0n * BSR_BS);
#pragma unroll
                    for (int t = 0; t < 8; ++t) copy_t(rsn, cvalidn, lane_okn, t0 * 16, t);
                }
                __builtin_amdgcn_s_waitcnt(0);
                asm volatile("s_barrier" ::: "memory");
                setup5();
            }
            if (windowed) {
                for (int t = t0; t < t1 - 1; ++t) tile(t, std::false_type{});
                tile(t1 - 1, std::true_type{});
            } else {
                direct();
            }
        }
        if (!first_windowed) continue;     // no next-strip set-up ran
        ready = pre;
    }
    __builtin_amdgcn_s_waitcnt(0);
}

// Float64 strip kernel (row-major blocks; values, B and C 32-byte aligned,
// ldb and ldc multiples of 4; 16 columns of B or C span less than 2^31 bytes).
// The fp32 strip kernel's design on v_mfma_f64_16x16x4_f64: a workgroup of
// BSR64_SR waves owns that many consecutive block-rows, one wave each, with
// the row's blocks (up to BSR_QCHUNK) held as A operands in registers for all
// of k; for each 16-column tile the strip's window of B (block-rows
// [J_min, J_max], each column one contiguous run of 128 bytes per block-row)
// is copied to LDS with direct global-to-LDS loads; every wave reads its B
// operands from the window, a barrier frees it, and the next tile's copies
// are issued between this tile's MFMAs.  In Float64 a window is twice the
// fp32 one (156 KB for a +-32 band), so one workgroup holds the CU's LDS and
// there are twice the VGPRs per wave (three waves per SIMD).  Operand layout
// (see bsr16_spmm_f64_kernel): lane (i, g) feeds A's row 4 (i % 4) + i / 4
// and holds C rows 4g .. 4g+3 of column i; the contraction rows it feeds
// (A's columns, B's rows) are kg, kg+1, kg+4, kg+5 with kg = 2 (g % 2) +
// 8 (g / 2), an order whose window reads meet no LDS bank conflict (below).
// The buffer resources of B and C are rebased per tile (B at the window's
// first row of column c0, C at column c0), so 32-bit offsets cover 16 columns
// of any height.  One workgroup per CU walks its XCD's strips (persistent),
// and a strip's set-up -- its rows' block ranges and columns, window and
// slots, and A operands -- is loaded during the previous strip's last tiles,
// so that the CU's MFMAs do not wait for it (set up at a strip's start, it
// took about a sixth of the time).
constexpr int BSR64_SR = 12;                      // block-rows (waves) per workgroup
constexpr int BSR64_WMAX = BSR64_SR + 64;         // used window block-rows held in LDS
constexpr int BSR64_SPAN = 128;                   // window block-rows the used-row mask covers
#ifndef JLUST_BSR64_PAD
#define JLUST_BSR64_PAD 32
#endif
constexpr int BSR64_PAD = JLUST_BSR64_PAD;        // bytes after each window column
#ifndef JLUST_BSR64_CFRONT
#define JLUST_BSR64_CFRONT 0
#endif
#ifndef JLUST_BSR64_CPB
#define JLUST_BSR64_CPB 3
#endif
constexpr int BSR64_CFRONT = JLUST_BSR64_CFRONT;  // window copies issued before the first block's MFMAs
constexpr int BSR64_CPB = JLUST_BSR64_CPB;        // window copies issued before each later block's MFMAs
constexpr int BSR64_CS = BSR64_WMAX * 128 + BSR64_PAD;   // LDS bytes per window column
constexpr int BSR64_BUF = 16 * BSR64_CS;          // the window buffer (156 KB)

__device__ __forceinline__ void raw_store_d4(doublex4 v, int32x4 rs, int voff, int soff)
{
    const bsr_floatx4 *f = reinterpret_cast<const bsr_floatx4 *>(&v);
    raw_buffer_store_v4f32(f[0], rs, voff, soff, 0);
    raw_buffer_store_v4f32(f[1], rs, voff + 16, soff, 0);
}

// Four doubles from two 16-byte LDS pieces 32 bytes apart.
__device__ __forceinline__ doublex4 lds_read_pieces(const char *p)
{
    doublex4 v;
    bsr_floatx4 *f = reinterpret_cast<bsr_floatx4 *>(&v);
    f[0] = *reinterpret_cast<const bsr_floatx4 *>(p);
    f[1] = *reinterpret_cast<const bsr_floatx4 *>(p + 32);
    return v;
}

__device__ __forceinline__ doublex4 raw_load_d4(int32x4 rs, int voff, int soff)
{
    doublex4 v;
    bsr_floatx4 *f = reinterpret_cast<bsr_floatx4 *>(&v);
    f[0] = raw_buffer_load_v4f32(rs, voff, soff, 0);
    f[1] = raw_buffer_load_v4f32(rs, voff + 16, soff, 0);
    return v;
}

template <bool BZ>
__global__ __launch_bounds__(64 * BSR64_SR) __attribute__((amdgpu_waves_per_eu(3)))
void bsr16_spmm_f64_strip_kernel(
    int64_t mb, int32_t origin, const int32_t *__restrict__ browptr,
    const int32_t *__restrict__ bcolind, const double *__restrict__ val, int64_t k, double alpha,
    const double *__restrict__ B, int64_t ldb, double beta, double *__restrict__ C, int64_t ldc)
{
    __shared__ __align__(16) char win[BSR64_BUF];
    // Set-up of a strip, double-buffered by strip parity: per wave its row's
    // first and last window block-row and block count, and the mask of the
    // window block-rows some block of the strip uses.
    __shared__ int32_t s_jmin[2][BSR64_SR], s_jmax[2][BSR64_SR], s_len[2][BSR64_SR];
    __shared__ uint32_t s_used[2][BSR64_SPAN / 32];
    // Persistent workgroups: XCD x = blockIdx % 8 owns strips [lo, hi), a
    // contiguous run, and its G workgroups take lo + w, lo + w + G, ... so
    // the strips in flight on an XCD are neighbours sharing B rows in its L2.
    // A last round of r <= G / 2 strips is cut into f = G / r column ranges
    // each, so that it takes 1 / f of a round.
    const int nstrips = (int)((mb + BSR64_SR - 1) / BSR64_SR);
    const int G = (int)gridDim.x / NUM_XCD;
    const int xcd = (int)blockIdx.x % NUM_XCD;
    const int wl = (int)blockIdx.x / NUM_XCD;
    const int lo = (int)((int64_t)xcd * nstrips / NUM_XCD), hi = (int)((int64_t)(xcd + 1) * nstrips / NUM_XCD);
    if (hi <= lo) return;                  // whole workgroup
    const int kk = (int)k;                      // k < 2^31 - 16 (checked by the host)
    const int ntiles = (kk + 15) / 16;
    const int rounds = (hi - lo + G - 1) / G;
    const int rlast = hi - lo - (rounds - 1) * G;          // strips in the last round, 1..G
    const int fsplit = min(2 * rlast <= G ? G / rlast : 1, ntiles);
    // Work unit it of this workgroup: strip s, tiles [t0, t1).
    auto unit = [&](int it, int &s, int &t0, int &t1) -> bool {
        if (it < rounds - 1) {
            s = lo + wl + it * G;
            t0 = 0;
            t1 = ntiles;
            return true;
        }
        if (it > rounds - 1 || wl >= rlast * fsplit) return false;
        s = lo + (rounds - 1) * G + wl / fsplit;
        const int c = wl % fsplit;
        t0 = c * ntiles / fsplit;
        t1 = (c + 1) * ntiles / fsplit;
        return true;
    };
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int i = lane & 15;
    const int g = lane >> 4;
    const int ar = 4 * (i & 3) + (i >> 2);     // the A row this lane feeds
    const int c_lane = (4 * g + i * (int)ldc) * 8;   // C: this lane's byte offset in a tile
    const int ldb8 = (int)ldb * 8;
    const int pbyte = wave * 1024;
    // A unit of four or more tiles sets up the next unit's strip during its
    // last four tiles; otherwise a strip is set up at its unit's start.
    const doublex4 zero = {0.0, 0.0, 0.0, 0.0};
    // Contraction split: lane (i, g) holds rows kg, kg + 1, kg + 4, kg + 5
    // of the block (kg = 2 (g % 2) + 8 (g / 2)) -- A's columns and B's rows,
    // MFMA u taking the u-th of them -- so it reads two 16-byte pieces of a
    // window row, 32 bytes apart, at byte 8 kg.  With window columns
    // BSR64_CS = 32 mod 512 bytes apart, the 32 lanes of a half-wave then
    // read distinct LDS banks in each 8-byte pass of a ds_read_b128
    // (SQ_LDS_BANK_CONFLICT: 0 cycles per read; 3.7 with rows 4g .. 4g + 3).
    const int kg = 2 * (g & 1) + 8 * (g >> 1);
    const uint32_t col_off = (uint32_t)(i * BSR64_CS + 8 * kg);
    auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
    auto tile_b = [&](int32_t jw, int c0) { return buffer_resource(B + (int64_t)jw * BSR_BS + (int64_t)c0 * ldb); };

    // ---- the strip being computed.
    bool live = false, windowed = false, copier = false, lane_ok = false;
    int q0 = 0, nq = 0, lane_off = 0, so_c = 0;
    int32_t jw0 = 0;
    uint32_t jrel[2] = {0u, 0u};           // window slots of the row's blocks, 8 bits each

    // ---- set-up of a strip in five steps: 1-4 write the *n variables (the
    // strip being set up), 5 adopts them as the strip being computed.
    int Rn = 0;
    bool liven = false;
    int32_t p0n = 0, p1n = 0, bcoln = 0, jw0n = 0;
    int q0n = 0, nqn = 0;
    bool windowedn = false;
    // 1: the row's block range.
    auto setup1 = [&](int sn) {
        Rn = sn * BSR64_SR + wave;
        liven = Rn < mb;
        p0n = liven ? browptr[Rn] : 0;
        p1n = liven ? browptr[Rn + 1] : 0;
    };
    // 2: the row's block columns (one per lane), for rows short enough to
    // be held as operands.
    auto setup2 = [&]() {
        q0n = __builtin_amdgcn_readfirstlane(p0n) - origin;
        const int q1n = __builtin_amdgcn_readfirstlane(p1n) - origin;
        nqn = liven ? q1n - q0n : 0;
        bcoln = 0;
        if (nqn <= BSR_QCHUNK && lane < nqn) bcoln = bcolind[q0n + lane] - origin;
    };
    // 3: per wave the row's column range and length; the used mask cleared.
    auto setup3 = [&](int par) {
        const bool has = nqn <= BSR_QCHUNK && lane < nqn;
        int32_t jmin = has ? bcoln : INT32_MAX, jmax = has ? bcoln : INT32_MIN;
#pragma unroll
        for (int off = 4; off > 0; off >>= 1) {    // the columns sit in lanes 0..7
            jmin = min(jmin, __shfl_xor(jmin, off, 64));
            jmax = max(jmax, __shfl_xor(jmax, off, 64));
        }
        if (lane == 0) {
            s_jmin[par][wave] = jmin;
            s_jmax[par][wave] = jmax;
            s_len[par][wave] = nqn;
        }
        if (threadIdx.x < BSR64_SPAN / 32) s_used[par][threadIdx.x] = 0;
    };
    // 4 (after a barrier): the strip's window; its used block-rows marked.
    auto setup4 = [&](int par) {
        // Lane w < BSR64_SR reads wave w's entries; a 16-lane reduction.
        int32_t jw0 = INT32_MAX, jw1 = INT32_MIN, lmax = 0;
        if (lane < BSR64_SR) {
            jw0 = s_jmin[par][lane];
            jw1 = s_jmax[par][lane];
            lmax = s_len[par][lane];
        }
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            jw0 = min(jw0, __shfl_xor(jw0, off, 64));
            jw1 = max(jw1, __shfl_xor(jw1, off, 64));
            lmax = max(lmax, __shfl_xor(lmax, off, 64));
        }
        jw0 = __builtin_amdgcn_readfirstlane(jw0);
        jw1 = __builtin_amdgcn_readfirstlane(jw1);
        lmax = __builtin_amdgcn_readfirstlane(lmax);
        const int32_t nwin = jw1 >= jw0 ? jw1 - jw0 + 1 : 0;
        jw0n = nwin > 0 ? jw0 : 0;
        windowedn = lmax <= BSR_QCHUNK && nwin <= BSR64_SPAN;
        if (windowedn && lane < nqn) {
            const int32_t r = bcoln - jw0n;
            atomicOr(&s_used[par][r >> 5], 1u << (r & 31));
        }
    };
    // 5 (after a barrier): adopt the strip; its window slots.  Only the used
    // window block-rows (about three quarters of a +-32 band's) are copied,
    // packed in order: slot s of a column is the s-th used row, so no line is
    // fetched for an unused row.  Each block's B rows sit at its row's slot
    // (wave-uniform).  Copies: wave w < npc moves part w -- slots [8 w,
    // 8 w + 8), 1024 bytes -- of every column (npc <= 10 for 76 used rows, one
    // part per wave); lane l moves bytes 16 (l % 8) .. +16 of slot
    // 8 w + l / 8, whose used row it looks up once; lanes past the last slot
    // are masked off.
    auto setup5 = [&](int par) {
        live = liven;
        q0 = q0n;
        nq = nqn;
        jw0 = jw0n;
        so_c = Rn * BSR_BS * 8;            // C: this wave's rows in a tile
        uint32_t used[BSR64_SPAN / 32];
        int nu = 0;
#pragma unroll
        for (int w = 0; w < BSR64_SPAN / 32; ++w) {
            used[w] = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_used[par][w]);
            nu += __builtin_popcount(used[w]);
        }
        windowed = windowedn && nu <= BSR64_WMAX;
        jrel[0] = jrel[1] = 0u;
#pragma unroll
        for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
            uint32_t slot = 0;
            if (qq < nqn) {
                const int32_t r = __builtin_amdgcn_readlane(bcoln, qq) - jw0n;
#pragma unroll
                for (int w = 0; w < BSR64_SPAN / 32; ++w)
                    if (32 * w < r)
                        slot += __builtin_popcount(32 * (w + 1) <= r ? used[w] : used[w] & ((1u << (r & 31)) - 1u));
            }
            jrel[qq >> 2] |= slot << (8 * (qq & 3));
        }
        const int npc = (nu + 7) / 8;
        copier = wave < npc;
        const int my_slot = 8 * wave + (lane >> 3);
        lane_ok = my_slot < nu;
        int my_row = 0, t = my_slot;
#pragma unroll
        for (int w = 0; w < BSR64_SPAN / 32; ++w) {
            const int c = __builtin_popcount(used[w]);
            if (t >= 0 && t < c) {
                uint32_t x = used[w];
                for (int u = 0; u < t; ++u) x &= x - 1u;
                my_row = 32 * w + __builtin_ctz(x);
            }
            t -= c;
        }
        lane_off = my_row * 128 + (lane & 7) * 16;
    };
    auto load_a = [&](doublex4 &dst, int qq) {
        const double *p = val + ((int64_t)q0n + qq) * 256 + ar * 16 + kg;
        bsr_floatx4 *f = reinterpret_cast<bsr_floatx4 *>(&dst);
        f[0] = *reinterpret_cast<const bsr_floatx4 *>(p);
        f[1] = *reinterpret_cast<const bsr_floatx4 *>(p + 4);
    };
    // Column j of the window of the tile at column cb; the copy's LDS
    // address and B offset advance column by column from values made opaque
    // per tile (sd, so), so the compiler keeps two SGPRs, not 32.
    auto copy_col = [&](int32x4 rs, int cb, int j, uint32_t &sd, int &so) {
        if (copier && cb + j < kk && lane_ok)
            raw_buffer_load_lds(rs, (lds_void *)(win + sd), 16, lane_off, so, 0, 0);
        sd += BSR64_CS;
        so += ldb8;
    };

    doublex4 a[BSR_QCHUNK];                // the row's blocks, A operands for all of k
#pragma unroll
    for (int qq = 0; qq < BSR_QCHUNK; ++qq) a[qq] = zero;
    // C of a tile is formed and stored at the next tile's start (possibly
    // the next strip's), after that tile's operand reads: the store needs no
    // wait of its own before them, and the MFMA chain drains while they run.
    // With beta != 0 the old C of a tile is loaded at the tile's start.
    doublex4 accp = zero, oldp = zero;
    int out_c0 = -1;
    int out_so = 0;
    bool out_live = false;
    auto flush = [&]() {
        if (out_live && out_c0 >= 0 && out_c0 + i < kk) {
            doublex4 out = alpha * accp;
            if (!BZ) out += beta * oldp;
            raw_store_d4(out, buffer_resource(C + (int64_t)out_c0 * ldc), c_lane, out_so);
        }
        out_c0 = -1;
    };

    // ready: steps 1-4 and the A operand loads of strip s were done during
    // the previous strip's tiles (step 4 in its last tile, before its final
    // barrier).
    bool ready = false;
    int par = 0;
    int s = 0, t0 = 0, t1 = 0, sn = 0, t0n = 0, t1n = 0;
    bool has = unit(0, s, t0, t1), hasn = false;
    for (int it = 0; has; ++it, par ^= 1, has = hasn, s = sn, t0 = t0n, t1 = t1n) {
        hasn = unit(it + 1, sn, t0n, t1n);
        const bool pre = hasn && t1 - t0 >= 4;  // steps 1-4 of strip sn run during this unit's tiles
        if (!ready) {
            setup1(s);
            setup2();
            setup3(par);
            barrier();
            setup4(par);
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq)
                if (liven && qq < nqn) load_a(a[qq], qq);
            barrier();
        }
        setup5(par);
        ready = false;

        if (!windowed) {
            // Direct operand loads (any row length, any window).
            flush();
            if (live) {
                for (int64_t c0 = (int64_t)t0 * 16; c0 < k && c0 < (int64_t)t1 * 16; c0 += 16) {
                    const int64_t colc = c0 + i < k ? c0 + i : k - 1;
                    doublex4 acc = zero;
                    for (int64_t q = q0; q < (int64_t)q0 + nq; ++q) {
                        const doublex4 av = *reinterpret_cast<const doublex4 *>(val + q * 256 + ar * 16 + 4 * g);
                        const int64_t brow = ((int64_t)bcolind[q] - origin) * BSR_BS + 4 * g;
                        const doublex4 bv = *reinterpret_cast<const doublex4 *>(B + brow + colc * ldb);
#pragma unroll
                        for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av[u], bv[u], acc, 0, 0, 0);
                    }
                    if (c0 + i < k) {
                        double *dst = C + (int64_t)Rn * BSR_BS + 4 * g + (c0 + i) * ldc;
                        doublex4 out = alpha * acc;
                        if (!BZ) out += beta * *reinterpret_cast<const doublex4 *>(dst);
                        *reinterpret_cast<doublex4 *>(dst) = out;
                    }
                }
            }
            __builtin_amdgcn_s_waitcnt(0);
            asm volatile("s_barrier" ::: "memory");   // every wave is past step 5's reads
            continue;
        }
        {
            const int32x4 rs0 = tile_b(jw0, t0 * 16);
            uint32_t sd = pbyte;
            int so = 0;
            for (int j = 0; j < 16; ++j) copy_col(rs0, t0 * 16, j, sd, so);
        }
        __builtin_amdgcn_s_waitcnt(0);
        asm volatile("s_barrier" ::: "memory");

        for (int t = t0; t < t1; ++t) {
            const int c0 = t * 16;
            const bool last = t == t1 - 1;
            // Nothing is in flight here (the previous tile or the strip's start
            // waited for everything); said explicitly, so that the compiler
            // adds no waits of its own before this tile's MFMAs for the next
            // strip's A loads of a last tile.
            __builtin_amdgcn_s_waitcnt(0);
            doublex4 b[BSR_QCHUNK];
            uint32_t co = col_off, jr0 = jrel[0], jr1 = jrel[1];
            asm volatile("" : "+v"(co), "+s"(jr0), "+s"(jr1));
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq)
                b[qq] = lds_read_pieces(win + co + (((qq < 4 ? jr0 : jr1) >> (8 * (qq & 3))) & 0xffu) * 128);
            barrier();                     // the window is free
            flush();
            if (!BZ && live && c0 + i < kk) oldp = raw_load_d4(buffer_resource(C + (int64_t)c0 * ldc), c_lane, so_c);
            if (pre && t == t1 - 4) setup1(sn);
            if (pre && t == t1 - 3) setup2();
            if (pre && last) setup4(par ^ 1);
            asm volatile("" ::: "memory");
            // The 16 copies of the next tile: BSR64_CFRONT before the first
            // block's MFMAs, then BSR64_CPB before each later block's.  In
            // the last tile the next strip's A operands are loaded instead,
            // each after its block's MFMAs have read this strip's.
            const bool more = !last;
            const int32x4 rsn = tile_b(jw0, more ? c0 + 16 : c0);
            const bool nxa = last && pre && liven;
            doublex4 acc = zero;
            int jn = 0;
            uint32_t sd = pbyte;
            int so = 0;
            asm volatile("" : "+s"(sd), "+s"(so));
            if (more) {
#pragma unroll
                for (int c = 0; c < BSR64_CFRONT; ++c) copy_col(rsn, c0 + 16, jn++, sd, so);
            }
#pragma unroll
            for (int qq = 0; qq < BSR_QCHUNK; ++qq) {
                if (more && qq > 0) {
#pragma unroll
                    for (int c = 0; c < BSR64_CPB; ++c)
                        if (jn < 16) copy_col(rsn, c0 + 16, jn++, sd, so);
                }
                asm volatile("" ::: "memory");
                if (live && qq < nq) {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(a[qq][u], b[qq][u], acc, 0, 0, 0);
                }
                if (nxa && qq < nqn) load_a(a[qq], qq);
            }
            if (more)
                while (jn < 16) copy_col(rsn, c0 + 16, jn++, sd, so);
            if (pre && t == t1 - 2) setup3(par ^ 1);
            accp = acc;
            out_c0 = c0;
            out_so = so_c;
            out_live = live;
            if (last) {
                // No window copies are in flight: the next strip's A operand
                // loads stay in flight into its first window's copies.
                barrier();
            } else {
                __builtin_amdgcn_s_waitcnt(0);
                asm volatile("s_barrier" ::: "memory");
            }
        }
        ready = pre;
    }
    flush();
    __builtin_amdgcn_s_waitcnt(0);
}

// JLUST_HIP_BSR_STRIP=0 keeps the row-wave kernel (read at each call, so a
// test can run both kernels in one process; the row-wave kernel is also the
// one for B or C whose byte offsets reach 2^31).
bool bsr_strip()
{
    const char *e = getenv("JLUST_HIP_BSR_STRIP");
    return !(e && e[0] == '0');
}

// 16x16 fp32 BSR SpMM with 24-row strips: JLUST_HIP_BSR_WIDE=1 always,
// =0 never (the 12-row kernel), unset when the rows hold 6 or more blocks
// on average -- the 24-row kernel runs all 8 block slots of every row, so
// on shorter rows it spends MFMAs on zeros.  Read at each call, so a test
// can run both kernels in one process.
bool bsr_wide(int64_t mb, int64_t nnzb)
{
    const char *e = getenv("JLUST_HIP_BSR_WIDE");
    if (e && e[0] == '1') return true;
    if (e && e[0] == '0') return false;
    return nnzb >= 6 * mb;
}

// JLUST_HIP_BSR_SPMV_SEGMENTS=0 keeps BSR SpMV on the one-thread-per-row
// kernel (read at each call, for tests and timing beside it).
bool bsr_spmv_segmented()
{
    const char *e = getenv("JLUST_HIP_BSR_SPMV_SEGMENTS");
    return !(e && e[0] == '0');
}

// ------------------------------------------------------------- BSR SpMV

// y = alpha*A*x + beta*y for BSR of any b1 x b2 blocks: one thread per
// scalar row 16R + r walks the blocks of its block-row in storage order and
// each block's row r in column order -- the order of the row's entries in the
// CSR expansion, so the sum is the expanded CSR row's.  x[16 bcol + s] is the
// same for every thread of a block-row (one broadcast load per wave).  Block
// ranges are clamped into [0, nnzb) and block columns into [0, nb), so a
// malformed browptr or bcolind cannot take a read out of bounds.
template <typename T, bool ROW_MAJOR, bool BZ>
__global__ __launch_bounds__(256) void bsr_spmv_kernel(int64_t mb, int64_t nb, int64_t b1, int64_t b2,
                                                      int64_t nnzb, int32_t origin,
                                                      const int32_t *__restrict__ browptr,
                                                      const int32_t *__restrict__ bcolind,
                                                      const T *__restrict__ val, T alpha,
                                                      const T *__restrict__ x, T beta, T *__restrict__ y)
{
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= mb * b1) return;
    const int64_t R = row / b1, r = row % b1, bb = b1 * b2;
    const int64_t q0 = min(max((int64_t)browptr[R] - origin, (int64_t)0), nnzb);
    const int64_t q1 = min(max((int64_t)browptr[R + 1] - origin, q0), nnzb);
    T acc = T(0);
    for (int64_t q = q0; q < q1; ++q) {
        const int64_t c = min(max((int64_t)bcolind[q] - origin, (int64_t)0), nb - 1) * b2;
        const T *v = val + q * bb + (ROW_MAJOR ? r * b2 : r);
        for (int64_t s = 0; s < b2; ++s) acc += v[ROW_MAJOR ? s : s * b1] * x[c + s];
    }
    y[row] = BZ ? alpha * acc : alpha * acc + beta * y[row];
}

// 16 x 16 blocks: segments of at most BSRMV_SEG blocks of one block-row, a
// wave each, so that a long block-row is spread over many waves and a short
// one costs one wave (one thread per scalar row leaves a power-law row
// pattern to its longest row: 12 ms for what the segments do in 0.2 ms).
// A block-row of n blocks has max(1, ceil(n / BSRMV_SEG)) segments (an empty
// one is a segment of no blocks, which writes beta*y).  Each lane holds a
// partial sum of one scalar row over 4 of the block's 16 columns, blocks in
// storage order; the 4 partials combine in a fixed order; a block-row of one
// segment writes y, one of several writes each segment's 16 sums to part[],
// and a second kernel adds them in segment order.  The result is the same
// on every call; its summation order differs from the CSR expansion's.
constexpr int BSRMV_SEG = 32;              // blocks per segment
#ifndef JLUST_BSRMV_UNROLL
#define JLUST_BSRMV_UNROLL 8
#endif
constexpr int BSRMV_UNROLL = JLUST_BSRMV_UNROLL;

// Segment counts: segstart[R] = max(1, ceil(n_R / BSRMV_SEG)) for R < mb and
// segstart[mb] = 0; an exclusive scan then makes segstart[R] the first
// segment of block-row R and segstart[mb] the count.  Block ranges are
// clamped as in bsr_spmv_kernel.
__global__ __launch_bounds__(256) void bsr16_spmv_count_kernel(int64_t mb, int64_t nnzb, int32_t origin,
                                                               const int32_t *__restrict__ browptr,
                                                               int32_t *__restrict__ segstart)
{
    const int64_t R = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (R > mb) return;
    if (R == mb) {
        segstart[mb] = 0;
        return;
    }
    const int64_t q0 = min(max((int64_t)browptr[R] - origin, (int64_t)0), nnzb);
    const int64_t q1 = min(max((int64_t)browptr[R + 1] - origin, q0), nnzb);
    segstart[R] = (int32_t)max((int64_t)1, (q1 - q0 + BSRMV_SEG - 1) / BSRMV_SEG);
}

// segrow[s] = the block-row of segment s, one thread per block-row.  Segment
// numbers are clamped to [0, nsegmax) (a canonical browptr has at most
// nsegmax segments), and every reader clamps what it reads, so a malformed
// browptr cannot take an access out of bounds.
__global__ __launch_bounds__(256) void bsr16_spmv_rows_kernel(int64_t mb, const int32_t *__restrict__ segstart,
                                                              int32_t *__restrict__ segrow, int64_t nsegmax)
{
    const int64_t R = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (R >= mb) return;
    const int64_t s0 = min(max((int64_t)segstart[R], (int64_t)0), nsegmax);
    const int64_t s1 = min(max((int64_t)segstart[R + 1], s0), nsegmax);
    for (int64_t s = s0; s < s1; ++s) segrow[s] = (int32_t)R;
}

template <typename T, bool RM, bool VEC, bool BZ>
__global__ __launch_bounds__(256) void bsr16_spmv_seg_kernel(int64_t mb, int64_t nb, int64_t nnzb, int32_t origin,
                                                             const int32_t *__restrict__ browptr,
                                                             const int32_t *__restrict__ bcolind,
                                                             const T *__restrict__ val, T alpha,
                                                             const T *__restrict__ x, T beta, T *__restrict__ y,
                                                             const int32_t *__restrict__ segstart,
                                                             const int32_t *__restrict__ segrow,
                                                             T *__restrict__ part, int64_t nsegmax)
{
    const int64_t sg_id = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (sg_id >= nsegmax || sg_id >= (int64_t)segstart[mb]) return;   // whole waves
    const int lane = threadIdx.x & 63;
    // Row-major blocks: lane (r, c4) = (lane / 4, lane % 4), 16 contiguous
    // bytes of row r; column-major: (lane % 16, lane / 16), one element of
    // each of 4 columns (16 lanes read 64 contiguous bytes).
    const int r = RM ? lane >> 2 : lane & 15;
    const int c4 = RM ? lane & 3 : lane >> 4;
    const int64_t R = min(max((int64_t)segrow[sg_id], (int64_t)0), mb - 1);
    const int64_t k = sg_id - segstart[R];
    const int64_t nsR = (int64_t)segstart[R + 1] - segstart[R];
    const int64_t rb = min(max((int64_t)browptr[R] - origin, (int64_t)0), nnzb);
    const int64_t re = min(max((int64_t)browptr[R + 1] - origin, rb), nnzb);
    const int64_t q0 = min(max(rb + k * BSRMV_SEG, rb), re), q1 = min(q0 + BSRMV_SEG, re);
    // Blocks in groups of BSRMV_UNROLL: the group's column indices, then its
    // value and x loads, then the products in storage order, so that a
    // wave keeps that many blocks' loads in flight.
    T acc = T(0);
    auto load = [&](int64_t q, T (&vv)[4], T (&xx)[4]) {
        const int64_t c = min(max((int64_t)bcolind[q] - origin, (int64_t)0), nb - 1) * 16 + 4 * c4;
        const T *v = val + q * 256;
        if (RM && VEC) {
            typedef T T2 __attribute__((ext_vector_type(2)));
            const T *vr = v + r * 16 + 4 * c4;
            const T2 v0 = *reinterpret_cast<const T2 *>(vr), v1 = *reinterpret_cast<const T2 *>(vr + 2);
            const T2 x0 = *reinterpret_cast<const T2 *>(x + c), x1 = *reinterpret_cast<const T2 *>(x + c + 2);
            vv[0] = v0.x; vv[1] = v0.y; vv[2] = v1.x; vv[3] = v1.y;
            xx[0] = x0.x; xx[1] = x0.y; xx[2] = x1.x; xx[3] = x1.y;
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                vv[u] = RM ? v[r * 16 + 4 * c4 + u] : v[(4 * c4 + u) * 16 + r];
                xx[u] = x[c + u];
            }
        }
    };
    int64_t q = q0;
    for (; q + BSRMV_UNROLL <= q1; q += BSRMV_UNROLL) {
        T vv[BSRMV_UNROLL][4], xx[BSRMV_UNROLL][4];
#pragma unroll
        for (int b = 0; b < BSRMV_UNROLL; ++b) load(q + b, vv[b], xx[b]);
#pragma unroll
        for (int b = 0; b < BSRMV_UNROLL; ++b)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc += vv[b][u] * xx[b][u];
    }
    for (; q < q1; ++q) {
        T vv[4], xx[4];
        load(q, vv, xx);
#pragma unroll
        for (int u = 0; u < 4; ++u) acc += vv[u] * xx[u];
    }
    // The 4 column groups of a row, in the order (0 + 1) + (2 + 3).
    const int m1 = RM ? 1 : 16, m2 = RM ? 2 : 32;
    acc += __shfl_xor(acc, m1, 64);
    acc += __shfl_xor(acc, m2, 64);
    if (c4 != 0) return;
    if (nsR == 1) {
        T *yr = y + R * 16 + r;
        *yr = BZ ? alpha * acc : alpha * acc + beta * *yr;
    } else {
        part[sg_id * 16 + r] = acc;
    }
}

// Blocks of any other shape: a thread per (segment, scalar row), blocks in
// storage order and each block's row in column order, as bsr_spmv_kernel
// (a block-row of one segment gets that kernel's sum).
template <typename T, bool RM, bool BZ>
__global__ __launch_bounds__(256) void bsr_spmv_seg_kernel(int64_t mb, int64_t nb, int64_t b1, int64_t b2,
                                                           int64_t nnzb, int32_t origin,
                                                           const int32_t *__restrict__ browptr,
                                                           const int32_t *__restrict__ bcolind,
                                                           const T *__restrict__ val, T alpha,
                                                           const T *__restrict__ x, T beta, T *__restrict__ y,
                                                           const int32_t *__restrict__ segstart,
                                                           const int32_t *__restrict__ segrow,
                                                           T *__restrict__ part, int64_t nsegmax)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t sg_id = t / b1, r = t % b1;
    if (sg_id >= nsegmax || sg_id >= (int64_t)segstart[mb]) return;
    const int64_t R = min(max((int64_t)segrow[sg_id], (int64_t)0), mb - 1);
    const int64_t k = sg_id - segstart[R];
    const int64_t nsR = (int64_t)segstart[R + 1] - segstart[R];
    const int64_t rb = min(max((int64_t)browptr[R] - origin, (int64_t)0), nnzb);
    const int64_t re = min(max((int64_t)browptr[R + 1] - origin, rb), nnzb);
    const int64_t q0 = min(max(rb + k * BSRMV_SEG, rb), re), q1 = min(q0 + BSRMV_SEG, re);
    const int64_t bb = b1 * b2;
    T acc = T(0);
    for (int64_t q = q0; q < q1; ++q) {
        const int64_t c = min(max((int64_t)bcolind[q] - origin, (int64_t)0), nb - 1) * b2;
        const T *v = val + q * bb + (RM ? r * b2 : r);
        for (int64_t s = 0; s < b2; ++s) acc += v[RM ? s : s * b1] * x[c + s];
    }
    if (nsR == 1) {
        T *yr = y + R * b1 + r;
        *yr = BZ ? alpha * acc : alpha * acc + beta * *yr;
    } else {
        part[sg_id * b1 + r] = acc;
    }
}

// y of the block-rows of several segments: their sums added in segment order.
template <typename T, bool BZ>
__global__ __launch_bounds__(256) void bsr_spmv_fix_kernel(int64_t mb, int64_t b1,
                                                           const int32_t *__restrict__ segstart,
                                                           const T *__restrict__ part, int64_t nsegmax,
                                                           T alpha, T beta, T *__restrict__ y)
{
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= mb * b1) return;
    const int64_t R = row / b1, r = row % b1;
    const int64_t s0 = segstart[R], s1 = segstart[R + 1];
    if (s1 - s0 <= 1 || s0 < 0 || s1 > nsegmax) return;
    // Eight partial sums loaded at a time, added in segment order.
    T acc = T(0);
    int64_t s = s0;
    for (; s + 8 <= s1; s += 8) {
        T p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) p[u] = part[(s + u) * b1 + r];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += p[u];
    }
    for (; s < s1; ++s) acc += part[s * b1 + r];
    y[row] = BZ ? alpha * acc : alpha * acc + beta * y[row];
}

// Segments of at most BSRMV_SEG blocks (a block-row of L blocks is ceil(L /
// BSRMV_SEG) of them, an empty one still one): nsegmax bounds their count.
int64_t bsr_spmv_nsegmax(int64_t mb, int64_t nnzb) { return mb + (nnzb + BSRMV_SEG - 1) / BSRMV_SEG; }

// The segment table: segstart (mb + 1, the first segment of each block-row)
// and segrow (nsegmax, the block-row of each segment).
int bsr_spmv_table(int64_t mb, int64_t nnzb, int32_t origin, const int32_t *browptr, int32_t *segstart,
                   int32_t *segrow, int64_t nsegmax, jlust_stream_t stream)
{
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(bsr16_spmv_count_kernel, dim3((unsigned)((mb + 1 + 255) / 256)), dim3(256), 0, s, mb, nnzb,
                       origin, browptr, segstart);
    if (int st = check_launch("bsr16_spmv_count_kernel")) return st;
    if (int st = exclusive_scan_i32(segstart, segstart, mb + 1, stream)) return st;
    hipLaunchKernelGGL(bsr16_spmv_rows_kernel, dim3((unsigned)((mb + 255) / 256)), dim3(256), 0, s, mb, segstart,
                       segrow, nsegmax);
    return check_launch("bsr16_spmv_rows_kernel");
}

// The product over a segment table: per-segment partial sums (part, nsegmax
// x b1), then each block-row's sum of its segments into y.
template <typename T>
int bsr_spmv_run(int64_t mb, int64_t nb, int64_t b1, int64_t b2, int64_t nnzb, int32_t origin,
                 const int32_t *browptr, const int32_t *bcolind, const T *val, int row_major_blocks, T alpha,
                 const T *x, T beta, T *y, const int32_t *segstart, const int32_t *segrow, T *part, int64_t nsegmax,
                 jlust_stream_t stream)
{
    hipStream_t s = (hipStream_t)stream;
    const bool bz = beta == T(0);
    if (b1 != 16 || b2 != 16) {
        const dim3 g((unsigned)((nsegmax * b1 + 255) / 256));
#define JLUST_BSRMVG(RM, Z)                                                                              \
        hipLaunchKernelGGL((bsr_spmv_seg_kernel<T, RM, Z>), g, dim3(256), 0, s, mb, nb, b1, b2, nnzb, origin, \
                           browptr, bcolind, val, alpha, x, beta, y, segstart, segrow, part, nsegmax)
        if (row_major_blocks) {
            if (bz) JLUST_BSRMVG(true, true); else JLUST_BSRMVG(true, false);
        } else {
            if (bz) JLUST_BSRMVG(false, true); else JLUST_BSRMVG(false, false);
        }
#undef JLUST_BSRMVG
        if (int st = check_launch("bsr_spmv_seg_kernel")) return st;
    } else {
        const bool vec = ((uintptr_t)val % (2 * sizeof(T)) == 0) && ((uintptr_t)x % (2 * sizeof(T)) == 0);
        const dim3 grid((unsigned)((nsegmax + 3) / 4));
#define JLUST_BSRMV16(RM, V, Z)                                                                             \
        hipLaunchKernelGGL((bsr16_spmv_seg_kernel<T, RM, V, Z>), grid, dim3(256), 0, s, mb, nb, nnzb, origin,  \
                           browptr, bcolind, val, alpha, x, beta, y, segstart, segrow, part, nsegmax)
        if (row_major_blocks) {
            if (vec) {
                if (bz) JLUST_BSRMV16(true, true, true); else JLUST_BSRMV16(true, true, false);
            } else {
                if (bz) JLUST_BSRMV16(true, false, true); else JLUST_BSRMV16(true, false, false);
            }
        } else {
            if (bz) JLUST_BSRMV16(false, false, true); else JLUST_BSRMV16(false, false, false);
        }
#undef JLUST_BSRMV16
        if (int st = check_launch("bsr16_spmv_seg_kernel")) return st;
    }
    const dim3 gfix((unsigned)((mb * b1 + 255) / 256));
    if (bz)
        hipLaunchKernelGGL((bsr_spmv_fix_kernel<T, true>), gfix, dim3(256), 0, s, mb, b1, segstart, part, nsegmax,
                           alpha, beta, y);
    else
        hipLaunchKernelGGL((bsr_spmv_fix_kernel<T, false>), gfix, dim3(256), 0, s, mb, b1, segstart, part, nsegmax,
                           alpha, beta, y);
    return check_launch("bsr_spmv_fix_kernel");
}

template <typename T>
int bsr_spmv_segments(int64_t mb, int64_t nb, int64_t b1, int64_t b2, int64_t nnzb, int32_t origin,
                      const int32_t *browptr, const int32_t *bcolind, const T *val, int row_major_blocks, T alpha,
                      const T *x, T beta, T *y, jlust_stream_t stream)
{
    // Scratch: the scan's own part, then segstart (mb + 1), segrow (nsegmax),
    // part (b1 sums per segment).
    const int64_t nsegmax = bsr_spmv_nsegmax(mb, nnzb);
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t start_off = up(exclusive_scan_scratch_bytes(mb + 1));
    const size_t row_off = start_off + up((size_t)(mb + 1) * sizeof(int32_t));
    const size_t part_off = row_off + up((size_t)nsegmax * sizeof(int32_t));
    void *ws = nullptr;
    if (int st = scratch(stream, part_off + (size_t)(nsegmax * b1) * sizeof(T), &ws)) return st;
    int32_t *segstart = (int32_t *)((char *)ws + start_off), *segrow = (int32_t *)((char *)ws + row_off);
    T *part = (T *)((char *)ws + part_off);
    if (int st = bsr_spmv_table(mb, nnzb, origin, browptr, segstart, segrow, nsegmax, stream)) return st;
    return bsr_spmv_run<T>(mb, nb, b1, b2, nnzb, origin, browptr, bcolind, val, row_major_blocks, alpha, x, beta, y,
                           segstart, segrow, part, nsegmax, stream);
}

template <typename T>
int bsr_spmv(int64_t mb, int64_t nb, int64_t b1, int64_t b2, int64_t nnzb, int32_t origin,
             const int32_t *browptr, const int32_t *bcolind, const T *val, int row_major_blocks, T alpha,
             const T *x, T beta, T *y, jlust_stream_t stream)
{
    clear_error();
    if (mb < 0 || nb < 0 || b1 <= 0 || b2 <= 0 || nnzb < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv: negative extent or block size");
    if (mb * b1 > INT32_MAX || nb * b2 > INT32_MAX || nnzb * b1 * b2 > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv: extents exceed the Int32 index range");
    if (int st = check_origin(origin)) return st;
    if ((mb > 0 && !browptr) || bad_ptr(bcolind, nnzb) || bad_ptr(val, nnzb * b1 * b2) ||
        (nnzb > 0 && !x) || bad_ptr(y, mb * b1))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv: null device pointer");
    if (nnzb > 0 && nb == 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv: blocks stored in a matrix with no columns");
    if (int st = require_device(nullptr)) return st;
    const int64_t m = mb * b1;
    if (m == 0) return JLUST_STATUS_SUCCESS;
    if (bsr_spmv_segmented())
        return bsr_spmv_segments<T>(mb, nb, b1, b2, nnzb, origin, browptr, bcolind, val, row_major_blocks, alpha, x,
                                    beta, y, stream);
    const dim3 grid((unsigned)((m + 255) / 256));
    hipStream_t s = (hipStream_t)stream;
#define JLUST_BSRMV(RM, Z)                                                                             \
    hipLaunchKernelGGL((bsr_spmv_kernel<T, RM, Z>), grid, dim3(256), 0, s, mb, nb, b1, b2, nnzb, origin, \
                       browptr, bcolind, val, alpha, x, beta, y)
    const bool bz = beta == T(0);
    if (row_major_blocks) {
        if (bz) JLUST_BSRMV(true, true); else JLUST_BSRMV(true, false);
    } else {
        if (bz) JLUST_BSRMV(false, true); else JLUST_BSRMV(false, false);
    }
#undef JLUST_BSRMV
    return check_launch("bsr_spmv_kernel");
}

// ------------------------------------------------- expansion to CSR

// rowptr of the expansion: scalar row b1*R + r starts after the entries of
// block-rows 0..R-1 (b1*b2 per block) and r rows of block-row R (its block
// count times b2 each).  One thread per scalar row, plus the final entry.
__global__ void bsr_expand_rowptr_kernel(int64_t mb, int64_t b1, int64_t b2, int32_t origin,
                                         const int32_t *__restrict__ browptr, int32_t *__restrict__ rowptr)
{
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row > mb * b1) return;
    const int64_t R = row / b1, r = row % b1;
    int64_t v;
    if (R == mb) {
        v = ((int64_t)browptr[mb] - origin) * b1 * b2;
    } else {
        const int64_t q0 = (int64_t)browptr[R] - origin, q1 = (int64_t)browptr[R + 1] - origin;
        v = q0 * b1 * b2 + r * (q1 - q0) * b2;
    }
    rowptr[row] = (int32_t)(v + origin);
}

// Columns and values (values only when colind is null): one thread per
// stored block entry (q, r, s).  The
// block-row of block q is found by binary search of browptr; an entry whose
// target position falls outside [0, total) -- possible only for a browptr
// that is not non-decreasing -- is not written.
template <typename T>
__global__ void bsr_expand_entries_kernel(int64_t mb, int64_t b1, int64_t b2, int64_t nnzb, int32_t origin,
                                          const int32_t *__restrict__ browptr,
                                          const int32_t *__restrict__ bcolind, const T *__restrict__ val,
                                          int row_major_blocks, int32_t *__restrict__ colind,
                                          T *__restrict__ out)
{
    const int64_t bb = b1 * b2, total = nnzb * bb;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t q = e / bb, w = e % bb;
        const int64_t r = w / b2, s = w % b2;           // the entry's row and column in its block
        int64_t lo = 0, hi = mb - 1;                    // last R with browptr[R] - origin <= q
        while (lo < hi) {
            const int64_t mid = (lo + hi + 1) >> 1;
            if ((int64_t)browptr[mid] - origin <= q) lo = mid; else hi = mid - 1;
        }
        const int64_t q0 = (int64_t)browptr[lo] - origin, q1 = (int64_t)browptr[lo + 1] - origin;
        if (q < q0 || q >= q1) continue;
        const int64_t pos = q0 * bb + r * (q1 - q0) * b2 + (q - q0) * b2 + s;
        if (pos < 0 || pos >= total) continue;
        if (colind) colind[pos] = (int32_t)(((int64_t)bcolind[q] - origin) * b2 + s + origin);
        out[pos] = row_major_blocks ? val[q * bb + r * b2 + s] : val[q * bb + s * b1 + r];
    }
}

int bsr_expand_entries(int64_t mb, int64_t b1, int64_t b2, int64_t nnzb, int32_t origin, const int32_t *browptr,
                       const int32_t *bcolind, const void *val, int value_type, int row_major_blocks,
                       int32_t *colind, void *val_out, hipStream_t s)
{
    const int64_t total = nnzb * b1 * b2;
    if (total == 0) return JLUST_STATUS_SUCCESS;
    const int64_t blocks = min((total + 255) / 256, (int64_t)65536);
    if (value_type == 0)
        hipLaunchKernelGGL((bsr_expand_entries_kernel<double>), dim3((unsigned)blocks), dim3(256), 0, s, mb, b1,
                           b2, nnzb, origin, browptr, bcolind, (const double *)val, row_major_blocks, colind,
                           (double *)val_out);
    else
        hipLaunchKernelGGL((bsr_expand_entries_kernel<float>), dim3((unsigned)blocks), dim3(256), 0, s, mb, b1,
                           b2, nnzb, origin, browptr, bcolind, (const float *)val, row_major_blocks, colind,
                           (float *)val_out);
    return check_launch("bsr_expand_entries_kernel");
}

int bsr_expand_csr(int64_t mb, int64_t b1, int64_t b2, int64_t nnzb, int32_t origin, const int32_t *browptr,
                   const int32_t *bcolind, const void *val, int value_type, int row_major_blocks,
                   int32_t *rowptr, int32_t *colind, void *val_out, jlust_stream_t stream)
{
    clear_error();
    if (mb < 0 || b1 <= 0 || b2 <= 0 || nnzb < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_expand_csr: negative extent or block size");
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE,
                    "bsr_expand_csr: value_type %d (0 = Float64, 1 = Float32)", value_type);
    if (int st = check_origin(origin)) return st;
    if (mb * b1 >= INT32_MAX || nnzb * b1 * b2 >= (int64_t)INT32_MAX - 1)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_expand_csr: the expansion exceeds the Int32 index range");
    const int64_t total = nnzb * b1 * b2;
    if (!browptr || !rowptr || bad_ptr(bcolind, nnzb) || bad_ptr(val, total) || bad_ptr(colind, total) ||
        bad_ptr(val_out, total))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_expand_csr: null device pointer");
    if (int st = require_device(nullptr)) return st;
    hipStream_t s = (hipStream_t)stream;
    // browptr must run from origin to origin + nnzb (two scalars read back).
    int32_t ends[2] = {0, 0};
    JLUST_HIP_TRY(hipMemcpyAsync(&ends[0], browptr, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    JLUST_HIP_TRY(hipMemcpyAsync(&ends[1], browptr + mb, sizeof(int32_t), hipMemcpyDeviceToHost, s));
    JLUST_HIP_TRY(hipStreamSynchronize(s));
    if (ends[0] != origin || (int64_t)ends[1] != nnzb + origin)
        return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                    "bsr_expand_csr: browptr runs from %d to %d, expected %d to %lld", ends[0], ends[1], origin,
                    (long long)(nnzb + origin));
    const int64_t rows = mb * b1 + 1;
    hipLaunchKernelGGL(bsr_expand_rowptr_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, mb, b1,
                       b2, origin, browptr, rowptr);
    if (int st = check_launch("bsr_expand_rowptr_kernel")) return st;
    return bsr_expand_entries(mb, b1, b2, nnzb, origin, browptr, bcolind, val, value_type, row_major_blocks,
                              colind, val_out, s);
}

int bsr_spmm(int64_t mb, int64_t nb, int64_t bs, int64_t nnzb, int32_t origin,
             const int32_t *browptr, const int32_t *bcolind, const float *val,
             int row_major_blocks, int64_t k, float alpha, const float *B, int64_t ldb,
             float beta, float *C, int64_t ldc, jlust_stream_t stream)
{
    clear_error();
    if (mb < 0 || nb < 0 || bs <= 0 || nnzb < 0 || k < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm: negative extent or block size");
    if (bs != BSR_BS)
        return fail(JLUST_STATUS_UNSUPPORTED_FORMAT,
                    "bsr_spmm: block size %lld x %lld (the MFMA path supports 16 x 16)",
                    (long long)bs, (long long)bs);
    if (mb * bs > INT32_MAX || nb * bs > INT32_MAX || nnzb > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm: extents exceed the Int32 index range");
    if (int st = check_origin(origin)) return st;
    const int64_t mrows = mb * bs, nrows = nb * bs;
    if (ldb < (nrows > 0 ? nrows : 1) || ldc < (mrows > 0 ? mrows : 1))
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "bsr_spmm: leading dimensions too small (ldb=%lld < %lld or ldc=%lld < %lld)",
                    (long long)ldb, (long long)nrows, (long long)ldc, (long long)mrows);
    if ((mb > 0 && !browptr) || bad_ptr(bcolind, nnzb) || bad_ptr(val, nnzb) ||
        bad_ptr(B, (nnzb > 0 && k > 0) ? nrows : 0) || bad_ptr(C, mrows * k))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (mb == 0 || k == 0) return JLUST_STATUS_SUCCESS;

    const bool vec = (ldb % 4 == 0) && (ldc % 4 == 0) && ((uintptr_t)B % 16 == 0) &&
                     ((uintptr_t)C % 16 == 0);
    const bool vals_aligned = ((uintptr_t)val % 16 == 0);
    const int64_t grid = (mb + NUM_XCD - 1) / NUM_XCD * NUM_XCD;
    hipStream_t s = (hipStream_t)stream;
    const int bz = beta == 0.f;
#define JLUST_BSR_LAUNCH(RM, V)                                                                   \
    hipLaunchKernelGGL((bsr16_spmm_mfma_kernel<RM, V>), dim3((unsigned)grid), dim3(64 * BSR_WAVES), \
                       0, s, mb, origin, browptr, bcolind, val, k, alpha, B, ldb, beta, bz, C, ldc)
    const bool rm = row_major_blocks && vals_aligned;
    if (row_major_blocks && !vals_aligned)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm: block values must be 16-byte aligned");
    // The strip kernel addresses B and C through 32-bit buffer offsets.
    const bool offsets_fit = ((uint64_t)(nrows + k * ldb) + 2048) * 4 < ((uint64_t)1 << 31) &&
                             ((uint64_t)(mrows + (k + 16) * ldc)) * 4 < ((uint64_t)1 << 31);
    if (rm && vec && offsets_fit && k < INT32_MAX - 16 && bsr_strip() && bsr_wide(mb, nnzb)) {
        // One resident workgroup per CU (the window takes most of its LDS),
        // each walking its XCD's strips.
        int dev = 0;
        if (int st = require_device(&dev)) return st;
        const int64_t strips = (mb + BSRW_SR - 1) / BSRW_SR;
        const int64_t per_xcd = std::max<int64_t>(1, device_info(dev).cu_count / NUM_XCD);
        const int64_t grids = std::min((strips + NUM_XCD - 1) / NUM_XCD, per_xcd) * NUM_XCD;
        // Rows of more than 8 blocks on average: the long-row kernel, which
        // also runs strips of 9 to 16 blocks a row in registers (two halves
        // of 12 rows); the 24-row kernel leaves such strips to the direct
        // operand loads.
#define JLUST_BSRW_LAUNCH(KERNEL)                                                                        \
        hipLaunchKernelGGL(KERNEL, dim3((unsigned)grids), dim3(64 * BSRW_WAVES), 0, s, mb, origin, browptr, \
                           bcolind, val, k, alpha, B, ldb, beta, C, ldc)
        const bool lg = nnzb > (int64_t)BSR_QCHUNK * mb;
        if (beta == 0.f) {
            if (lg) JLUST_BSRW_LAUNCH(bsr16_spmm_wide_long_kernel<true>);
            else JLUST_BSRW_LAUNCH(bsr16_spmm_wide_strip_kernel<true>);
        } else {
            if (lg) JLUST_BSRW_LAUNCH(bsr16_spmm_wide_long_kernel<false>);
            else JLUST_BSRW_LAUNCH(bsr16_spmm_wide_strip_kernel<false>);
        }
#undef JLUST_BSRW_LAUNCH
        return check_launch(lg ? "bsr16_spmm_wide_long_kernel" : "bsr16_spmm_wide_strip_kernel");
    }
    if (rm && vec && offsets_fit && bsr_strip()) {
        const int64_t strips = (mb + BSR_SR - 1) / BSR_SR;
        const int64_t grids = (strips + NUM_XCD - 1) / NUM_XCD * NUM_XCD;
        if (beta == 0.f)
            hipLaunchKernelGGL((bsr16_spmm_strip_kernel<true>), dim3((unsigned)grids), dim3(64 * BSR_SR), 0, s,
                               mb, origin, browptr, bcolind, val, k, alpha, B, ldb, beta, C, ldc);
        else
            hipLaunchKernelGGL((bsr16_spmm_strip_kernel<false>), dim3((unsigned)grids), dim3(64 * BSR_SR), 0, s,
                               mb, origin, browptr, bcolind, val, k, alpha, B, ldb, beta, C, ldc);
        return check_launch("bsr16_spmm_strip_kernel");
    }
    if (rm && vec) {
        const int64_t wgs = (mb + 3) / 4;
        const int64_t grid4 = (wgs + NUM_XCD - 1) / NUM_XCD * NUM_XCD;
        if (beta == 0.f)
            hipLaunchKernelGGL((bsr16_spmm_rowwave_kernel<true>), dim3((unsigned)grid4), dim3(256), 0, s,
                               mb, origin, browptr, bcolind, val, k, alpha, B, ldb, beta, C, ldc);
        else
            hipLaunchKernelGGL((bsr16_spmm_rowwave_kernel<false>), dim3((unsigned)grid4), dim3(256), 0, s,
                               mb, origin, browptr, bcolind, val, k, alpha, B, ldb, beta, C, ldc);
        return check_launch("bsr16_spmm_rowwave_kernel");
    }
    if (rm && vec) JLUST_BSR_LAUNCH(true, true);
    else if (rm) JLUST_BSR_LAUNCH(true, false);
    else if (vec) JLUST_BSR_LAUNCH(false, true);
    else JLUST_BSR_LAUNCH(false, false);
#undef JLUST_BSR_LAUNCH
    return check_launch("bsr16_spmm_mfma_kernel");
}

int bsr_spmm_f64(int64_t mb, int64_t nb, int64_t bs, int64_t nnzb, int32_t origin,
                 const int32_t *browptr, const int32_t *bcolind, const double *val,
                 int row_major_blocks, int64_t k, double alpha, const double *B, int64_t ldb,
                 double beta, double *C, int64_t ldc, jlust_stream_t stream)
{
    clear_error();
    if (mb < 0 || nb < 0 || bs <= 0 || nnzb < 0 || k < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm: negative extent or block size");
    if (bs != BSR_BS)
        return fail(JLUST_STATUS_UNSUPPORTED_FORMAT,
                    "bsr_spmm: block size %lld x %lld (the MFMA path supports 16 x 16)",
                    (long long)bs, (long long)bs);
    if (mb * bs > INT32_MAX || nb * bs > INT32_MAX || nnzb > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm: extents exceed the Int32 index range");
    if (int st = check_origin(origin)) return st;
    const int64_t mrows = mb * bs, nrows = nb * bs;
    if (ldb < (nrows > 0 ? nrows : 1) || ldc < (mrows > 0 ? mrows : 1))
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "bsr_spmm: leading dimensions too small (ldb=%lld < %lld or ldc=%lld < %lld)",
                    (long long)ldb, (long long)nrows, (long long)ldc, (long long)mrows);
    if ((mb > 0 && !browptr) || bad_ptr(bcolind, nnzb) || bad_ptr(val, nnzb) ||
        bad_ptr(B, (nnzb > 0 && k > 0) ? nrows : 0) || bad_ptr(C, mrows * k))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (mb == 0 || k == 0) return JLUST_STATUS_SUCCESS;
    const bool vec = (ldb % 4 == 0) && (ldc % 4 == 0) && ((uintptr_t)B % 32 == 0) &&
                     ((uintptr_t)C % 32 == 0) && ((uintptr_t)val % 32 == 0);
    const int64_t grid = (mb + NUM_XCD - 1) / NUM_XCD * NUM_XCD;
    hipStream_t s = (hipStream_t)stream;
    const int bz = beta == 0.0;
    // The strip kernel addresses 16 columns of B (from the window's first row)
    // and of C through 32-bit buffer offsets.
    const bool strip_fits = (uint64_t)(16 * ldb + BSR64_SPAN * BSR_BS) * 8 < ((uint64_t)1 << 31) &&
                            (uint64_t)(16 * ldc + mrows) * 8 < ((uint64_t)1 << 31) && k < INT32_MAX - 16;
    if (row_major_blocks && vec && strip_fits && bsr_strip()) {
        // One resident workgroup per CU (the window takes its LDS), each
        // walking its XCD's strips.
        int dev = 0;
        if (int st = require_device(&dev)) return st;
        const int64_t strips = (mb + BSR64_SR - 1) / BSR64_SR;
        const int64_t per_xcd = std::max<int64_t>(1, device_info(dev).cu_count / NUM_XCD);
        const int64_t grids = std::min((strips + NUM_XCD - 1) / NUM_XCD, per_xcd) * NUM_XCD;
        if (bz)
            hipLaunchKernelGGL((bsr16_spmm_f64_strip_kernel<true>), dim3((unsigned)grids), dim3(64 * BSR64_SR), 0,
                               s, mb, origin, browptr, bcolind, val, k, alpha, B, ldb, beta, C, ldc);
        else
            hipLaunchKernelGGL((bsr16_spmm_f64_strip_kernel<false>), dim3((unsigned)grids), dim3(64 * BSR64_SR),
                               0, s, mb, origin, browptr, bcolind, val, k, alpha, B, ldb, beta, C, ldc);
        return check_launch("bsr16_spmm_f64_strip_kernel");
    }
#define JLUST_BSR64_LAUNCH(RM, V)                                                                   \
    hipLaunchKernelGGL((bsr16_spmm_f64_kernel<RM, V>), dim3((unsigned)grid), dim3(64 * BSR_WAVES), \
                       0, s, mb, origin, browptr, bcolind, val, k, alpha, B, ldb, beta, bz, C, ldc)
    if (row_major_blocks && vec) JLUST_BSR64_LAUNCH(true, true);
    else if (row_major_blocks) JLUST_BSR64_LAUNCH(true, false);
    else if (vec) JLUST_BSR64_LAUNCH(false, true);
    else JLUST_BSR64_LAUNCH(false, false);
#undef JLUST_BSR64_LAUNCH
    return check_launch("bsr16_spmm_f64_kernel");
}

}  // namespace
}  // namespace jlust

extern "C" int jlust_hip_bsr_spmm_f64_i32(int64_t mb, int64_t nb, int64_t bs, int64_t nnzb,
                                          int32_t origin, const int32_t *browptr,
                                          const int32_t *bcolind, const double *val,
                                          int row_major_blocks, int64_t k, double alpha,
                                          const double *B, int64_t ldb, double beta, double *C,
                                          int64_t ldc, jlust_stream_t stream)
{
    return jlust::bsr_spmm_f64(mb, nb, bs, nnzb, origin, browptr, bcolind, val, row_major_blocks, k,
                               alpha, B, ldb, beta, C, ldc, stream);
}

extern "C" int jlust_hip_bsr_spmm_f32_i32(int64_t mb, int64_t nb, int64_t bs, int64_t nnzb,
                                          int32_t origin, const int32_t *browptr,
                                          const int32_t *bcolind, const float *val,
                                          int row_major_blocks, int64_t k, float alpha,
                                          const float *B, int64_t ldb, float beta, float *C,
                                          int64_t ldc, jlust_stream_t stream)
{
    return jlust::bsr_spmm(mb, nb, bs, nnzb, origin, browptr, bcolind, val, row_major_blocks, k,
                           alpha, B, ldb, beta, C, ldc, stream);
}

extern "C" int jlust_hip_bsr_spmv_f64_i32(int64_t mb, int64_t nb, int64_t b1, int64_t b2, int64_t nnzb,
                                          int32_t origin, const int32_t *browptr, const int32_t *bcolind,
                                          const double *val, int row_major_blocks, double alpha,
                                          const double *x, double beta, double *y, jlust_stream_t stream)
{
    return jlust::bsr_spmv<double>(mb, nb, b1, b2, nnzb, origin, browptr, bcolind, val, row_major_blocks,
                                   alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_bsr_spmv_f32_i32(int64_t mb, int64_t nb, int64_t b1, int64_t b2, int64_t nnzb,
                                          int32_t origin, const int32_t *browptr, const int32_t *bcolind,
                                          const float *val, int row_major_blocks, float alpha,
                                          const float *x, float beta, float *y, jlust_stream_t stream)
{
    return jlust::bsr_spmv<float>(mb, nb, b1, b2, nnzb, origin, browptr, bcolind, val, row_major_blocks,
                                  alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_bsr_expand_csr_i32(int64_t mb, int64_t b1, int64_t b2, int64_t nnzb, int32_t origin,
                                            const int32_t *browptr, const int32_t *bcolind, const void *val,
                                            int value_type, int row_major_blocks, int32_t *rowptr,
                                            int32_t *colind, void *val_out, jlust_stream_t stream)
{
    return jlust::bsr_expand_csr(mb, b1, b2, nnzb, origin, browptr, bcolind, val, value_type,
                                 row_major_blocks, rowptr, colind, val_out, stream);
}

// ------------------------------------------------------------------- plans

// A prepared BSR SpMM (the analyse-once handle of the C ABI; the cuSPARSE SpMM
// handle contract, ext/CUDAExt/ops/spmm.jl:8-70, for BSR).  16 x 16 blocks,
// Float32 or Float64, keep the MFMA kernels and the caller's buffers
// (update_values swaps the value pointer).  Any other block shape is
// expanded to CSR once (the plan owns the expansion) and runs through a CSR
// SpMM plan over it; update_values re-expands the values only, on the stream.
static size_t bsr_align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct jlust_bsr_plan {
    int64_t mb = 0, nb = 0, b1 = 0, b2 = 0, nnzb = 0, k = 0;
    int32_t origin = 0;
    int value_type = 0, row_major = 1, device = 0;
    const int32_t *browptr = nullptr;
    const int32_t *bcolind = nullptr;
    const void *val = nullptr;
    bool mfma = false;
    void *mem = nullptr;                // expansion: rowptr | colind | values
    int32_t *rowptr = nullptr;
    int32_t *colind = nullptr;
    void *cval = nullptr;
    jlust_spmm_plan_t csr = nullptr;
};

static int bsr_spmm_plan_create_body(int64_t mb, int64_t nb, int64_t b1, int64_t b2, int64_t nnzb,
                                     int32_t origin, int value_type, int row_major_blocks,
                                     const int32_t *browptr, const int32_t *bcolind, const void *val,
                                     int64_t k, jlust_stream_t stream, jlust_bsr_plan_t *plan_out)
{
    using namespace jlust;
    clear_error();
    if (!plan_out) return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_create: null plan_out");
    *plan_out = nullptr;
    if (mb < 0 || nb < 0 || b1 <= 0 || b2 <= 0 || nnzb < 0 || k < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_create: negative extent or block size");
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE,
                    "bsr_spmm_plan_create: value_type %d (0 = Float64, 1 = Float32)", value_type);
    if (int st = check_origin(origin)) return st;
    if (mb * b1 >= INT32_MAX || nb * b2 >= INT32_MAX || nnzb * b1 * b2 >= (int64_t)INT32_MAX - 1)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_create: extents exceed the Int32 index range");
    const int64_t total = nnzb * b1 * b2;
    if (!browptr || bad_ptr(bcolind, nnzb) || bad_ptr(val, total))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_create: null device pointer");
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    std::unique_ptr<jlust_bsr_plan> p(new jlust_bsr_plan());
    p->mb = mb;
    p->nb = nb;
    p->b1 = b1;
    p->b2 = b2;
    p->nnzb = nnzb;
    p->k = k;
    p->origin = origin;
    p->value_type = value_type;
    p->row_major = row_major_blocks ? 1 : 0;
    p->device = dev;
    p->browptr = browptr;
    p->bcolind = bcolind;
    p->val = val;
    // 16 x 16 blocks run the MFMA kernels on A's buffers (fp32 row-major
    // blocks need 16-byte aligned values; fp64 takes any alignment).
    p->mfma = b1 == BSR_BS && b2 == BSR_BS &&
              (value_type == 0 || !row_major_blocks || (uintptr_t)val % 16 == 0);
    if (!p->mfma) {
        const size_t tsz = value_type == 0 ? sizeof(double) : sizeof(float);
        const size_t nz = (size_t)(total > 0 ? total : 1);
        const size_t sz_rp = bsr_align_up(sizeof(int32_t) * (size_t)(mb * b1 + 1), 256);
        const size_t sz_ci = bsr_align_up(sizeof(int32_t) * nz, 256);
        JLUST_HIP_TRY(hipMalloc(&p->mem, sz_rp + sz_ci + bsr_align_up(tsz * nz, 256)));
        char *b = (char *)p->mem;
        p->rowptr = (int32_t *)b;
        p->colind = (int32_t *)(b + sz_rp);
        p->cval = b + sz_rp + sz_ci;
        int st = bsr_expand_csr(mb, b1, b2, nnzb, origin, browptr, bcolind, val, value_type, p->row_major,
                                p->rowptr, p->colind, p->cval, stream);
        if (!st)
            st = jlust_hip_csr_spmm_plan_create(mb * b1, nb * b2, k, total, origin, value_type, p->rowptr,
                                                p->colind, p->cval, stream, &p->csr);
        if (st) {
            (void)hipStreamSynchronize((hipStream_t)stream);
            (void)hipFree(p->mem);
            return st;
        }
    }
    *plan_out = p.release();
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_bsr_spmm_plan_create(int64_t mb, int64_t nb, int64_t b1, int64_t b2, int64_t nnzb,
                                              int32_t origin, int value_type, int row_major_blocks,
                                              const int32_t *browptr, const int32_t *bcolind, const void *val,
                                              int64_t k, jlust_stream_t stream, jlust_bsr_plan_t *plan_out)
{
    return jlust::host_guard("bsr_spmm_plan_create", [&] {
        return bsr_spmm_plan_create_body(mb, nb, b1, b2, nnzb, origin, value_type, row_major_blocks,
                                         browptr, bcolind, val, k, stream, plan_out);
    });
}

extern "C" int jlust_hip_bsr_spmm_plan_update_values(jlust_bsr_plan_t plan, const void *val, jlust_stream_t stream)
{
    using namespace jlust;
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_update_values: null plan");
    const int64_t total = plan->nnzb * plan->b1 * plan->b2;
    if (bad_ptr(val, total)) return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_update_values: null values");
    if (plan->mfma && plan->value_type == 1 && plan->row_major && (uintptr_t)val % 16 != 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_update_values: block values must be 16-byte aligned");
    plan->val = val;
    if (plan->mfma) return JLUST_STATUS_SUCCESS;     // the kernels read the values in place
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    if (dev != plan->device)
        return fail(JLUST_STATUS_INVALID_ARGUMENT,
                    "bsr_spmm_plan_update_values: plan belongs to device %d, current device is %d", plan->device, dev);
    return bsr_expand_entries(plan->mb, plan->b1, plan->b2, plan->nnzb, plan->origin, plan->browptr, plan->bcolind,
                              val, plan->value_type, plan->row_major, nullptr, plan->cval, (hipStream_t)stream);
}

extern "C" int jlust_hip_bsr_spmm_plan_execute_f32(jlust_bsr_plan_t plan, float alpha, const float *B, int64_t ldb,
                                                   float beta, float *C, int64_t ldc, jlust_stream_t stream)
{
    using namespace jlust;
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_execute: null plan");
    if (plan->value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "bsr_spmm_plan_execute: plan was created for Float64 values");
    if (!plan->mfma)
        return jlust_hip_csr_spmm_plan_execute_f32(plan->csr, alpha, B, ldb, beta, C, ldc, 0, stream);
    return bsr_spmm(plan->mb, plan->nb, BSR_BS, plan->nnzb, plan->origin, plan->browptr, plan->bcolind,
                    (const float *)plan->val, plan->row_major, plan->k, alpha, B, ldb, beta, C, ldc, stream);
}

extern "C" int jlust_hip_bsr_spmm_plan_execute_f64(jlust_bsr_plan_t plan, double alpha, const double *B, int64_t ldb,
                                                   double beta, double *C, int64_t ldc, jlust_stream_t stream)
{
    using namespace jlust;
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_execute: null plan");
    if (plan->value_type != 0)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "bsr_spmm_plan_execute: plan was created for Float32 values");
    if (!plan->mfma)
        return jlust_hip_csr_spmm_plan_execute_f64(plan->csr, alpha, B, ldb, beta, C, ldc, 0, stream);
    return bsr_spmm_f64(plan->mb, plan->nb, BSR_BS, plan->nnzb, plan->origin, plan->browptr, plan->bcolind,
                        (const double *)plan->val, plan->row_major, plan->k, alpha, B, ldb, beta, C, ldc, stream);
}

extern "C" int jlust_hip_bsr_spmm_plan_info(jlust_bsr_plan_t plan, int32_t *path)
{
    jlust::clear_error();
    if (!plan) return jlust::fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmm_plan_info: null plan");
    if (path) *path = plan->mfma ? 0 : 1;
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_bsr_spmm_plan_destroy(jlust_bsr_plan_t plan)
{
    jlust::clear_error();
    if (!plan) return JLUST_STATUS_SUCCESS;
    // Work queued on any stream may still read the plan's buffers.
    hipError_t e = hipDeviceSynchronize();
    int st = plan->csr ? jlust_hip_csr_spmm_plan_destroy(plan->csr) : JLUST_STATUS_SUCCESS;
    if (plan->mem) {
        const hipError_t e2 = hipFree(plan->mem);
        if (e == hipSuccess) e = e2;
    }
    delete plan;
    if (e != hipSuccess) return jlust::hip_fail(e, "bsr_spmm_plan_destroy");
    return st;
}

// ---- prepared BSR SpMV: the segment table built once.
struct jlust_bsr_spmv_plan {
    int64_t mb = 0, nb = 0, b1 = 0, b2 = 0, nnzb = 0, nsegmax = 0;
    int32_t origin = 0;
    int value_type = 0, row_major = 1, device = 0;
    const int32_t *browptr = nullptr;
    const int32_t *bcolind = nullptr;
    const void *val = nullptr;
    void *mem = nullptr;                // segstart | segrow | partial sums
    int32_t *segstart = nullptr;
    int32_t *segrow = nullptr;
    void *part = nullptr;
};

static int bsr_spmv_plan_create_body(int64_t mb, int64_t nb, int64_t b1, int64_t b2, int64_t nnzb,
                                     int32_t origin, int value_type, int row_major_blocks,
                                     const int32_t *browptr, const int32_t *bcolind, const void *val,
                                     jlust_stream_t stream, jlust_bsr_spmv_plan_t *plan_out)
{
    using namespace jlust;
    clear_error();
    if (!plan_out) return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_create: null plan_out");
    *plan_out = nullptr;
    if (mb < 0 || nb < 0 || b1 <= 0 || b2 <= 0 || nnzb < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_create: negative extent or block size");
    if (value_type != 0 && value_type != 1)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE,
                    "bsr_spmv_plan_create: value_type %d (0 = Float64, 1 = Float32)", value_type);
    if (int st = check_origin(origin)) return st;
    if (mb * b1 > INT32_MAX || nb * b2 > INT32_MAX || nnzb * b1 * b2 > INT32_MAX)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_create: extents exceed the Int32 index range");
    if ((mb > 0 && !browptr) || bad_ptr(bcolind, nnzb) || bad_ptr(val, nnzb * b1 * b2))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_create: null device pointer");
    if (nnzb > 0 && nb == 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_create: blocks stored in a matrix with no columns");
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    std::unique_ptr<jlust_bsr_spmv_plan> p(new jlust_bsr_spmv_plan());
    p->mb = mb;
    p->nb = nb;
    p->b1 = b1;
    p->b2 = b2;
    p->nnzb = nnzb;
    p->origin = origin;
    p->value_type = value_type;
    p->row_major = row_major_blocks ? 1 : 0;
    p->device = dev;
    p->browptr = browptr;
    p->bcolind = bcolind;
    p->val = val;
    if (mb > 0) {
        // browptr's ends, read back: the table's kernels would only clamp a
        // malformed pointer array.
        hipStream_t s = (hipStream_t)stream;
        int32_t ends[2] = {0, 0};
        JLUST_HIP_TRY(hipMemcpyAsync(&ends[0], browptr, sizeof(int32_t), hipMemcpyDeviceToHost, s));
        JLUST_HIP_TRY(hipMemcpyAsync(&ends[1], browptr + mb, sizeof(int32_t), hipMemcpyDeviceToHost, s));
        JLUST_HIP_TRY(hipStreamSynchronize(s));
        if (ends[0] != origin || (int64_t)ends[1] != nnzb + origin)
            return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                        "bsr_spmv_plan_create: browptr runs from %d to %d, expected %d to %lld", ends[0], ends[1],
                        origin, (long long)(nnzb + origin));
        const size_t tsz = value_type == 0 ? sizeof(double) : sizeof(float);
        p->nsegmax = bsr_spmv_nsegmax(mb, nnzb);
        const size_t sz_st = bsr_align_up(sizeof(int32_t) * (size_t)(mb + 1), 256);
        const size_t sz_rw = bsr_align_up(sizeof(int32_t) * (size_t)p->nsegmax, 256);
        JLUST_HIP_TRY(hipMalloc(&p->mem, sz_st + sz_rw + bsr_align_up(tsz * (size_t)(p->nsegmax * b1), 256)));
        char *b = (char *)p->mem;
        p->segstart = (int32_t *)b;
        p->segrow = (int32_t *)(b + sz_st);
        p->part = b + sz_st + sz_rw;
        int st = bsr_spmv_table(mb, nnzb, origin, browptr, p->segstart, p->segrow, p->nsegmax, stream);
        if (!st) {
            const hipError_t e = hipStreamSynchronize(s);  // the plan may then run on any stream
            if (e != hipSuccess) st = hip_fail(e, "bsr_spmv_plan_create");
        }
        if (st) {
            (void)hipStreamSynchronize(s);
            (void)hipFree(p->mem);
            return st;
        }
    }
    *plan_out = p.release();
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_bsr_spmv_plan_create(int64_t mb, int64_t nb, int64_t b1, int64_t b2, int64_t nnzb,
                                              int32_t origin, int value_type, int row_major_blocks,
                                              const int32_t *browptr, const int32_t *bcolind, const void *val,
                                              jlust_stream_t stream, jlust_bsr_spmv_plan_t *plan_out)
{
    return jlust::host_guard("bsr_spmv_plan_create", [&] {
        return bsr_spmv_plan_create_body(mb, nb, b1, b2, nnzb, origin, value_type, row_major_blocks, browptr,
                                         bcolind, val, stream, plan_out);
    });
}

extern "C" int jlust_hip_bsr_spmv_plan_update_values(jlust_bsr_spmv_plan_t plan, const void *val,
                                                     jlust_stream_t stream)
{
    using namespace jlust;
    (void)stream;                           // a pointer swap: nothing to enqueue
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_update_values: null plan");
    if (bad_ptr(val, plan->nnzb * plan->b1 * plan->b2))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_update_values: null values");
    plan->val = val;
    return JLUST_STATUS_SUCCESS;
}

template <typename T>
static int bsr_spmv_plan_execute(jlust_bsr_spmv_plan_t plan, int value_type, T alpha, const T *x, T beta, T *y,
                                 jlust_stream_t stream)
{
    using namespace jlust;
    clear_error();
    if (!plan) return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_execute: null plan");
    if (plan->value_type != value_type)
        return fail(JLUST_STATUS_UNSUPPORTED_VALUE_TYPE, "bsr_spmv_plan_execute: plan was created for %s values",
                    plan->value_type == 0 ? "Float64" : "Float32");
    if ((plan->nnzb > 0 && !x) || bad_ptr(y, plan->mb * plan->b1))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_execute: null device pointer");
    int dev = 0;
    if (int st = require_device(&dev)) return st;
    if (dev != plan->device)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "bsr_spmv_plan_execute: plan belongs to device %d, current device is %d",
                    plan->device, dev);
    if (plan->mb == 0) return JLUST_STATUS_SUCCESS;
    return bsr_spmv_run<T>(plan->mb, plan->nb, plan->b1, plan->b2, plan->nnzb, plan->origin, plan->browptr,
                           plan->bcolind, (const T *)plan->val, plan->row_major, alpha, x, beta, y, plan->segstart,
                           plan->segrow, (T *)plan->part, plan->nsegmax, stream);
}

extern "C" int jlust_hip_bsr_spmv_plan_execute_f64(jlust_bsr_spmv_plan_t plan, double alpha, const double *x,
                                                   double beta, double *y, jlust_stream_t stream)
{
    return bsr_spmv_plan_execute<double>(plan, 0, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_bsr_spmv_plan_execute_f32(jlust_bsr_spmv_plan_t plan, float alpha, const float *x,
                                                   float beta, float *y, jlust_stream_t stream)
{
    return bsr_spmv_plan_execute<float>(plan, 1, alpha, x, beta, y, stream);
}

extern "C" int jlust_hip_bsr_spmv_plan_destroy(jlust_bsr_spmv_plan_t plan)
{
    jlust::clear_error();
    if (!plan) return JLUST_STATUS_SUCCESS;
    // Work queued on any stream may still read the plan's buffers.
    hipError_t e = hipDeviceSynchronize();
    if (plan->mem) {
        const hipError_t e2 = hipFree(plan->mem);
        if (e == hipSuccess) e = e2;
    }
    delete plan;
    if (e != hipSuccess) return jlust::hip_fail(e, "bsr_spmv_plan_destroy");
    return JLUST_STATUS_SUCCESS;
}

namespace jlust {
int preload_bsr()
{
    JLUST_PRELOAD_KERNEL(bsr_expand_rowptr_kernel);
    JLUST_PRELOAD_KERNEL(bsr16_spmv_count_kernel);
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
