// fn.hip -- elementwise transforms around SpMV: the input_fn / output_fn of
// JLUST's SpMV (execute(::EmitterBackend, ::Op{:SpMV}; input_fn, output_fn),
// ext/KernelAbstractionsExt/ops/spmv.jl:371-374; applied to every gathered
// x element at the leaf, :141,154, and to each row sum before the write,
// :168-169).
//
//   y = alpha * out_fn(A * in_fn.(x)) + beta * y
//
// runs here as dst = in_fn(x) over n elements, the SpMV with alpha = 1 and
// beta = 0 into a row-sum vector, and y = alpha * out_fn(rowsum) + beta * y
// over m elements.  Multiplying a sum by 1 and a beta = 0 write-only store
// are exact, so the result equals the fused form's; the extra passes move
// O(n + m) bytes next to the O(nnz) of the product.  Products and sums are
// not contracted into FMAs, as in the reference's generic Julia code.
#include "common.hpp"

#include <cmath>

namespace jlust {
namespace {

constexpr int FN_BLOCK = 256;

template <typename T>
__device__ __forceinline__ T apply(int kind, T a, T b, T v)
{
#pragma clang fp contract(off)
    switch (kind) {
    case JLUST_FN_AFFINE: return a * v + b;
    case JLUST_FN_ABS: return fabs(v);
    case JLUST_FN_SQUARE: return v * v;
    case JLUST_FN_SQRT: return sqrt(v);
    case JLUST_FN_EXP: return exp(v);
    case JLUST_FN_LOG: return log(v);
    case JLUST_FN_RELU: return v > T(0) ? v : (v != v ? v : T(0));
    default: return v;
    }
}

template <typename T>
__global__ __launch_bounds__(FN_BLOCK) void apply_fn_kernel(int64_t n, int kind, T a, T b,
                                                            const T *__restrict__ src, T alpha, T beta,
                                                            T *dst)
{
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * FN_BLOCK + threadIdx.x;
    if (i >= n) return;
    const T f = apply<T>(kind, a, b, src[i]);
    dst[i] = beta == T(0) ? alpha * f : alpha * f + beta * dst[i];
}

template <typename T>
int apply_fn(int64_t n, int32_t kind, T a, T b, const T *src, T alpha, T beta, T *dst, jlust_stream_t stream)
{
    clear_error();
    if (n < 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "apply_fn: negative length");
    if (kind < JLUST_FN_IDENTITY || kind > JLUST_FN_RELU)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "apply_fn: unknown function kind %d", kind);
    if (bad_ptr(src, n) || bad_ptr(dst, n)) return fail(JLUST_STATUS_INVALID_ARGUMENT, "apply_fn: null device pointer");
    if (int st = require_device(nullptr)) return st;
    if (n == 0) return JLUST_STATUS_SUCCESS;
    hipLaunchKernelGGL((apply_fn_kernel<T>), dim3((unsigned)((n + FN_BLOCK - 1) / FN_BLOCK)), dim3(FN_BLOCK), 0,
                       (hipStream_t)stream, n, (int)kind, a, b, src, alpha, beta, dst);
    return check_launch("apply_fn_kernel");
}

}  // namespace
}  // namespace jlust

extern "C" int jlust_hip_apply_fn_f64(int64_t n, int32_t kind, double a, double b, const double *src,
                                      double alpha, double beta, double *dst, jlust_stream_t stream)
{
    return jlust::apply_fn<double>(n, kind, a, b, src, alpha, beta, dst, stream);
}

extern "C" int jlust_hip_apply_fn_f32(int64_t n, int32_t kind, float a, float b, const float *src,
                                      float alpha, float beta, float *dst, jlust_stream_t stream)
{
    return jlust::apply_fn<float>(n, kind, a, b, src, alpha, beta, dst, stream);
}

namespace jlust {
int preload_fn()
{
    JLUST_PRELOAD_KERNEL(apply_fn_kernel<double>);
    return JLUST_STATUS_SUCCESS;
}
}  // namespace jlust
