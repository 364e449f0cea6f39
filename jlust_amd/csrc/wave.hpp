// wave.hpp -- wave64 cross-lane helpers (DPP segmented scan) shared by the
// SpMV kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace jlust {

// ---- wave64 DPP (GFX9 controls): row_shr:n = 0x110+n, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143, wave_shr:1 = 0x138.  Lanes without a source keep `old`.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int32_t dpp_i32(int32_t old, int32_t v)
{
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xf, false);
}

template <int CTRL, int ROW_MASK, typename T>
__device__ __forceinline__ T dpp_val(T old, T v)
{
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, dpp_i32<CTRL, ROW_MASK>(__builtin_bit_cast(int32_t, old),
                                                             __builtin_bit_cast(int32_t, v)));
    } else {
        const uint64_t o = __builtin_bit_cast(uint64_t, old), x = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = (uint32_t)dpp_i32<CTRL, ROW_MASK>((int32_t)o, (int32_t)x);
        const uint32_t hi = (uint32_t)dpp_i32<CTRL, ROW_MASK>((int32_t)(o >> 32), (int32_t)(x >> 32));
        return __builtin_bit_cast(T, ((uint64_t)hi << 32) | lo);
    }
}

template <int CTRL, int ROW_MASK, typename T>
__device__ __forceinline__ void seg_scan_step(int32_t key, T &v)
{
    const int32_t k2 = dpp_i32<CTRL, ROW_MASK>(-1, key);
    const T v2 = dpp_val<CTRL, ROW_MASK>(T(0), v);
    if (k2 == key) v += v2;
}

// Inclusive scan of v over the wave in lane order, segmented by key (keys are
// non-decreasing with the lane and never -1).
template <typename T>
__device__ __forceinline__ T wave_seg_scan(int32_t key, T v)
{
    seg_scan_step<0x111, 0xf>(key, v);
    seg_scan_step<0x112, 0xf>(key, v);
    seg_scan_step<0x114, 0xf>(key, v);
    seg_scan_step<0x118, 0xf>(key, v);
    seg_scan_step<0x142, 0xa>(key, v);
    seg_scan_step<0x143, 0xc>(key, v);
    return v;
}

}  // namespace jlust
