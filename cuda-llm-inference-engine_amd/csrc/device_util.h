// device_util.h — small gfx950 device helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ie {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// DPP row rotate-right by n lanes within each 16-lane row (ROW_ROR:n).
template <int N>
__device__ __forceinline__ float dpp_row_ror(float v) {
    static_assert(N >= 1 && N <= 15, "row_ror range");
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                           0x120 + N, 0xf, 0xf, false));
}
template <int N>
__device__ __forceinline__ int dpp_row_ror(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x120 + N, 0xf, 0xf, false);
}

// Sum over the 16 lanes of each DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_row_ror<8>(v);
    v += dpp_row_ror<4>(v);
    v += dpp_row_ror<2>(v);
    v += dpp_row_ror<1>(v);
    return v;
}
__device__ __forceinline__ int row16_sum(int v) {
    v += dpp_row_ror<8>(v);
    v += dpp_row_ror<4>(v);
    v += dpp_row_ror<2>(v);
    v += dpp_row_ror<1>(v);
    return v;
}

// Exchange between the four 16-lane rows of a wave (lane ^ 16, lane ^ 32).
__device__ __forceinline__ float xor16(float v) { return __shfl_xor(v, 16, 64); }
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}

// Round-to-nearest-even fp32 -> bf16 bit pattern; NaN stays NaN (quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// 8-bit signed dot product accumulate: acc + sum_i a.byte[i] * b.byte[i].
__device__ __forceinline__ int32_t dot4_i8(int32_t a, int32_t b, int32_t acc) {
    return __builtin_amdgcn_sdot4(a, b, acc, false);
}

}  // namespace ie
