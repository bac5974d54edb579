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

// Combining the four 16-lane rows of a wave with gfx950's v_permlane16_swap /
// v_permlane32_swap (plain VALU ops, no LDS round trip as ds_bpermute has):
// with both registers holding v, lane l ends with {v[l & ~16], v[l | 16]}
// (resp. 32), so op(lo, hi) is the same value in both lanes of a pair, in a
// fixed order.  The instruction rewrites both of its registers; it is issued
// from inline assembly because the compiler's builtin (ROCm 7.2) drops the
// second result when both operands hold the same value.  The leading s_nop
// covers the VALU-write-then-permlane-read hazard, as the compiler does for
// the builtin.
__device__ __forceinline__ void pair16(float v, float& lo, float& hi) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    __asm__ volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    lo = __builtin_bit_cast(float, a);
    hi = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ void pair32(float v, float& lo, float& hi) {
    uint32_t a = __builtin_bit_cast(uint32_t, v), b = a;
    __asm__ volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    lo = __builtin_bit_cast(float, a);
    hi = __builtin_bit_cast(float, b);
}
// v + v[l ^ 16] and v + v[l ^ 32] (rows paired), and the max forms.
__device__ __forceinline__ float sum_xor16(float v) {
    float a, b;
    pair16(v, a, b);
    return a + b;
}
__device__ __forceinline__ float sum_xor32(float v) {
    float a, b;
    pair32(v, a, b);
    return a + b;
}
__device__ __forceinline__ float max_xor16(float v) {
    float a, b;
    pair16(v, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float v) {
    float a, b;
    pair32(v, a, b);
    return fmaxf(a, b);
}

// Whole-wave reductions: DPP within each row, then the row pairs.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_row_ror<8>(v));
    v = fmaxf(v, dpp_row_ror<4>(v));
    v = fmaxf(v, dpp_row_ror<2>(v));
    v = fmaxf(v, dpp_row_ror<1>(v));
    return v;
}
__device__ __forceinline__ float wave_max(float v) { return max_xor32(max_xor16(row16_max(v))); }
__device__ __forceinline__ float wave_sum(float v) { return sum_xor32(sum_xor16(row16_sum(v))); }

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

// The per-row symmetric quantizer's arithmetic (kernels/quantization/
// 14_int8_gemm.cu:37-51 of the reference): scale = row_max / 127 (1 for an
// all-zero row), byte = clamp(rint(x * (1 / scale)), -128, 127).  Shared by
// the standalone quantizer and the GEMV prologues, so both give identical
// bytes for the same row.
__device__ __forceinline__ float quant_scale(float row_max) {
    return row_max > 0.0f ? row_max / 127.0f : 1.0f;
}
__device__ __forceinline__ uint32_t quant_byte(float x, float inv) {
    const float r = fminf(fmaxf(rintf(x * inv), -128.0f), 127.0f);
    return (uint32_t)((int32_t)r) & 0xffu;
}
__device__ __forceinline__ int32_t quant_word(float4 v, float inv) {
    return (int32_t)(quant_byte(v.x, inv) | (quant_byte(v.y, inv) << 8) |
                     (quant_byte(v.z, inv) << 16) | (quant_byte(v.w, inv) << 24));
}

// LayerNorm of one row held by one wave (kernels/layernorm/
// 15_layernorm_residual.cu:59-103 of the reference: mean = E[x],
// var = E[x^2] - mean^2, y = gamma (x - mean) rsqrt(var + eps) + beta).
// Lane l accumulates its float4s l, l + 64, ... in index order (x, y, z, w),
// then the wave combines the partials in a fixed butterfly.  The standalone
// LayerNorm and the GEMV prologue both use these, so they give identical
// bits for the same row.
__device__ __forceinline__ void ln_accum(float4 v, float& s, float& s2) {
    s += v.x;
    s += v.y;
    s += v.z;
    s += v.w;
    s2 = fmaf(v.x, v.x, s2);
    s2 = fmaf(v.y, v.y, s2);
    s2 = fmaf(v.z, v.z, s2);
    s2 = fmaf(v.w, v.w, s2);
}
__device__ __forceinline__ void ln_finish(float s, float s2, int cols, float eps, float& mean,
                                          float& rs) {
    s = wave_sum(s);
    s2 = wave_sum(s2);
    mean = s / (float)cols;
    const float var = fmaf(-mean, mean, s2 / (float)cols);
    rs = rsqrtf(var + eps);
}
__device__ __forceinline__ float4 ln_apply(float4 v, float4 g, float4 b, float mean, float rs) {
    return make_float4(fmaf(g.x * (v.x - mean), rs, b.x), fmaf(g.y * (v.y - mean), rs, b.y),
                       fmaf(g.z * (v.z - mean), rs, b.z), fmaf(g.w * (v.w - mean), rs, b.w));
}

// 8-bit signed dot product accumulate: acc + sum_i a.byte[i] * b.byte[i].
__device__ __forceinline__ int32_t dot4_i8(int32_t a, int32_t b, int32_t acc) {
    return __builtin_amdgcn_sdot4(a, b, acc, false);
}

template <typename T>
using global_ptr = __attribute__((address_space(1))) const T*;

// The same global address with its provenance hidden from alias analysis.
// Loads through a const __restrict__ kernel argument count as invariant, and
// the compiler moves invariant loads freely (sinking them past a ring's exit
// branches or below the MFMAs of the pass that issues them), which turns a
// register ring into issue-all-then-drain.  Loads through the returned
// pointer keep their place relative to memory clobbers and scheduling
// barriers (and stay global loads: the address space survives).
template <typename T>
__device__ __forceinline__ const T* opaque_global(const T* p) {
    global_ptr<T> g = (global_ptr<T>)p;
    asm volatile("" : "+s"(g));
    return (const T*)g;
}

// 2^x as the one instruction v_exp_f32.  exp2f wraps it in a range step
// (compare, select, add, select, ldexp) so that results below 2^-126 come out
// denormal instead of flushed; every other result is the same bits.  The
// softmax weights are 2^(s - running max) <= 1, and a weight below 2^-126 is
// added to sums that already hold the running maximum's weight of 1.
__device__ __forceinline__ float exp2_sm(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace ie
