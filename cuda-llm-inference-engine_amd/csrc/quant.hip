// quant.hip — per-row symmetric FP32 -> INT8 quantizer for gfx950.
//
// Semantics follow kernels/quantization/14_int8_gemm.cu:10-60 of the
// reference bit for bit: row_max = max|x|, scale = row_max/127 (1 for an
// all-zero row), q = clamp(rint(x * (1/scale)), -128, 127), four q packed
// little-endian per int32 word.  Division is IEEE (correctly rounded) and
// rint is round-half-to-even, as on the reference's device.
//
// Layout on MI355X: the row is read once and kept in registers.
//   * cols <= 1024: one wave per row (four rows per 256-thread workgroup);
//     lane l holds the row's float4s l, l + 64, ... and the row max is a
//     wave reduction (no LDS, no barrier);
//   * cols <= 4096: one 256-thread workgroup per row, up to four float4s per
//     lane, the four wave maxima combined through LDS;
//   * wider rows: the same workgroup walks the row twice (max, then
//     quantize; the second pass hits L2).
// Every form issues its loads unconditionally with the index clamped into the
// row, so they all go out before the first wait; a clamped duplicate cannot
// change the max, and only in-row words are stored.  The max is exact in any
// order, so all forms give the same bits.
#include "device_util.h"
#include "ie_internal.h"

namespace ie {
namespace {

__device__ __forceinline__ float abs_max4(float4 v) {
    return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// cols <= 64 NV * 4: one wave per row, NV float4s per lane.
template <int NV>
__global__ __launch_bounds__(256) void quantize_rows_wave_kernel(int rows, int cols, const float* __restrict__ in,
                                                                 int32_t* __restrict__ out,
                                                                 float* __restrict__ scales) {
    const int lane = threadIdx.x & 63;
    const int row = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (row >= rows) return;
    const int n4 = cols >> 2;
    const float4* x = reinterpret_cast<const float4*>(in + (size_t)row * cols);
    float4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = x[min(lane + 64 * j, n4 - 1)];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) m = fmaxf(m, abs_max4(v[j]));
    m = wave_max(m);
    const float scale = quant_scale(m);
    const float inv = 1.0f / scale;
    if (lane == 0) scales[row] = scale;
    int32_t* o = out + (size_t)row * n4;
#pragma unroll
    for (int j = 0; j < NV; ++j)
        if (lane + 64 * j < n4) o[lane + 64 * j] = quant_word(v[j], inv);
}

// Maximum of the four waves' m through LDS (every thread gets it).
__device__ __forceinline__ float block4_max(float m) {
    __shared__ float wmax[4];
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    return fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
}

// cols <= 256 NV * 4: one workgroup per row, NV float4s per thread.
template <int NV>
__global__ __launch_bounds__(256) void quantize_rows_reg_kernel(int cols, const float* __restrict__ in,
                                                                int32_t* __restrict__ out,
                                                                float* __restrict__ scales) {
    const int row = blockIdx.x;
    const int n4 = cols >> 2;
    const float4* x = reinterpret_cast<const float4*>(in + (size_t)row * cols);
    float4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = x[min((int)threadIdx.x + 256 * j, n4 - 1)];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) m = fmaxf(m, abs_max4(v[j]));
    m = block4_max(m);
    const float scale = quant_scale(m);
    const float inv = 1.0f / scale;
    if (threadIdx.x == 0) scales[row] = scale;
    int32_t* o = out + (size_t)row * n4;
#pragma unroll
    for (int j = 0; j < NV; ++j)
        if ((int)threadIdx.x + 256 * j < n4) o[threadIdx.x + 256 * j] = quant_word(v[j], inv);
}

// Any cols: one workgroup per row, two passes.
__global__ __launch_bounds__(256) void quantize_rows_kernel(
    int cols, const float* __restrict__ in, int32_t* __restrict__ out,
    float* __restrict__ scales) {
    const int row = blockIdx.x;
    const int n4 = cols >> 2;
    const float4* x = reinterpret_cast<const float4*>(in + (size_t)row * cols);

    float m = 0.0f;
    for (int i = threadIdx.x; i < n4; i += 256) m = fmaxf(m, abs_max4(x[i]));
    m = block4_max(m);

    const float scale = quant_scale(m);
    const float inv = 1.0f / scale;
    if (threadIdx.x == 0) scales[row] = scale;

    int32_t* o = out + (size_t)row * n4;
    for (int i = threadIdx.x; i < n4; i += 256) {
        o[i] = quant_word(x[i], inv);
    }
}

}  // namespace

void launch_quantize(int rows, int cols, const float* in, int32_t* packed,
                     float* scales, hipStream_t s) {
    if (rows == 0) return;
    if (cols == 0) {
        // every row is all-zero: scale 1, nothing packed
        quantize_rows_kernel<<<rows, 256, 0, s>>>(cols, in, packed, scales);
        return;
    }
    const int n4 = cols >> 2;
    const unsigned wblocks = (unsigned)((rows + 3) / 4);
    if (n4 <= 64)
        quantize_rows_wave_kernel<1><<<wblocks, 256, 0, s>>>(rows, cols, in, packed, scales);
    else if (n4 <= 128)
        quantize_rows_wave_kernel<2><<<wblocks, 256, 0, s>>>(rows, cols, in, packed, scales);
    else if (n4 <= 192)
        quantize_rows_wave_kernel<3><<<wblocks, 256, 0, s>>>(rows, cols, in, packed, scales);
    else if (n4 <= 256)
        quantize_rows_wave_kernel<4><<<wblocks, 256, 0, s>>>(rows, cols, in, packed, scales);
    else if (n4 <= 512)
        quantize_rows_reg_kernel<2><<<rows, 256, 0, s>>>(cols, in, packed, scales);
    else if (n4 <= 768)
        quantize_rows_reg_kernel<3><<<rows, 256, 0, s>>>(cols, in, packed, scales);
    else if (n4 <= 1024)
        quantize_rows_reg_kernel<4><<<rows, 256, 0, s>>>(cols, in, packed, scales);
    else
        quantize_rows_kernel<<<rows, 256, 0, s>>>(cols, in, packed, scales);
}

}  // namespace ie
