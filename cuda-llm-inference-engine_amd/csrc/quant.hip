// quant.hip — per-row symmetric FP32 -> INT8 quantizer for gfx950.
//
// Semantics follow kernels/quantization/14_int8_gemm.cu:10-60 of the
// reference bit for bit: row_max = max|x|, scale = row_max/127 (1 for an
// all-zero row), q = clamp(rint(x * (1/scale)), -128, 127), four q packed
// little-endian per int32 word.  Division is IEEE (correctly rounded) and
// rint is round-half-to-even, as on the reference's device.
//
// Layout on MI355X: one 256-thread workgroup per row; every lane moves 16 B
// (one float4 in, one packed int32 out) per step, so a wave reads 1 KiB and
// writes 256 B contiguous per instruction.  The second pass over the row hits
// L2 (a row is at most a few tens of KiB).
#include "device_util.h"
#include "ie_internal.h"

namespace ie {
namespace {

__global__ __launch_bounds__(256) void quantize_rows_kernel(
    int cols, const float* __restrict__ in, int32_t* __restrict__ out,
    float* __restrict__ scales) {
    const int row = blockIdx.x;
    const int n4 = cols >> 2;
    const float4* x = reinterpret_cast<const float4*>(in + (size_t)row * cols);

    float m = 0.0f;
    for (int i = threadIdx.x; i < n4; i += 256) {
        const float4 v = x[i];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    m = wave_max(m);
    __shared__ float wmax[4];
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));

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
    quantize_rows_kernel<<<rows, 256, 0, s>>>(cols, in, packed, scales);
}

}  // namespace ie
