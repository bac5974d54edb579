// support.hip — the non-GEMM, non-attention operations of the decode step:
// LayerNorm, token+position embedding, fp32 vocabulary projection and a
// device-side argmax.  They run once or twice per layer on [M, d] rows, so they
// are written for low latency, not as roofline kernels.
#include <cfloat>

#include "device_util.h"
#include "ie_internal.h"

namespace ie {
namespace {

// kernels/layernorm/15_layernorm_residual.cu:59-103: mean = E[x],
// var = E[x^2] - mean^2, out = gamma * (x - mean) * rsqrt(var + eps) + beta.
// One workgroup per row; in place (out == x) is allowed because every element
// is read and written by the same thread.
__global__ __launch_bounds__(256) void layernorm_kernel(int cols, const float* x,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta,
                                                        float* out, float eps) {
    const float* xr = x + (size_t)blockIdx.x * cols;
    float* orow = out + (size_t)blockIdx.x * cols;
    float s = 0.0f, s2 = 0.0f;
    for (int c = threadIdx.x; c < cols; c += 256) {
        const float v = xr[c];
        s += v;
        s2 = fmaf(v, v, s2);
    }
    s = wave_sum(s);
    s2 = wave_sum(s2);
    __shared__ float red[2][4];
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = s;
        red[1][threadIdx.x >> 6] = s2;
    }
    __syncthreads();
    s = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    s2 = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    const float mean = s / cols;
    const float var = s2 / cols - mean * mean;
    const float inv = rsqrtf(var + eps);
    for (int c = threadIdx.x; c < cols; c += 256)
        orow[c] = gamma[c] * (xr[c] - mean) * inv + beta[c];
}

// kernels/layernorm/15_embed.cu:4-21.
__global__ __launch_bounds__(256) void embedding_kernel(const int* __restrict__ ids, int seq_len,
                                                        int start_pos, int d,
                                                        const float* __restrict__ wte,
                                                        const float* __restrict__ wpe,
                                                        float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)seq_len * d) return;
    const int t = (int)(idx / d);
    const int i = (int)(idx - (size_t)t * d);
    out[idx] = wte[(size_t)ids[t] * d + i] + wpe[(size_t)(start_pos + t) * d + i];
}

__global__ __launch_bounds__(256) void embedding_batch_kernel(int B, const int* __restrict__ ids,
                                                              const int* __restrict__ positions,
                                                              int d, const float* __restrict__ wte,
                                                              const float* __restrict__ wpe,
                                                              float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)B * d) return;
    const int b = (int)(idx / d);
    const int i = (int)(idx - (size_t)b * d);
    out[idx] = wte[(size_t)ids[b] * d + i] + wpe[(size_t)positions[b] * d + i];
}

// src/gpt2_engine.cu:391-403: logits[r][j] = hidden[r] . wte[j].  Each 16-lane
// row owns one vocabulary row and streams it with 16-byte loads (the
// reference gives each thread a whole row, which does not coalesce).
template <int RT>
__global__ __launch_bounds__(256) void vocab_proj_kernel(int rows, const float* __restrict__ h,
                                                         const float* __restrict__ wte,
                                                         float* __restrict__ logits, int d,
                                                         int V) {
    const int lane = threadIdx.x & 63, li = lane & 15;
    const int j = blockIdx.x * 16 + (threadIdx.x >> 6) * 4 + (lane >> 4);
    const bool ok = j < V;
    float acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = 0.0f;
    if (ok) {
        const float* w = wte + (size_t)j * d;
#pragma unroll 4
        for (int k = li * 4; k < d; k += 64) {
            const float4 wv = *reinterpret_cast<const float4*>(w + k);
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int rr = r < rows ? r : rows - 1;
                const float4 hv = *reinterpret_cast<const float4*>(h + (size_t)rr * d + k);
                float a = acc[r];
                a = fmaf(wv.x, hv.x, a);
                a = fmaf(wv.y, hv.y, a);
                a = fmaf(wv.z, hv.z, a);
                a = fmaf(wv.w, hv.w, a);
                acc[r] = a;
            }
        }
    }
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const float t = row16_sum(acc[r]);
        if (li == r) mine = t;
    }
    if (ok && li < rows && li < RT) logits[(size_t)li * V + j] = mine;
}

// src/sampler.cu:10-14 on the device: first index of the maximum.
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ logits, int n,
                                                     int* __restrict__ out) {
    const float* x = logits + (size_t)blockIdx.x * n;
    float best = -FLT_MAX;
    int bi = n;  // sentinel larger than any index
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = x[i];
        if (v > best || (bi == n && v == best)) {
            best = v;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ob = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ob > best || (ob == best && oi < bi)) {
            best = ob;
            bi = oi;
        }
    }
    __shared__ float sb[4];
    __shared__ int si[4];
    if ((threadIdx.x & 63) == 0) {
        sb[threadIdx.x >> 6] = best;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w)
            if (sb[w] > best || (sb[w] == best && si[w] < bi)) {
                best = sb[w];
                bi = si[w];
            }
        out[blockIdx.x] = bi < n ? bi : 0;
    }
}

}  // namespace

void launch_layernorm(int rows, int cols, const float* x, const float* g, const float* b,
                      float* out, float eps, hipStream_t s) {
    if (rows == 0) return;
    layernorm_kernel<<<rows, 256, 0, s>>>(cols, x, g, b, out, eps);
}

void launch_embedding(const int* ids, int seq_len, int start_pos, int d, const float* wte,
                      const float* wpe, float* out, hipStream_t s) {
    const size_t total = (size_t)seq_len * d;
    if (total == 0) return;
    embedding_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(ids, seq_len, start_pos, d,
                                                                     wte, wpe, out);
}

void launch_embedding_batch(int B, const int* ids, const int* positions, int d,
                            const float* wte, const float* wpe, float* out, hipStream_t s) {
    const size_t total = (size_t)B * d;
    if (total == 0) return;
    embedding_batch_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(B, ids, positions, d,
                                                                           wte, wpe, out);
}

void launch_vocab_proj(int rows, const float* h, const float* wte, float* logits, int d, int V,
                       hipStream_t s) {
    if (rows == 0 || V == 0) return;
    const unsigned blocks = (unsigned)((V + 15) / 16);
    if (rows == 1)
        vocab_proj_kernel<1><<<blocks, 256, 0, s>>>(rows, h, wte, logits, d, V);
    else
        vocab_proj_kernel<16><<<blocks, 256, 0, s>>>(rows, h, wte, logits, d, V);
}

void launch_argmax(int rows, const float* logits, int n, int* out, hipStream_t s) {
    if (rows == 0) return;
    argmax_kernel<<<rows, 256, 0, s>>>(logits, n, out);
}

}  // namespace ie
