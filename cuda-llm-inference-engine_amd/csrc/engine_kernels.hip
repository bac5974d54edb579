// engine_kernels.hip — small kernels private to the decode-step engine.
//
// qkv_split_append fuses the reference's qkv_split_kernel and
// kv_cache_write_kernel (src/gpt2_engine.cu:292-315, 321-346): from the QKV
// projection [B, 3d] (per token Q || K || V, HF c_attn order) it writes Q
// [B, d] contiguously for attention, appends K and V at each sequence's
// current position through its block-table row, and sets the attention
// context length pos + 1.  advance moves every sequence one position on.
// Positions and token ids live in device memory, so a captured decode step
// replays without host involvement.  prefill_qkv_write does the same split and
// append for a prompt chunk (P tokens per sequence, src/gpt2_engine.cu:466-
// 481 with seq_len = P).  ln_quant is prefill's LayerNorm and per-row
// quantizer in one launch.
#include <stdexcept>

#include "device_util.h"
#include "gemv_common.h"
#include "ie_internal.h"

namespace ie {
namespace {

template <typename KV>
__device__ __forceinline__ KV to_kv(float x);
template <>
__device__ __forceinline__ float to_kv<float>(float x) { return x; }
template <>
__device__ __forceinline__ uint16_t to_kv<uint16_t>(float x) { return f32_to_bf16_rne(x); }

template <typename KV>
__global__ __launch_bounds__(256) void qkv_split_append_kernel(
    int B, int d, const float* __restrict__ qkv, const int* __restrict__ positions,
    const int* __restrict__ block_table, int nbps, int block_size, float* __restrict__ Q,
    KV* __restrict__ kc, KV* __restrict__ vc, int* __restrict__ ctx_lens) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= B * d) return;
    const int b = idx / d, i = idx - (idx / d) * d;
    const float* row = qkv + (size_t)b * 3 * d;
    const int pos = positions[b];
    const int blk = pos / block_size;
    const size_t slot = (size_t)block_table[(size_t)b * nbps + blk] * block_size + (pos - blk * block_size);
    Q[idx] = row[i];
    kc[slot * d + i] = to_kv<KV>(row[d + i]);
    vc[slot * d + i] = to_kv<KV>(row[2 * d + i]);
    if (i == 0) ctx_lens[b] = pos + 1;
}

__global__ void advance_kernel(int B, int* __restrict__ positions) {
    const int b = blockIdx.x * 64 + threadIdx.x;
    if (b < B) positions[b] += 1;
}

// Prefill: row m = b * P + t of the QKV projection is token t of sequence b,
// at position start + t.
template <typename KV>
__global__ __launch_bounds__(256) void prefill_qkv_write_kernel(
    int B, int P, int start, int d, const float* __restrict__ qkv, const int* __restrict__ block_table,
    int nbps, int block_size, float* __restrict__ Q, KV* __restrict__ kc, KV* __restrict__ vc) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)B * P * d) return;
    const int m = (int)(idx / d), i = (int)(idx - (size_t)m * d);
    const int b = m / P, pos = start + (m - b * P);
    const float* row = qkv + (size_t)m * 3 * d;
    const int blk = pos / block_size;
    const size_t slot = (size_t)block_table[(size_t)b * nbps + blk] * block_size + (pos - blk * block_size);
    Q[idx] = row[i];
    kc[slot * d + i] = to_kv<KV>(row[d + i]);
    vc[slot * d + i] = to_kv<KV>(row[2 * d + i]);
}

// The cache slot of every row of a prompt chunk (the addressing of
// prefill_qkv_write), for the QKV GEMM that stores K/V itself.
__global__ __launch_bounds__(256) void prefill_row_slots_kernel(int B, int P, int start,
                                                                const int* __restrict__ block_table, int nbps,
                                                                int block_size, int* __restrict__ row_slot) {
    const int m = blockIdx.x * 256 + threadIdx.x;
    if (m >= B * P) return;
    const int b = m / P, pos = start + (m - b * P);
    const int blk = pos / block_size;
    row_slot[m] = block_table[(size_t)b * nbps + blk] * block_size + (pos - blk * block_size);
}

// Prefill's LayerNorm (src/gpt2_engine.cu:455) and the per-row quantizer
// of the GEMM input after it (:460) in one launch: one wave per row, the
// row's float4s loaded once, normalised and quantized in registers
// (stage_row: the LayerNorm's and then the quantizer's arithmetic, so the
// bytes and scale equal those of ie_layernorm followed by
// ie_quantize_fp32_to_int8), and the fp32 LayerNorm output never written.
template <int K>
__global__ __launch_bounds__(256) void ln_quant_kernel(int rows, const float* __restrict__ x,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, float eps,
                                                       int32_t* __restrict__ q, float* __restrict__ scales) {
    const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (row >= rows) return;  // whole waves
    GemvFusion f;
    f.gamma = gamma;
    f.beta = beta;
    f.eps = eps;
    stage_row<K, kSrcLnQuant>(x + (size_t)row * K, f, q + (size_t)row * (K / 4), scales + row,
                              (int)(threadIdx.x & 63));
}

// The fp32 comparison backend's epilogue after a vendor fp32 GEMM g [M, N]
// (src/gpt2_engine.cu:349-390): bias, bias + tanh-GELU, or bias + residual,
// in the reference's order of additions (C += bias + residual).  out may be
// residual (the hidden state updated in place).
__global__ __launch_bounds__(256) void fp32_epilogue_kernel(int M, int N, const float* __restrict__ g,
                                                            const float* __restrict__ bias,
                                                            const float* residual, float* out, int epi) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)M * N) return;
    const int j = (int)(idx % (size_t)N);
    const float c = g[idx];
    if (epi == IE_EPI_BIAS_GELU) {
        const float v = c + bias[j];
        const float v3 = v * v * v;
        out[idx] = 0.5f * v * (1.0f + tanhf(0.7978845608f * fmaf(0.044715f, v3, v)));
    } else if (epi == IE_EPI_BIAS_RESIDUAL) {
        out[idx] = c + (bias[j] + residual[idx]);
    } else {
        out[idx] = c + bias[j];
    }
}

__global__ void set_positions_kernel(int B, int pos, int* __restrict__ positions, int* __restrict__ ctx_lens) {
    const int b = blockIdx.x * 64 + threadIdx.x;
    if (b < B) {
        positions[b] = pos;
        ctx_lens[b] = pos;
    }
}

}  // namespace

void launch_qkv_split_append(int B, int d, const float* qkv, const int* positions,
                             const int* block_table, int nbps, int block_size, float* Q,
                             void* kc, void* vc, int kv_dtype, int* ctx_lens, hipStream_t s) {
    const unsigned blocks = (unsigned)((B * d + 255) / 256);
    if (kv_dtype == IE_KV_BF16)
        qkv_split_append_kernel<uint16_t><<<blocks, 256, 0, s>>>(
            B, d, qkv, positions, block_table, nbps, block_size, Q, static_cast<uint16_t*>(kc),
            static_cast<uint16_t*>(vc), ctx_lens);
    else
        qkv_split_append_kernel<float><<<blocks, 256, 0, s>>>(
            B, d, qkv, positions, block_table, nbps, block_size, Q, static_cast<float*>(kc),
            static_cast<float*>(vc), ctx_lens);
}

void launch_advance(int B, int* positions, hipStream_t s) {
    advance_kernel<<<(B + 63) / 64, 64, 0, s>>>(B, positions);
}

void launch_prefill_qkv_write(int B, int P, int start, int d, const float* qkv,
                              const int* block_table, int nbps, int block_size, float* Q,
                              void* kc, void* vc, int kv_dtype, hipStream_t s) {
    const size_t total = (size_t)B * P * d;
    if (total == 0) return;
    const unsigned blocks = (unsigned)((total + 255) / 256);
    if (kv_dtype == IE_KV_BF16)
        prefill_qkv_write_kernel<uint16_t><<<blocks, 256, 0, s>>>(
            B, P, start, d, qkv, block_table, nbps, block_size, Q, static_cast<uint16_t*>(kc),
            static_cast<uint16_t*>(vc));
    else
        prefill_qkv_write_kernel<float><<<blocks, 256, 0, s>>>(
            B, P, start, d, qkv, block_table, nbps, block_size, Q, static_cast<float*>(kc),
            static_cast<float*>(vc));
}

void launch_prefill_row_slots(int B, int P, int start, const int* block_table, int nbps, int block_size,
                              int* row_slot, hipStream_t s) {
    const int rows = B * P;
    if (rows == 0) return;
    prefill_row_slots_kernel<<<(rows + 255) / 256, 256, 0, s>>>(B, P, start, block_table, nbps, block_size,
                                                                 row_slot);
}

bool ln_quant_supported(int cols) { return cols == 768; }

void launch_ln_quant(int rows, int cols, const float* x, const float* gamma, const float* beta, float eps,
                     int32_t* q, float* scales, hipStream_t s) {
    if (rows == 0) return;
    if (cols != 768) throw std::logic_error("launch_ln_quant: no kernel for this width");
    ln_quant_kernel<768><<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(rows, x, gamma, beta, eps, q, scales);
}

void launch_fp32_epilogue(int M, int N, const float* g, const float* bias, const float* residual, float* out,
                          int epi, hipStream_t s) {
    const size_t total = (size_t)M * N;
    if (total == 0) return;
    fp32_epilogue_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(M, N, g, bias, residual, out, epi);
}

void launch_set_positions(int B, int pos, int* positions, int* ctx_lens, hipStream_t s) {
    set_positions_kernel<<<(B + 63) / 64, 64, 0, s>>>(B, pos, positions, ctx_lens);
}

}  // namespace ie
