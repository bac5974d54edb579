// kv_cache.hip — paged KV-cache writes.
//
// Layout (src/gpt2_engine.cu:321-346 of the reference): cache
// [num_phys_blocks][block_size][n_heads][d_head]; logical position pos of a
// sequence lives in physical block block_table[pos / block_size] at slot
// pos % block_size.  bf16 caches store round-to-nearest-even bfloat16.
#include "device_util.h"
#include "ie_internal.h"

namespace ie {
namespace {

template <typename KV>
__device__ __forceinline__ KV cvt(float x);
template <>
__device__ __forceinline__ float cvt<float>(float x) { return x; }
template <>
__device__ __forceinline__ uint16_t cvt<uint16_t>(float x) { return f32_to_bf16_rne(x); }

template <typename KV>
__global__ __launch_bounds__(256) void kv_write_kernel(const float* __restrict__ K,
                                                       const float* __restrict__ V,
                                                       KV* __restrict__ kc, KV* __restrict__ vc,
                                                       const int* __restrict__ bt, int seq_len,
                                                       int start_pos, int H, int dh, int bs) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t row = (size_t)H * dh;
    if (idx >= (size_t)seq_len * row) return;
    const int t = (int)(idx / row);
    const size_t rem = idx - (size_t)t * row;
    const int pos = start_pos + t;
    const int blk = pos / bs;
    const size_t dst = ((size_t)bt[blk] * bs + (pos - blk * bs)) * row + rem;
    kc[dst] = cvt<KV>(K[idx]);
    vc[dst] = cvt<KV>(V[idx]);
}

template <typename KV>
__global__ __launch_bounds__(256) void kv_append_batch_kernel(
    int B, const float* __restrict__ K, const float* __restrict__ V, KV* __restrict__ kc,
    KV* __restrict__ vc, const int* __restrict__ bt, int nbps, const int* __restrict__ positions,
    int H, int dh, int bs) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t row = (size_t)H * dh;
    if (idx >= (size_t)B * row) return;
    const int b = (int)(idx / row);
    const size_t rem = idx - (size_t)b * row;
    const int pos = positions[b];
    const int blk = pos / bs;
    const size_t dst = ((size_t)bt[(size_t)b * nbps + blk] * bs + (pos - blk * bs)) * row + rem;
    kc[dst] = cvt<KV>(K[idx]);
    vc[dst] = cvt<KV>(V[idx]);
}

}  // namespace

void launch_kv_write(const float* K, const float* V, void* kc, void* vc, int kv_dtype,
                     const int* bt, int seq_len, int start_pos, int H, int dh, int bs,
                     hipStream_t s) {
    const size_t total = (size_t)seq_len * H * dh;
    if (total == 0) return;
    const unsigned blocks = (unsigned)((total + 255) / 256);
    if (kv_dtype == IE_KV_BF16)
        kv_write_kernel<uint16_t><<<blocks, 256, 0, s>>>(
            K, V, static_cast<uint16_t*>(kc), static_cast<uint16_t*>(vc), bt, seq_len,
            start_pos, H, dh, bs);
    else
        kv_write_kernel<float><<<blocks, 256, 0, s>>>(K, V, static_cast<float*>(kc),
                                                      static_cast<float*>(vc), bt, seq_len,
                                                      start_pos, H, dh, bs);
}

void launch_kv_append_batch(int B, const float* K, const float* V, void* kc, void* vc,
                            int kv_dtype, const int* bt, int nbps, const int* positions,
                            int H, int dh, int bs, hipStream_t s) {
    const size_t total = (size_t)B * H * dh;
    if (total == 0) return;
    const unsigned blocks = (unsigned)((total + 255) / 256);
    if (kv_dtype == IE_KV_BF16)
        kv_append_batch_kernel<uint16_t><<<blocks, 256, 0, s>>>(
            B, K, V, static_cast<uint16_t*>(kc), static_cast<uint16_t*>(vc), bt, nbps,
            positions, H, dh, bs);
    else
        kv_append_batch_kernel<float><<<blocks, 256, 0, s>>>(
            B, K, V, static_cast<float*>(kc), static_cast<float*>(vc), bt, nbps, positions, H,
            dh, bs);
}

}  // namespace ie
