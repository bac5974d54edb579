// ie_internal.h — shared declarations between the C ABI (capi.cpp) and the
// kernel translation units.  Launchers assume their arguments were validated.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "ie_amd.h"

namespace ie {

// Records a failure message for ie_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Maps a HIP error after a launch to IE_ERR_HIP with a message.
int check_launch(const char* what);

// ---- quantizer (quant.hip) ----
void launch_quantize(int rows, int cols, const float* in, int32_t* packed,
                     float* scales, hipStream_t s);

// ---- INT8 GEMM ----
// Where a prefill QKV projection's outputs go when the GEMM stores them
// itself (launch_gemm_i8_qkv_route), as prefill_qkv_write moves them: output
// column n < d of row m goes to q[m * d + n], column d + i (2d + i) to
// element i of the K (V) cache row of slot row_slot[m] (bf16 rounded to
// nearest even when kv_dtype is IE_KV_BF16).  row_slot comes from
// launch_prefill_row_slots, once per prompt chunk (every layer's cache has
// the same slots).
struct QkvRoute {
    float* q = nullptr;
    void* kc = nullptr;
    void* vc = nullptr;
    int kv_dtype = IE_KV_F32;
    const int* row_slot = nullptr;
    int d = 0;
};

struct GemmArgs {
    int M, N, K;
    const int32_t* A;
    const int32_t* BT;
    const float* sA;
    const float* sB;
    const float* bias;
    const float* residual;
    void* C;
    int epi;
    QkvRoute route{};  // epi == kEpiQKVRoute only
};
// The bias epilogue with the output routed by GemmArgs::route (C unused).
constexpr int kEpiQKVRoute = 9;
// The prefill QKV projection: the bias-epilogue INT8 GEMM [M, 3d] on the
// small-grid or tile kernel, as launch_gemm_i8_mfma would choose, its
// outputs stored by a.route (gemm_i8_mfma.hip).
void launch_gemm_i8_qkv_route(const GemmArgs& a, hipStream_t s);
// dot4 GEMV for small M (gemv_i8.hip); M in [1, 16].
void launch_gemv_i8(const GemmArgs& a, hipStream_t s);

// Decode-step fusions of the small-M GEMV (gemv_i8.hip), used by the engine.
// The activation operand is built inside the GEMV from fp32 rows instead of
// being read as int8 (src 1: the per-row quantizer of quant.hip, same
// arithmetic; src 2: LayerNorm first), and the QKV epilogue writes Q and
// appends K/V to the paged cache instead of storing [M, 3d].
enum { kSrcInt8 = 0, kSrcQuant = 1, kSrcLnQuant = 2 };
constexpr int kEpiQKV = 8;  // bias epilogue routed to Q / K cache / V cache
struct GemvFusion {
    int src = kSrcInt8;
    const float* x = nullptr;      // [M, K] fp32 rows (src 1, 2)
    const float* gamma = nullptr;  // LayerNorm weight and bias [K] (src 2)
    const float* beta = nullptr;
    float eps = 1e-5f;
    // kEpiQKV: N = 3d; Q [M, d]; K/V of token positions[m] of sequence m go
    // to slot table[m * nbps + pos / block_size] * block_size + pos % block_size
    // of the [slots, d] caches; ctx_lens[m] = pos + 1.
    float* q = nullptr;
    void* kc = nullptr;
    void* vc = nullptr;
    int kv_dtype = IE_KV_F32;
    const int* positions = nullptr;
    const int* table = nullptr;
    int nbps = 0;
    int block_size = 16;
    int* ctx_lens = nullptr;
    // launch_qkv_attn only: with ids set, row m of x is not read but built
    // as wte[ids[m]] + wpe[positions[m]] (the embedding, same arithmetic as
    // embedding_batch_kernel) and stored to x.
    const int* ids = nullptr;
    const float* wte = nullptr;
    const float* wpe = nullptr;
    // launch_qkv_attn only: read the cache with non-temporal loads (a step's
    // cache stream larger than the caches keep beside the weights)
    bool kv_stream = false;
};
// The engine's QKV projection + decode attention in one launch, one
// workgroup per (sequence, head) (qkv_attn.hip): f as for the kEpiQKV GEMV
// with src kSrcLnQuant (x, LayerNorm gamma/beta), a one-split plan; O [B, d]
// receives the attention output.  Bit-identical to launch_gemv_fused(QKV)
// followed by launch_decode_attn with one split (with f.ids set, to the
// embedding kernel followed by those two).
bool qkv_attn_supported(int d_model, int n_heads, int d_head, int block_size);
void launch_qkv_attn(int B, int H, const int32_t* BT, const float* sB, const float* bias, const GemvFusion& f,
                     float* O, hipStream_t s);
// Whether launch_gemv_fused has a kernel for this combination (M <= 16).
bool gemv_fused_supported(int M, int K, int src, int epi);
void launch_gemv_fused(const GemmArgs& a, const GemvFusion& f, hipStream_t s);
// MFMA tile GEMM (gemm_i8_mfma.hip); any M.
void launch_gemm_i8_mfma(const GemmArgs& a, hipStream_t s);
// 256x256-tile MFMA GEMM for large M, N (gemm_i8_mfma256.hip).
bool gemm_i8_big_applies(const GemmArgs& a);
void launch_gemm_i8_big(const GemmArgs& a, hipStream_t s);
// Write-dominated shapes (K == 768, M <= 1024, wide N; gemm_i8_wide.hip).
bool gemm_i8_wide_applies(const GemmArgs& a);
void launch_gemm_i8_wide(const GemmArgs& a, hipStream_t s);
// LDS-tiled MFMA GEMM for prefill-sized problems (gemm_i8_tile.hip): tile
// shape BM * 1000 + BN chosen for a problem, applicability, launch.
int gemm_i8_tile_shape(const GemmArgs& a);
bool gemm_i8_tile_applies(const GemmArgs& a);
void launch_gemm_i8_tile(const GemmArgs& a, hipStream_t s);
// Register-streamed MFMA GEMM for mid-size problems (gemm_i8_stream.hip).
bool gemm_i8_stream_applies(const GemmArgs& a);
void launch_gemm_i8_stream(const GemmArgs& a, hipStream_t s);
// One thread per output; any K % 4 == 0 and any alignment (gemv_i8.hip).
void launch_gemm_i8_generic(const GemmArgs& a, hipStream_t s);
constexpr int kGemvMaxM = 16;

// ---- decode attention (decode_attn.hip) ----
struct DecodeArgs {
    int B, H_q, H_kv, d;
    const float* Q;
    const void* k_cache;
    const void* v_cache;
    int kv_dtype;
    const int* block_table;
    const int* context_lens;
    int block_size;
    int num_blocks_per_seq;
    int num_splits;        // plan: splits per (b, head)
    int blocks_per_split;  // plan: KV blocks per split
    float* O;
    float* workspace;      // [B, H_q, num_splits, d + 2]
};
void launch_decode_attn(const DecodeArgs& a, hipStream_t s);
// Host-side validation shared by ie_decode_attn and ie_decode_attn_noalloc
// (capi.cpp): everything but the workspace; on IE_OK, *splits is the plan's
// split count and *need_bytes its workspace size (0 when B == 0).
int check_decode_attn(int B, int H_q, int H_kv, int d, const float* Q, const void* k_cache, const void* v_cache,
                      int kv_dtype, const int* block_table, const int* context_lens, int max_context_len,
                      int block_size, int num_blocks_per_seq, const float* O, int num_splits, size_t* need_bytes,
                      int* splits);
// Looks up (once per device) the address of ie_decode_attn_noalloc's scratch
// array on the current device (decode_attn_noalloc.hip); called by ie_init.
int decode_scratch_init();

// Compute units of the current device (gemv_i8.hip).
int num_cus();

// ---- prefill attention (prefill_attn.hip) ----
// paged: Q/O [B, P, H_q, d], K/V = the paged caches (kv_dtype), query t at
// position start_pos + t attending to cached positions 0 .. start_pos + t.
// !paged: Q/K/V/O contiguous fp32 [B, H, P, d] (H_q = H_kv), start_pos 0.
struct PrefillArgs {
    int B, P, H_q, H_kv, d;
    const float* Q;
    const void* k;
    const void* v;
    int kv_dtype;
    bool paged;
    const int* block_table;
    int num_blocks_per_seq;
    int block_size;
    int start_pos;
    bool causal;
    float* O;
};
void launch_prefill_attn(const PrefillArgs& a, hipStream_t s);

// ---- KV cache (kv_cache.hip) ----
void launch_kv_write(const float* K, const float* V, void* kc, void* vc,
                     int kv_dtype, const int* bt, int seq_len, int start_pos,
                     int H, int dh, int bs, hipStream_t s);
void launch_kv_append_batch(int B, const float* K, const float* V, void* kc,
                            void* vc, int kv_dtype, const int* bt, int nbps,
                            const int* positions, int H, int dh, int bs,
                            hipStream_t s);

// ---- decode-step engine kernels (engine_kernels.hip) ----
void launch_qkv_split_append(int B, int d, const float* qkv, const int* positions,
                             const int* block_table, int nbps, int block_size, float* Q,
                             void* kc, void* vc, int kv_dtype, int* ctx_lens, hipStream_t s);
void launch_advance(int B, int* positions, hipStream_t s);
// Prefill chunk of P tokens per sequence at positions start .. start+P-1:
// from QKV rows [B*P, 3d] (row b*P + t) writes Q [B*P, d] and appends K/V.
void launch_prefill_qkv_write(int B, int P, int start, int d, const float* qkv,
                              const int* block_table, int nbps, int block_size, float* Q,
                              void* kc, void* vc, int kv_dtype, hipStream_t s);
// positions[b] = ctx_lens[b] = pos for every sequence.
void launch_set_positions(int B, int pos, int* positions, int* ctx_lens, hipStream_t s);
// LayerNorm of rows x cols fp32 then the per-row int8 quantizer, in one
// launch, the bytes and scales of ie_layernorm + ie_quantize_fp32_to_int8
// (engine_kernels.hip); only for widths where ln_quant_supported.
bool ln_quant_supported(int cols);
// row_slot[m] for the rows m = b * P + t of a prompt chunk (token t of
// sequence b at position start + t): its cache slot table[b * nbps + pos /
// block_size] * block_size + pos % block_size (engine_kernels.hip).
void launch_prefill_row_slots(int B, int P, int start, const int* block_table, int nbps, int block_size,
                              int* row_slot, hipStream_t s);
void launch_ln_quant(int rows, int cols, const float* x, const float* gamma, const float* beta, float eps,
                     int32_t* q, float* scales, hipStream_t s);
// fp32 comparison backend: out = epilogue(g) for epi in {BIAS, BIAS_GELU,
// BIAS_RESIDUAL}, g [M, N] the vendor GEMM's output (out may alias residual).
void launch_fp32_epilogue(int M, int N, const float* g, const float* bias, const float* residual, float* out,
                          int epi, hipStream_t s);

// ---- support ops (support.hip) ----
void launch_layernorm(int rows, int cols, const float* x, const float* g,
                      const float* b, float* out, float eps, hipStream_t s);
// residual_out = x + res, out = LayerNorm(residual_out); any aliasing allowed.
void launch_layernorm_residual(int rows, int cols, const float* x, const float* res, const float* g,
                               const float* b, float* out, float* res_out, float eps, hipStream_t s);
void launch_embedding(const int* ids, int seq_len, int start_pos, int d,
                      const float* wte, const float* wpe, float* out,
                      hipStream_t s);
void launch_embedding_batch(int B, const int* ids, const int* positions, int d,
                            const float* wte, const float* wpe, float* out,
                            hipStream_t s);
void launch_vocab_proj(int rows, const float* h, const float* wte, float* logits,
                       int d, int V, hipStream_t s);
// The decode step's head in one launch (support.hip): final LayerNorm of the
// rows x [rows, d] (the standalone LayerNorm's bits), fp32 LM head over wte
// into logits [rows, V], each row's first-maximum index merged into
// keys[row], and the last workgroup (counter `done`) writes the token ids,
// clears keys and counter (both 0 before the first launch) and (advance)
// moves the positions on; with host_ids (pinned [2][B]) the ids also land in
// slot positions[b] & 1 there.
bool vocab_head_supported(int rows, int d);
void launch_vocab_head(int rows, const float* x, const float* gamma, const float* beta, float eps,
                       const float* wte, float* logits, int d, int V, unsigned long long* keys, unsigned* done,
                       int* tokens, int* positions, bool advance, int* host_ids, hipStream_t s);
void launch_argmax(int rows, const float* logits, int n, int* out,
                   hipStream_t s);

// ---- top-k sampler (sampler.hip, host/sampler.cpp) ----
constexpr int kTopkMax = 1024;  // largest k selected on the device
// Makes the pinned buffer of sample_argmax / sample_top_k (called by
// ie_init, so the compat samplers allocate nothing afterwards).
int compat_sampler_init();
// k above kTopkMax: the reference's own route (src/sampler.cu:18-26), the
// whole row to the host and a partial sort, equal values in index order,
// then the reference's draw; IE_OK or an error code (message set).
int host_top_k_token(const float* d_logits, int V, int k, float temperature, unsigned seed, hipStream_t s,
                     int* token);
void launch_topk(int rows, const float* logits, int n, int k, float* out_vals,
                 int* out_idx, hipStream_t s);

}  // namespace ie
