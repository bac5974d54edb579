/*
 * ie_amd.h — C ABI of the MI355X (gfx950) quantized decode hot path.
 *
 * Plain C: device pointers, sizes and a stream handle.  Every entry point
 * validates its arguments on the host before any HIP call and returns an
 * ie_status; ie_last_error() gives the message of the calling thread's last
 * failure.  Kernels are asynchronous on the given stream (NULL = the null
 * stream); all pointers are caller-owned device memory, nothing here allocates
 * device memory after ie_init().
 *
 * Reference interfaces replaced (paths inside the reference repository):
 *   ie_quantize_fp32_to_int8  run_quantize_fp32_to_int8
 *                             kernels/quantization/14_int8_gemm.cuh:20-23
 *   ie_int8_gemm              run_int8_gemm / _bias / _bias_gelu / _bias_residual
 *                             kernels/quantization/14_int8_gemm.cuh:27-64
 *                             (epilogue = I8Epilogue, 14_int8_gemm.cuh:36)
 *   ie_decode_attn            run_decode_attn  kernels/decode/13_decode_attn.cuh:192-199
 *   ie_prefill_attn           run_flash_attn_v2 as the engine's prefill uses it
 *                             (src/gpt2_engine.cu:484-493), over the paged cache
 *   ie_flash_attn             run_flash_attn_v2
 *                             kernels/flash_attention/10_flash_attn_v2.cuh:7-9
 *   ie_kv_cache_write         kv_cache_write_kernel / GPT2Engine::kv_cache_append
 *                             src/gpt2_engine.cu:321-346, 431-445
 *   ie_layernorm              run_layernorm  kernels/layernorm/15_layernorm_residual.cu:120-130
 *   ie_layernorm_residual     run_layernorm_residual
 *                             kernels/layernorm/15_layernorm_residual.cuh:7-15, .cu:6-57,105-118
 *   ie_embedding              run_embedding  kernels/layernorm/15_embed.cu:24-30
 *   ie_vocab_proj             run_vocab_proj src/gpt2_engine.cu:391-410
 *   ie_argmax                 sample_argmax  src/sampler.cu:10-14 (device-side)
 *   ie_topk                   sample_top_k's partial_sort, src/sampler.cu:20-26
 *                             (device-side; only k pairs reach the host)
 *   ie_top_k_draw             sample_top_k's softmax and draw, src/sampler.cu:28-44
 * The reference's own C++ signatures are kept, unchanged, in ie_compat.h.
 */
#ifndef IE_AMD_H
#define IE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same object as hipStream_t; NULL selects the null stream. */
typedef struct ihipStream_t* ie_stream_t;

typedef enum {
    IE_OK = 0,
    IE_ERR_INVALID = 1,      /* bad argument (null pointer, size, alignment) */
    IE_ERR_UNSUPPORTED = 2,  /* valid in principle, not implemented (e.g. d=96) */
    IE_ERR_WORKSPACE = 3,    /* workspace too small for the requested split plan */
    IE_ERR_HIP = 4           /* HIP runtime reported an error */
} ie_status;

/* Epilogues, in the order of the reference's I8Epilogue
 * (kernels/quantization/14_int8_gemm.cuh:36).  IE_EPI_I32 writes the raw
 * int32 accumulators (no reference counterpart; used for bit-exact checks). */
typedef enum {
    IE_EPI_PLAIN = 0,
    IE_EPI_BIAS = 1,
    IE_EPI_BIAS_GELU = 2,
    IE_EPI_BIAS_RESIDUAL = 3,
    IE_EPI_I32 = 4
} ie_epilogue;

/* GEMM kernel selection: AUTO picks the dot4 GEMV for M <= 16 and the MFMA
 * tile kernel otherwise. */
typedef enum { IE_PATH_AUTO = 0, IE_PATH_GEMV = 1, IE_PATH_MFMA = 2 } ie_gemm_path;

/* KV-cache element type.  BF16 caches hold raw bfloat16 bit patterns. */
typedef enum { IE_KV_F32 = 0, IE_KV_BF16 = 1 } ie_kv_dtype;

/* Maximum split count of the reference plan (DA_MAX_SPLITS,
 * kernels/decode/13_decode_attn.cuh:12) and of ie_decode_attn. */
#define IE_DA_REF_MAX_SPLITS 16
#define IE_DA_MAX_SPLITS 256

const char* ie_last_error(void);
int ie_version(void);
/* Optional: checks that the current device is gfx950, makes the small pinned
 * host buffer of the compat samplers (sample_argmax / sample_top_k in
 * ie_compat.h), so nothing allocates afterwards, and looks up the current
 * device's address of ie_decode_attn_noalloc's scratch; calling it first also
 * keeps the HIP runtime's one-time start-up out of timed regions. */
int ie_init(void);

/* Per-row symmetric quantizer: scales[r] = max|x_r|/127 (1 for a zero row),
 * output_packed[r][i] = 4 int8 of row r, columns 4i..4i+3, little-endian.
 * cols % 4 == 0.  Bit-exact with kernels/quantization/14_int8_gemm.cu:10-60. */
int ie_quantize_fp32_to_int8(int rows, int cols, const float* input,
                             int32_t* output_packed, float* scales,
                             ie_stream_t stream);

/* C[M,N] = epilogue(sum_k A[m,k] * BT[n,k], scale_A[m], scale_B[n], ...).
 * A_packed [M, K/4], BT_packed [N, K/4] int8x4 words; K % 4 == 0.
 * bias [N] for epilogues 1-3, residual [M,N] for 3 (may alias C). */
int ie_int8_gemm(int M, int N, int K, const int32_t* A_packed,
                 const int32_t* BT_packed, const float* scale_A,
                 const float* scale_B, int epilogue, const float* bias,
                 const float* residual, float* C, ie_stream_t stream);

/* As ie_int8_gemm with an explicit kernel path; with IE_EPI_I32, C receives
 * int32 accumulators (scale pointers may be NULL). */
int ie_int8_gemm_ex(int M, int N, int K, const int32_t* A_packed,
                    const int32_t* BT_packed, const float* scale_A,
                    const float* scale_B, int epilogue, const float* bias,
                    const float* residual, void* C, int path,
                    ie_stream_t stream);

/* Split plan.  num_splits <= 0 gives the reference rule
 * clamp(ceil(max_ctx/bs)/4, 1, 16) (kernels/decode/13_decode_attn.cu:63-65). */
int ie_decode_num_splits(int max_context_len, int block_size, int num_splits);
/* Bytes of workspace for [B, H_q, num_splits, d+2] fp32 partials. */
size_t ie_decode_attn_workspace_bytes(int B, int H_q, int d, int num_splits);

/* Split-K paged decode attention for one query token per sequence.
 * Q [B,H_q,d] fp32; k_cache/v_cache [num_phys_blocks, block_size, H_kv, d] in
 * kv_dtype; block_table [B, num_blocks_per_seq] int32; context_lens [B] int32
 * (device) with every entry <= max_context_len (host); O [B,H_q,d] fp32.
 * d in {64,128}; H_q/H_kv in {1,2,4,8}.  workspace_bytes must cover
 * ie_decode_attn_workspace_bytes(B, H_q, d, plan splits). */
int ie_decode_attn(int B, int H_q, int H_kv, int d, const float* Q,
                   const void* k_cache, const void* v_cache, int kv_dtype,
                   const int* block_table, const int* context_lens,
                   int max_context_len, int block_size, int num_blocks_per_seq,
                   float* O, float* workspace, size_t workspace_bytes,
                   int num_splits, ie_stream_t stream);

/* ie_decode_attn without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * split partials go to a scratch array that the library holds on each GPU
 * until the process ends: IE_DECODE_SCRATCH_BYTES, so B * H_q * splits *
 * (d + 2) * 4 must fit (else IE_ERR_WORKSPACE, outputs untouched).  Nothing
 * is allocated and the scratch needs no clearing (every split slot is written
 * before the merge reads it), but all calls on one GPU share it: calls that
 * overlap in time on that GPU (other streams, other host threads) race.
 * Same kernels, split plan and results as ie_decode_attn. */
#define IE_DECODE_SCRATCH_BYTES ((size_t)32 << 20)
int ie_decode_attn_noalloc(int B, int H_q, int H_kv, int d, const float* Q,
                           const void* k_cache, const void* v_cache,
                           int kv_dtype, const int* block_table,
                           const int* context_lens, int max_context_len,
                           int block_size, int num_blocks_per_seq, float* O,
                           int num_splits, ie_stream_t stream);

/* Causal attention of a prompt chunk over the paged cache: P query tokens per
 * sequence, token t of sequence b at position start_pos + t, whose K/V (and
 * those of every earlier position) are already in the cache; each attends to
 * cached positions 0 .. start_pos + t.  Q and O are token-major
 * [B, P, H_q, d] fp32 (the QKV projection's layout); caches, block table and
 * kv_dtype as ie_decode_attn, with start_pos + P <= num_blocks_per_seq *
 * block_size.  d in {64,128}; H_q a multiple of H_kv. */
int ie_prefill_attn(int B, int P, int H_q, int H_kv, int d, const float* Q,
                    const void* k_cache, const void* v_cache, int kv_dtype,
                    const int* block_table, int num_blocks_per_seq,
                    int block_size, int start_pos, float* O,
                    ie_stream_t stream);

/* FlashAttention forward over contiguous fp32 Q, K, V, O [B, H, N, d]
 * (run_flash_attn_v2, kernels/flash_attention/10_flash_attn_v2.cuh:7-9):
 * softmax(Q K^T / sqrt(d)) V per (b, h), keys j <= i when causal.  d in
 * {64,128}; O must not overlap Q, K or V. */
int ie_flash_attn(int B, int H, int N, int d, const float* Q, const float* K,
                  const float* V, float* O, int causal, ie_stream_t stream);

/* Writes K/V rows [seq_len, n_heads, d_head] fp32 for positions
 * start_pos..start_pos+seq_len-1 of one sequence into the paged caches
 * (fp32 or bf16, rounded to nearest even). */
int ie_kv_cache_write(const float* K_src, const float* V_src, void* k_cache,
                      void* v_cache, int kv_dtype, const int* block_table,
                      int seq_len, int start_pos, int n_heads, int d_head,
                      int block_size, ie_stream_t stream);

/* Batched decode append: sequence b writes its one new token (K_src/V_src
 * [B, n_heads, d_head]) at position positions[b] (device int32) through row b
 * of block_table [B, num_blocks_per_seq]. */
int ie_kv_cache_append_batch(int B, const float* K_src, const float* V_src,
                             void* k_cache, void* v_cache, int kv_dtype,
                             const int* block_table, int num_blocks_per_seq,
                             const int* positions, int n_heads, int d_head,
                             int block_size, ie_stream_t stream);

/* Support operations of the decode step. */
int ie_layernorm(int rows, int cols, const float* x, const float* gamma,
                 const float* beta, float* out, float eps, ie_stream_t stream);
/* residual_out = x + residual (one fp32 add per element), out =
 * LayerNorm(residual_out) with ie_layernorm's arithmetic (so out equals
 * ie_layernorm of residual_out bit for bit).  [rows, cols] row-major; out and
 * residual_out may alias x, residual or each other, as in the reference. */
int ie_layernorm_residual(int rows, int cols, const float* x,
                          const float* residual, const float* gamma,
                          const float* beta, float* out, float* residual_out,
                          float eps, ie_stream_t stream);
int ie_embedding(const int* token_ids, int seq_len, int start_pos,
                 int d_model, const float* wte, const float* wpe, float* out,
                 ie_stream_t stream);
/* Batched embedding for one decode token per sequence: positions[b]. */
int ie_embedding_batch(int B, const int* token_ids, const int* positions,
                       int d_model, const float* wte, const float* wpe,
                       float* out, ie_stream_t stream);
int ie_vocab_proj(int rows, const float* hidden, const float* wte,
                  float* logits, int d, int V, ie_stream_t stream);
/* out_idx[r] = first index of the maximum of logits[r, 0:n]. */
int ie_argmax(int rows, const float* logits, int n, int* out_idx,
              ie_stream_t stream);

/* Largest k selectable by ie_topk. */
#define IE_TOPK_MAX 1024
/* The k largest of logits[r, 0:n] for each row r, 1 <= k <= min(n,
 * IE_TOPK_MAX): out_vals[r, 0:k] by value descending, equal values by index
 * ascending, out_idx[r, 0:k] their indices (device pointers).  NaN logits
 * are not supported. */
int ie_topk(int rows, const float* logits, int n, int k, float* out_vals,
            int* out_idx, ie_stream_t stream);
/* Host side of sample_top_k: from k >= 1 sorted (value, index) pairs, such
 * as ie_topk's (host memory), p_i = expf((v_i - v_0) / temperature) normalised,
 * and the first i whose running sum exceeds r = rand() / RAND_MAX, where the
 * generator is reseeded with srand(seed) whenever seed differs from the
 * previous call's (the reference's rule).  The library keeps that generator
 * state privately (glibc's rand() algorithm), so the process-wide rand() is
 * untouched.  *token = the chosen index. */
int ie_top_k_draw(const float* vals, const int* idx, int k, float temperature,
                  unsigned int seed, int* token);

/* Host-side check of token ids before they reach a device embedding
 * (ie_embedding* index wte rows without a bound, as run_embedding does,
 * kernels/layernorm/15_embed.cu:4-21): IE_OK when every ids[i], i < n, lies
 * in [0, vocab_size); otherwise IE_ERR_INVALID naming the first offender.
 * No HIP call.  The engine runs it on every host token it is given. */
int ie_check_token_ids(int n, const int* ids, int vocab_size);

#ifdef __cplusplus
}
#endif
#endif
