/*
 * ie_compat.h — the reference's own C++ launch signatures, unchanged, so code
 * written against the reference (its engine, tests and benchmarks) links
 * against libie_amd.so without edits.
 *
 *   kernels/quantization/14_int8_gemm.cuh:20-64   quantizer, INT8 GEMM, epilogues
 *   kernels/decode/13_decode_attn.cuh:12,192-199   DA_MAX_SPLITS, run_decode_attn
 *   kernels/flash_attention/10_flash_attn_v2.cuh   run_flash_attn_v2
 *   kernels/quantization/14_int8_gemm.cuh:11-16    I8_BM ... I8_NTHREADS
 *   kernels/layernorm/15_layernorm_residual.cuh    run_layernorm_residual, run_layernorm
 *   kernels/layernorm/15_embed.cuh                 run_embedding
 *   include/sampler.cuh                            sample_argmax, sample_top_k
 *
 * As in the reference: void return, caller-owned device pointers, the null
 * stream, asynchronous.  Unlike the reference, invalid arguments never reach a
 * kernel: the call prints the reason to stderr, leaves the outputs untouched
 * and records it for ie_last_error().  For stream selection, status codes,
 * bf16 KV or more than DA_MAX_SPLITS splits, use ie_amd.h.
 */
#ifndef IE_COMPAT_H
#define IE_COMPAT_H

#include <cstdint>

#include "ie_amd.h"

/* The reference K14 kernel's tile constants (its 64x64 tile, 16-byte K step,
 * 4x4 thread tile, 256 threads), kept for callers that print or size with
 * them, e.g. the reference's INT8 bench header line.  They describe the
 * reference's kernel, not this library's tiling (MFMA tiles chosen per
 * shape), and size nothing a caller passes to it. */
#define I8_BM 64
#define I8_BN 64
#define I8_BK 16
#define I8_TM 4
#define I8_TN 4
#define I8_NTHREADS 256

/* Workspace sizing used by callers of run_decode_attn:
 * [B, H_q, DA_MAX_SPLITS, d + 2] floats (src/gpt2_engine.cu:156). */
#define DA_MAX_SPLITS 16

void run_quantize_fp32_to_int8(int rows, int cols, const float* input,
                               int32_t* output_packed, float* scales);

void run_int8_gemm(int M, int N, int K, const int32_t* A_packed,
                   const int32_t* BT_packed, const float* scale_A,
                   const float* scale_B, float* C);

enum class I8Epilogue { Plain, BiasOnly, BiasGELU, BiasResidual };

void run_int8_gemm_bias(int M, int N, int K, const int32_t* A_packed,
                        const int32_t* BT_packed, const float* scale_A,
                        const float* scale_B, const float* bias, float* C);

void run_int8_gemm_bias_gelu(int M, int N, int K, const int32_t* A_packed,
                             const int32_t* BT_packed, const float* scale_A,
                             const float* scale_B, const float* bias, float* C);

void run_int8_gemm_bias_residual(int M, int N, int K, const int32_t* A_packed,
                                 const int32_t* BT_packed, const float* scale_A,
                                 const float* scale_B, const float* bias,
                                 const float* residual, float* C);

void run_decode_attn(int B, int H_q, int H_kv, int d, const float* Q,
                     const float* k_cache, const float* v_cache,
                     const int* block_table, const int* context_lens,
                     int max_context_len, int block_size,
                     int num_blocks_per_seq, float* O, float* workspace);

/* kernels/flash_attention/10_flash_attn_v2.cuh:7-9: Q, K, V, O [B, H, N, d]
 * fp32, scale 1/sqrt(d).  d in {64,128}.  O must not overlap Q, K or V (an
 * overlapping call is reported and leaves O untouched). */
void run_flash_attn_v2(int B, int H, int N, int d, const float* Q,
                       const float* K, const float* V, float* O, bool causal);

/* out = LayerNorm(x + residual), residual_out = x + residual; out and
 * residual_out may alias the inputs. */
void run_layernorm_residual(int rows, int cols, const float* x,
                            const float* residual, const float* gamma,
                            const float* beta, float* out, float* residual_out,
                            float eps = 1e-5f);

void run_layernorm(int rows, int cols, const float* x, const float* gamma,
                   const float* beta, float* out, float eps = 1e-5f);

void run_embedding(const int* token_ids, int seq_len, int start_pos,
                   int d_model, const float* wte, const float* wpe, float* out);

/* Samplers over device logits [vocab_size] (src/sampler.cu).  The argmax and
 * the top-k selection run on the device and write their 4 bytes (argmax) or
 * k value/index pairs (top-k) straight into pinned host memory instead of the
 * whole row coming back; k is clamped to vocab_size as in the reference, and
 * k above IE_TOPK_MAX takes the reference's route (the whole row to the host,
 * a partial sort).  The draw follows the reference's float arithmetic and its
 * srand(seed) / rand() rule with a generator private to the library (see
 * ie_top_k_draw).  Their small pinned buffer is made by ie_init(), or by the
 * first call when ie_init() was not called, and kept.  -1 on error. */
int sample_argmax(const float* d_logits, int vocab_size);
int sample_top_k(const float* d_logits, int vocab_size, int k,
                 float temperature, unsigned int seed);

#endif
