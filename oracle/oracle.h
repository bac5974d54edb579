/*
 * oracle.h — CPU restatement of the reference's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or, for cpu_baseline, as the reported CPU figure).  The product library
 * (libie_amd.so) never links, loads or calls anything here.
 *
 * Every function names the reference file:line it restates.  Paths are
 * relative to the reference repository root (kernels/, src/, tests/, python/).
 *
 * Parity pins (each function is checked by tests/test_oracle_*.py against
 * something other than a retyping of its own formula):
 *   orc_rng_*                 libc rand() itself (ctypes), same seed/order
 *   orc_quantize_fp32_to_int8 hand-derived known answers (ties to even,
 *                             argmax -> +-127, zero row -> scale 1, byte
 *                             order), |q*scale - x| <= scale/2, numpy
 *   orc_int8_gemm_i32         numpy int64 matmul (library routine), identity
 *                             and all-ones closed forms, K=0..8 brute force
 *   orc_int8_gemm (epilogues) fp64 GEMM within 0.012*sqrt(K) (the reference's
 *                             own acceptance test on its own srand(42) inputs),
 *                             torch gelu(approximate='tanh') in fp64
 *   orc_decode_attn*          numpy/torch fp64 softmax attention on the
 *                             gathered cache, ctx=1 -> V0, constant V, block
 *                             table permutation invariance, split invariance
 *   orc_kv_cache_write        closed-form index map (numpy fancy indexing)
 *   orc_layernorm             torch layer_norm in fp64
 *   orc_layernorm_residual    numpy fp32 add, torch layer_norm in fp64 of the
 *                             sum; not LN(x) + residual nor LN(residual); the
 *                             reference test's own srand(42) cases and bound
 *   orc_embedding, orc_vocab_proj, orc_argmax
 *                             numpy gather / matmul / argmax
 *   orc_topk                  Python sorted() by (-value, index) brute force,
 *                             numpy argsort, k = n is a permutation
 *   orc_top_k_draw            k = 1 and a cold temperature pick idx[0]; r just
 *                             below / above a hand-computed cumulative bound;
 *                             pick frequencies over 20000 seeds against the
 *                             softmax probabilities (chi-square)
 *   Ties in orc_topk: the reference's partial_sort leaves their order
 *   unspecified, so that order is parity unpinned against the reference.
 */
#ifndef IE_ORACLE_H
#define IE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- thread control for the CPU baseline (OpenMP) ---- */
void orc_set_threads(int n);
int orc_get_threads(void);

/* ---- glibc TYPE_3 additive generator with private state ----
 * Reproduces the reference tests' inputs: srand(42) then
 * (float)rand() / RAND_MAX * 2.0f - 1.0f
 * (tests/test_int8_gemm.cu:24-28, tests/test_decode_attention.cu:66-73). */
void* orc_rng_new(unsigned seed);
void orc_rng_free(void* rng);
int orc_rng_next(void* rng);                 /* one raw rand() value */
void orc_rng_uniform(void* rng, float* out, long n);
void orc_rng_uniform_pair(void* rng, float* a, float* b, long n); /* interleaved draws */

/* ---- K14 quantizer: kernels/quantization/14_int8_gemm.cu:10-60 ---- */
int orc_quantize_fp32_to_int8(int rows, int cols, const float* input,
                              int32_t* output_packed, float* scales);

/* ---- K14 integer core: 14_int8_gemm.cu:96-140 (sum of dp4a) ---- */
int orc_int8_gemm_i32(int M, int N, int K, const int32_t* A_packed,
                      const int32_t* BT_packed, int32_t* acc);

/* ---- K14 with epilogue: 14_int8_gemm.cu:142-169, epi = I8Epilogue order
 * (14_int8_gemm.cuh:36): 0 Plain, 1 BiasOnly, 2 BiasGELU, 3 BiasResidual ---- */
int orc_int8_gemm(int M, int N, int K, const int32_t* A_packed,
                  const int32_t* BT_packed, const float* scale_A,
                  const float* scale_B, int epilogue, const float* bias,
                  const float* residual, float* C);

/* fp64 GEMM of the unquantized fp32 operands, C = A[M,K] @ B[K,N]
 * (stands in for the K06 fp32 oracle of tests/test_int8_gemm.cu:41). */
void orc_gemm_f64(int M, int N, int K, const float* A, const float* B, double* C);

/* ---- K13 split plan: kernels/decode/13_decode_attn.cu:63-65 ---- */
int orc_decode_num_splits(int max_context_len, int block_size);

/* ---- K13 decode attention, reference split plan, fp64 accumulation ----
 * 13_decode_attn.cuh:30-189 (pass 1) and 13_decode_attn.cu:10-53 (pass 2),
 * with the intended semantics for empty splits (they contribute nothing).
 * kv_dtype 0 = fp32 cache, 1 = bf16 cache (raw uint16 bit patterns).
 * num_splits <= 0 selects the reference's rule. */
int orc_decode_attn(int B, int H_q, int H_kv, int d, const float* Q,
                    const void* k_cache, const void* v_cache, int kv_dtype,
                    const int* block_table, const int* context_lens,
                    int max_context_len, int block_size,
                    int num_blocks_per_seq, int num_splits, float* O);

/* Same plan in fp32 with the reference's per-block token interleave over 8
 * warps (13_decode_attn.cuh:89-131) and warp merge (:150-176); expf replaces
 * the device fast exponential. */
int orc_decode_attn_f32(int B, int H_q, int H_kv, int d, const float* Q,
                        const void* k_cache, const void* v_cache, int kv_dtype,
                        const int* block_table, const int* context_lens,
                        int max_context_len, int block_size,
                        int num_blocks_per_seq, int num_splits, float* O);

/* ---- paged KV write: src/gpt2_engine.cu:321-346 ---- */
int orc_kv_cache_write(const float* K_src, const float* V_src, float* k_cache,
                       float* v_cache, const int* block_table, int seq_len,
                       int start_pos, int n_heads, int d_head, int block_size);

/* ---- support ops for the decode step ---- */
/* kernels/layernorm/15_layernorm_residual.cu:59-103 */
void orc_layernorm(int rows, int cols, const float* x, const float* gamma,
                   const float* beta, float* out, float eps);
/* kernels/layernorm/15_layernorm_residual.cu:6-57 */
void orc_layernorm_residual(int rows, int cols, const float* x, const float* residual,
                            const float* gamma, const float* beta, float* out,
                            float* residual_out, float eps);
/* kernels/layernorm/15_embed.cu:4-21 */
void orc_embedding(const int* token_ids, int seq_len, int start_pos,
                   int d_model, const float* wte, const float* wpe, float* out);
/* src/gpt2_engine.cu:391-403 */
void orc_vocab_proj(const float* hidden, const float* wte, float* logits,
                    int d, int V);
/* src/sampler.cu:10-14: first index of the maximum */
int orc_argmax(const float* logits, int n);

/* ---- top-k sampler: src/sampler.cu:16-45 ----
 * orc_topk: the k largest of each row, value descending, equal values by
 * index ascending.  orc_rand_unit: (float)rand() / RAND_MAX (:37).
 * orc_top_k_draw: the index drawn at threshold r from sorted pairs. */
int orc_topk(int rows, int n, int k, const float* logits, float* vals, int* idx);
float orc_rand_unit(void* rng);
int orc_top_k_draw(const float* vals, const int* idx, int k, float temperature, float r);

#ifdef __cplusplus
}
#endif
#endif
