/*
 * ie_engine.h — C ABI of the GPT-2 decode engine (ie_gpt2_engine.h), for
 * harnesses that cannot use the C++ class.  Mirrors GPT2Engine's constructor,
 * generate loop and InferenceMetrics (src/gpt2_engine.cuh:9-33,
 * include/gpt2_types.cuh:68-83 of the reference); batch, bf16 KV, INT8 LM head
 * and graph replay are extensions.  Functions return ie_status codes.
 */
#ifndef IE_ENGINE_H
#define IE_ENGINE_H

#include <stdint.h>

#include "ie_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ie_engine ie_engine;

/* Backends (InferenceBackend in ie_gpt2_engine.h). */
#define IE_BACKEND_INT8 0 /* the INT8 decode hot path (reference CUSTOM_INT8) */
#define IE_BACKEND_FP32 1 /* vendor fp32 GEMMs (reference CUBLAS_FP32) */

/* InferenceMetrics without its `generating` flag. */
typedef struct {
    float ttft_ms, tpot_ms, itl_min_ms, itl_max_ms, itl_p95_ms, tps;
    int tokens_generated, max_tokens;
    float kv_cache_pct, vram_used_mb, vram_total_mb, mbu, end_to_end_ms;
} ie_metrics;

/* model_dir != NULL loads the reference on-disk format and ignores the
 * shape arguments; model_dir == NULL builds a random model of that shape.
 * fuse selects the fused decode step, prefill / prefill_chunk the prompt path,
 * backend IE_BACKEND_INT8 or IE_BACKEND_FP32 (GPT2EngineOptions). */
int ie_engine_create(ie_engine** out, const char* model_dir, int n_layers, int n_heads,
                     int d_model, int d_ff, int vocab_size, int max_seq_len,
                     unsigned long long seed, int max_batch, int kv_dtype,
                     int int8_lm_head, int use_graph, int fuse, int prefill,
                     int prefill_chunk, int backend);
int ie_engine_destroy(ie_engine* e);
int ie_engine_write_random_model(const char* dir, int n_layers, int n_heads, int d_model,
                                 int d_ff, int vocab_size, int max_seq_len,
                                 unsigned long long seed);
int ie_engine_reset(ie_engine* e);
/* Greedy generation for `batch` prompts of prompt_len ids (row-major).
 * out_tokens [batch, max_new] receives the ids, -1 past a sequence's end. */
int ie_engine_generate(ie_engine* e, int batch, int prompt_len, const int* prompts, int max_new,
                       int ignore_eos, int* out_tokens, ie_metrics* metrics);
/* GPT2Engine::generate for one prompt (src/gpt2_engine.cu:628-770):
 * greedy != 0 takes the argmax, else top-k sampling at `temperature` with
 * the reference's seeds (42, then 43, 44, ...).  Stops at <|endoftext|>
 * (50256) as the reference.  out_tokens [max_new] receives the ids, -1 past
 * the end; *n_out the count.  reset_kv != 0 starts a fresh session. */
int ie_engine_generate_one(ie_engine* e, int prompt_len, const int* prompt, int max_new,
                           float temperature, int top_k, int greedy, int reset_kv,
                           int* out_tokens, int* n_out, ie_metrics* metrics);
/* One decode step at the current position; optional host copies of the
 * logits [batch, vocab] and of the argmax ids [batch]. */
int ie_engine_step(ie_engine* e, int batch, const int* tokens, float* logits_host,
                   int* argmax_host);
/* Prefill of prompt_len tokens per sequence (tokens [batch, prompt_len])
 * at the current position; optional host copies of the last token's logits
 * [batch, vocab] and of their argmax ids [batch]. */
int ie_engine_prefill(ie_engine* e, int batch, int prompt_len, const int* tokens,
                      float* logits_host, int* argmax_host);
int ie_engine_session_tokens(ie_engine* e);
/* cfg[7] = n_layers, n_heads, d_model, d_ff, vocab_size, max_seq_len, d_head. */
int ie_engine_config(ie_engine* e, int* cfg);
double ie_engine_step_bytes(ie_engine* e, int batch);

#ifdef __cplusplus
}
#endif
#endif
