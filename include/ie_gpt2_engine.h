/*
 * ie_gpt2_engine.h — GPT-2 decode engine over the INT8 decode hot path (C++).
 *
 * Mirrors the reference engine's public surface (src/gpt2_engine.cuh:9-33,
 * include/gpt2_types.cuh:6-83): GPT2Config, QuantWeight, InferenceMetrics,
 * GPT2Engine(model_dir), generate(prompt, max_new, temperature, top_k, greedy,
 * callback, metrics, reset_kv), reset_session(), session_tokens(), config().
 * The model directory uses the reference's on-disk format
 * (python/export_gpt2.py:73-167): config.json, wte.bin, wpe.bin, ln_f_*.bin,
 * layer_%02d/{ln1,ln2}_{gamma,beta}.bin, {qkv,out,ffn_up,ffn_down}_{weight,
 * scale,bias}.bin with weights int8x4-packed [N, K/4] and per-row scales [N].
 *
 * Extensions with no reference counterpart: a batch of sequences decoded
 * together (generate_batch), bf16 KV cache, an INT8 LM head, a decode step
 * captured once as a HIP graph and replayed per token, and chunked prefill
 * that also serves continuation prompts.
 */
#ifndef IE_GPT2_ENGINE_H
#define IE_GPT2_ENGINE_H

#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "ie_amd.h"

/* include/gpt2_types.cuh:6-14 */
struct GPT2Config {
    int n_layers;
    int n_heads;
    int d_model;
    int d_ff;
    int vocab_size;
    int max_seq_len;
    int d_head;
};

/* include/gpt2_types.cuh:16-21: int8x4-packed [N, K/4] and per-row scales [N]. */
struct QuantWeight {
    int32_t* packed;
    float* scale;
    int N;
    int K;
};

/* include/gpt2_types.cuh:68-83; mbu uses MI355X's 8 TB/s and the bytes the
 * decode step actually streams. */
struct InferenceMetrics {
    float ttft_ms;
    float tpot_ms;
    float itl_min_ms;
    float itl_max_ms;
    float itl_p95_ms;
    float tps;
    int tokens_generated;
    int max_tokens;
    float kv_cache_pct;
    float vram_used_mb;
    float vram_total_mb;
    float mbu;
    float end_to_end_ms;
    bool generating;
};

/* include/gpt2_types.cuh:43.  CUBLAS_FP32 keeps the reference's enumerator
 * name so its callers compile unchanged; here that backend runs the four
 * linears as vendor fp32 GEMMs (rocBLAS sgemm on the exporter's
 * {name}_weight_fp32.bin [K, N] weights, src/gpt2_engine.cu:530-610) with
 * this library's LayerNorm, paged KV cache, decode attention and LM head:
 * the reference's fp32 comparison point for the INT8 path. */
enum class InferenceBackend { CUSTOM_INT8, CUBLAS_FP32 };

struct GPT2EngineOptions {
    int max_batch = 1;          /* sequences decoded together */
    int kv_dtype = IE_KV_F32;   /* IE_KV_F32 (reference) or IE_KV_BF16 */
    bool int8_lm_head = false;  /* reference: fp32 head over tied wte */
    bool use_graph = true;      /* replay one captured decode step per token */
    /* Fused decode step: LayerNorm and the activation quantizer run inside
     * the GEMVs and QKV appends to the KV cache in its epilogue (GPT-2
     * widths d = 768, ff = 3072; other shapes use the unfused step). */
    bool fuse = true;
    /* Prompts run through prefill: M = sequences x tokens GEMMs and a causal
     * prefill attention over the paged cache (d_head 64 or 128; otherwise, or
     * when false, one decode step per prompt position). */
    bool prefill = true;
    int prefill_chunk = 0; /* tokens per sequence per prefill pass; 0 = 4096 / batch */
    /* CUBLAS_FP32: vendor fp32 GEMMs (needs the fp32 weight files, or a
     * random model); runs the unfused step without graph capture. */
    InferenceBackend backend = InferenceBackend::CUSTOM_INT8;
};

class GPT2Engine {
public:
    /* Loads a model directory in the reference format. */
    explicit GPT2Engine(const std::string& model_dir, GPT2EngineOptions opt = {});
    /* The reference's constructor (src/gpt2_engine.cuh:11-12). */
    GPT2Engine(const std::string& model_dir, InferenceBackend backend);
    /* Random-initialised model (weights and biases N(0, 0.02), LayerNorm
     * gamma 1, beta 0), quantized per row exactly as the exporter does. */
    GPT2Engine(const GPT2Config& cfg, uint64_t seed, GPT2EngineOptions opt = {});
    ~GPT2Engine();
    GPT2Engine(const GPT2Engine&) = delete;
    GPT2Engine& operator=(const GPT2Engine&) = delete;

    /* src/gpt2_engine.cu:629-783 for one sequence.  Greedy uses a device
     * argmax (first index of the maximum, as std::max_element); otherwise
     * top-k sampling with the reference's host procedure. */
    void generate(const std::vector<int>& prompt_tokens, int max_new_tokens, float temperature,
                  int top_k, bool greedy, std::function<void(int token_id)> token_callback,
                  InferenceMetrics& metrics, bool reset_kv = true);

    /* Greedy decoding of B = prompts.size() <= max_batch sequences with equal
     * prompt lengths; out[b] receives the generated ids.  With ignore_eos the
     * loop always runs max_new_tokens steps (benchmarking). */
    void generate_batch(const std::vector<std::vector<int>>& prompts, int max_new_tokens,
                        std::vector<std::vector<int>>& out, InferenceMetrics& metrics,
                        bool ignore_eos = false);

    void reset_session();
    int session_tokens() const;
    const GPT2Config& config() const;

    /* Prefill of `len` tokens for each of the first `batch` sequences
     * (tokens[b * len + t]) at the current position; logits of every
     * sequence's last token are left on the device. */
    void prefill(const int* tokens, int batch, int len);

    /* One decode step for the first `batch` sequences at the current position
     * (tokens on the host); logits of every sequence are left on the device. */
    void step(const int* tokens, int batch);
    const float* logits_device() const;
    /* Bytes the next decode step reads from HBM (weights, LM head, and the
     * KV of its pos + 1 cached tokens) for `batch` sequences.  The MBU of a
     * generate call uses the mean context of its timed steps instead. */
    double step_bytes(int batch) const;

    /* Writes a random-initialised model in the reference's on-disk format,
     * with the exporter's fp32 [K, N] copies of the linear weights
     * ({name}_weight_fp32.bin, python/export_gpt2.py:48-57). */
    static void write_random_model(const std::string& dir, const GPT2Config& cfg, uint64_t seed);

    struct Impl;

private:
    std::unique_ptr<Impl> impl_;
};

#endif
