// engine_capi.cpp — extern "C" wrapper of GPT2Engine (include/ie_engine.h).
// Exceptions from the engine become IE_ERR_* codes with the message kept for
// ie_last_error().
#include "ie_engine.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <exception>
#include <vector>

#include "../csrc/ie_internal.h"
#include "ie_gpt2_engine.h"

struct ie_engine {
    GPT2Engine* eng;
};

namespace {
template <typename F>
int guarded(const char* fn, F&& f) {
    try {
        f();
        return IE_OK;
    } catch (const std::exception& ex) {
        return ie::fail(IE_ERR_INVALID, "%s: %s", fn, ex.what());
    }
}

GPT2Config make_cfg(int L, int H, int d, int ff, int V, int S) {
    GPT2Config c;
    c.n_layers = L;
    c.n_heads = H;
    c.d_model = d;
    c.d_ff = ff;
    c.vocab_size = V;
    c.max_seq_len = S;
    c.d_head = H > 0 ? d / H : 0;
    return c;
}

void to_c(const InferenceMetrics& m, ie_metrics* o) {
    if (!o) return;
    o->ttft_ms = m.ttft_ms;
    o->tpot_ms = m.tpot_ms;
    o->itl_min_ms = m.itl_min_ms;
    o->itl_max_ms = m.itl_max_ms;
    o->itl_p95_ms = m.itl_p95_ms;
    o->tps = m.tps;
    o->tokens_generated = m.tokens_generated;
    o->max_tokens = m.max_tokens;
    o->kv_cache_pct = m.kv_cache_pct;
    o->vram_used_mb = m.vram_used_mb;
    o->vram_total_mb = m.vram_total_mb;
    o->mbu = m.mbu;
    o->end_to_end_ms = m.end_to_end_ms;
}
}  // namespace

extern "C" {

int ie_engine_create(ie_engine** out, const char* model_dir, int n_layers, int n_heads, int d_model,
                     int d_ff, int vocab_size, int max_seq_len, unsigned long long seed, int max_batch,
                     int kv_dtype, int int8_lm_head, int use_graph, int fuse, int prefill,
                     int prefill_chunk, int backend) {
    if (!out) return ie::fail(IE_ERR_INVALID, "ie_engine_create: out is null");
    *out = nullptr;
    GPT2EngineOptions opt;
    opt.max_batch = max_batch;
    opt.kv_dtype = kv_dtype;
    opt.int8_lm_head = int8_lm_head != 0;
    opt.use_graph = use_graph != 0;
    opt.fuse = fuse != 0;
    opt.prefill = prefill != 0;
    opt.prefill_chunk = prefill_chunk;
    if (prefill_chunk < 0) return ie::fail(IE_ERR_INVALID, "ie_engine_create: prefill_chunk=%d", prefill_chunk);
    if (backend != IE_BACKEND_INT8 && backend != IE_BACKEND_FP32)
        return ie::fail(IE_ERR_INVALID, "ie_engine_create: backend=%d", backend);
    opt.backend = backend == IE_BACKEND_FP32 ? InferenceBackend::CUBLAS_FP32 : InferenceBackend::CUSTOM_INT8;
    return guarded("ie_engine_create", [&] {
        GPT2Engine* e = model_dir ? new GPT2Engine(std::string(model_dir), opt)
                                  : new GPT2Engine(make_cfg(n_layers, n_heads, d_model, d_ff, vocab_size,
                                                            max_seq_len),
                                                   seed, opt);
        *out = new ie_engine{e};
    });
}

int ie_engine_destroy(ie_engine* e) {
    if (!e) return IE_OK;
    delete e->eng;
    delete e;
    return IE_OK;
}

int ie_engine_write_random_model(const char* dir, int n_layers, int n_heads, int d_model, int d_ff,
                                 int vocab_size, int max_seq_len, unsigned long long seed) {
    if (!dir) return ie::fail(IE_ERR_INVALID, "ie_engine_write_random_model: dir is null");
    return guarded("ie_engine_write_random_model", [&] {
        GPT2Engine::write_random_model(dir, make_cfg(n_layers, n_heads, d_model, d_ff, vocab_size, max_seq_len),
                                       seed);
    });
}

int ie_engine_reset(ie_engine* e) {
    if (!e) return ie::fail(IE_ERR_INVALID, "ie_engine_reset: null engine");
    return guarded("ie_engine_reset", [&] { e->eng->reset_session(); });
}

int ie_engine_generate(ie_engine* e, int batch, int prompt_len, const int* prompts, int max_new,
                       int ignore_eos, int* out_tokens, ie_metrics* metrics) {
    if (!e || !prompts || batch <= 0 || prompt_len <= 0 || max_new < 0)
        return ie::fail(IE_ERR_INVALID, "ie_engine_generate: bad arguments");
    return guarded("ie_engine_generate", [&] {
        std::vector<std::vector<int>> p(batch), out;
        for (int b = 0; b < batch; ++b) p[b].assign(prompts + (size_t)b * prompt_len, prompts + (size_t)(b + 1) * prompt_len);
        InferenceMetrics m;
        e->eng->generate_batch(p, max_new, out, m, ignore_eos != 0);
        if (out_tokens)
            for (int b = 0; b < batch; ++b)
                for (int t = 0; t < max_new; ++t)
                    out_tokens[(size_t)b * max_new + t] = t < (int)out[b].size() ? out[b][t] : -1;
        to_c(m, metrics);
    });
}

int ie_engine_generate_one(ie_engine* e, int prompt_len, const int* prompt, int max_new, float temperature,
                           int top_k, int greedy, int reset_kv, int* out_tokens, int* n_out, ie_metrics* metrics) {
    if (!e || !prompt || prompt_len <= 0 || max_new < 0)
        return ie::fail(IE_ERR_INVALID, "ie_engine_generate_one: bad arguments");
    if (!greedy && !(temperature > 0.0f))
        return ie::fail(IE_ERR_INVALID, "ie_engine_generate_one: temperature must be > 0 when sampling");
    return guarded("ie_engine_generate_one", [&] {
        std::vector<int> p(prompt, prompt + prompt_len), got;
        InferenceMetrics m;
        e->eng->generate(p, max_new, temperature, top_k, greedy != 0, [&](int t) { got.push_back(t); }, m,
                         reset_kv != 0);
        if (out_tokens)
            for (int t = 0; t < max_new; ++t) out_tokens[t] = t < (int)got.size() ? got[t] : -1;
        if (n_out) *n_out = (int)got.size();
        to_c(m, metrics);
    });
}

namespace {
// Host copies of the logits [batch, V] left by the last step or prefill, and
// their first-maximum ids.
void fetch_logits(GPT2Engine* eng, int batch, float* logits_host, int* argmax_host) {
    const int V = eng->config().vocab_size;
    std::vector<float> l;
    float* dst = logits_host;
    if (!dst && argmax_host) {
        l.resize((size_t)batch * V);
        dst = l.data();
    }
    if (!dst) return;
    hipError_t er = hipMemcpy(dst, eng->logits_device(), sizeof(float) * (size_t)batch * V, hipMemcpyDeviceToHost);
    if (er != hipSuccess) throw std::runtime_error(hipGetErrorString(er));
    if (argmax_host)
        for (int b = 0; b < batch; ++b) {
            const float* r = dst + (size_t)b * V;
            argmax_host[b] = (int)(std::max_element(r, r + V) - r);
        }
}
}  // namespace

int ie_engine_prefill(ie_engine* e, int batch, int prompt_len, const int* tokens, float* logits_host,
                      int* argmax_host) {
    if (!e || !tokens || batch <= 0 || prompt_len <= 0)
        return ie::fail(IE_ERR_INVALID, "ie_engine_prefill: bad arguments");
    return guarded("ie_engine_prefill", [&] {
        e->eng->prefill(tokens, batch, prompt_len);
        fetch_logits(e->eng, batch, logits_host, argmax_host);
    });
}

int ie_engine_step(ie_engine* e, int batch, const int* tokens, float* logits_host, int* argmax_host) {
    if (!e || !tokens) return ie::fail(IE_ERR_INVALID, "ie_engine_step: bad arguments");
    return guarded("ie_engine_step", [&] {
        e->eng->step(tokens, batch);
        fetch_logits(e->eng, batch, logits_host, argmax_host);
    });
}

int ie_engine_session_tokens(ie_engine* e) { return e ? e->eng->session_tokens() : -1; }

int ie_engine_config(ie_engine* e, int* cfg) {
    if (!e || !cfg) return ie::fail(IE_ERR_INVALID, "ie_engine_config: bad arguments");
    const GPT2Config& c = e->eng->config();
    const int v[7] = {c.n_layers, c.n_heads, c.d_model, c.d_ff, c.vocab_size, c.max_seq_len, c.d_head};
    std::memcpy(cfg, v, sizeof(v));
    return IE_OK;
}

double ie_engine_step_bytes(ie_engine* e, int batch) { return e ? e->eng->step_bytes(batch) : 0.0; }

}  // extern "C"
