// gpt2_engine.cpp — GPT-2 decode engine over the INT8 decode hot path.
//
// The decode step follows the reference's GPT2Engine::forward_layer decode
// branch (src/gpt2_engine.cu:447-528) and generate loop (:629-783):
//   embed -> 12 x [LN1 -> quantize -> QKV GEMM+bias -> split/KV append ->
//   split-K paged decode attention -> quantize -> out GEMM+bias+residual ->
//   LN2 -> quantize -> up GEMM+bias+GELU -> quantize -> down GEMM+bias+
//   residual] -> final LN -> LM head -> argmax.
// Differences in mechanism, not in arithmetic: no device-to-device residual
// copies (the residual stream x is read by LayerNorm and updated in place by
// the residual epilogues); the QKV split and KV write are one kernel; block
// tables, positions and token ids live on the device and a captured HIP graph
// replays a whole step; argmax runs on the device and only B token ids come
// back per step (the reference copies all 50257 logits to the host).
#include "ie_gpt2_engine.h"

#include <hip/hip_runtime.h>
#include <sys/stat.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <numeric>
#include <random>
#include <sstream>
#include <stdexcept>

#include "../csrc/ie_internal.h"
#include "vendor_blas.h"

namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPC(x) hip_check((x), #x)

void ie_check(int st, const char* what) {
    if (st != IE_OK) throw std::runtime_error(std::string(what) + ": " + ie_last_error());
}
#define IEC(x) ie_check((x), #x)

// ---------------------------------------------------------------- host RNG
// SplitMix64 (Steele, Lea, Flood 2014) feeding Box-Muller normals; one stream
// per tensor so every tensor is reproducible on its own.
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
};

std::vector<float> normal(size_t n, float stddev, uint64_t seed) {
    std::vector<float> v(n);
    Rng r(seed);
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = r.uniform(), u2 = r.uniform();
        const double rad = std::sqrt(-2.0 * std::log(u1));
        v[i] = (float)(rad * std::cos(6.283185307179586 * u2)) * stddev;
        if (i + 1 < n) v[i + 1] = (float)(rad * std::sin(6.283185307179586 * u2)) * stddev;
    }
    return v;
}

// python/export_gpt2.py:10-40 (quantize_per_row): per-row symmetric int8 in
// float32 arithmetic, round half to even, little-endian packing.
void quantize_rows_host(const std::vector<float>& w, int rows, int cols, std::vector<int32_t>& packed,
                        std::vector<float>& scales) {
    packed.assign((size_t)rows * cols / 4, 0);
    scales.assign(rows, 1.0f);
    for (int r = 0; r < rows; ++r) {
        const float* x = w.data() + (size_t)r * cols;
        float m = 0.0f;
        for (int c = 0; c < cols; ++c) m = std::max(m, std::fabs(x[c]));
        const float scale = m > 0.0f ? m / 127.0f : 1.0f;
        const float inv = 1.0f / scale;
        scales[r] = scale;
        for (int i = 0; i < cols / 4; ++i) {
            uint32_t word = 0;
            for (int j = 0; j < 4; ++j) {
                float q = std::nearbyint(x[4 * i + j] * inv);
                q = std::min(std::max(q, -128.0f), 127.0f);
                word |= (uint32_t)(uint8_t)(int8_t)q << (8 * j);
            }
            packed[(size_t)r * (cols / 4) + i] = (int32_t)word;
        }
    }
}

// ---------------------------------------------------------------- model I/O
template <typename T>
std::vector<T> read_bin(const std::string& path, size_t count) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    std::vector<T> v(count);
    f.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(count * sizeof(T)));
    if ((size_t)f.gcount() != count * sizeof(T)) throw std::runtime_error("short file " + path);
    return v;
}

template <typename T>
void write_bin(const std::string& path, const std::vector<T>& v) {
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot write " + path);
    f.write(reinterpret_cast<const char*>(v.data()), (std::streamsize)(v.size() * sizeof(T)));
}

// src/gpt2_engine.cu:41-60: the config keys, read by name.
GPT2Config read_config(const std::string& path) {
    std::ifstream f(path);
    if (!f) throw std::runtime_error("cannot open " + path);
    std::stringstream ss;
    ss << f.rdbuf();
    const std::string s = ss.str();
    auto get = [&](const char* key) {
        const auto k = s.find(std::string("\"") + key + "\"");
        if (k == std::string::npos) throw std::runtime_error(std::string("config.json lacks ") + key);
        const auto c = s.find(':', k);
        return std::atoi(s.c_str() + c + 1);
    };
    GPT2Config c;
    c.n_layers = get("n_layers");
    c.n_heads = get("n_heads");
    c.d_model = get("d_model");
    c.d_ff = get("d_ff");
    c.vocab_size = get("vocab_size");
    c.max_seq_len = get("max_seq_len");
    c.d_head = get("d_head");
    return c;
}

void validate(const GPT2Config& c) {
    if (c.n_layers <= 0 || c.n_heads <= 0 || c.d_model <= 0 || c.d_ff <= 0 || c.vocab_size <= 0 ||
        c.max_seq_len <= 0 || c.d_head * c.n_heads != c.d_model)
        throw std::runtime_error("invalid GPT2Config");
    if (c.d_model % 16 || c.d_ff % 16) throw std::runtime_error("d_model and d_ff must be multiples of 16");
    if (c.d_head != 64 && c.d_head != 128) throw std::runtime_error("d_head must be 64 or 128");
}

// Host copy of every tensor, in the on-disk layout.
struct HostModel {
    GPT2Config cfg;
    std::vector<float> wte, wpe, lnf_g, lnf_b;
    struct Layer {
        std::vector<float> ln1_g, ln1_b, ln2_g, ln2_b, qkv_b, out_b, up_b, down_b;
        std::vector<float> qkv_s, out_s, up_s, down_s;
        std::vector<int32_t> qkv_w, out_w, up_w, down_w;
        // fp32 weights in the exporter's [K, N] layout (fp32 backend, writer)
        std::vector<float> qkv_f, out_f, up_f, down_f;
    };
    std::vector<Layer> layers;
};

// [rows, cols] -> [cols, rows]
std::vector<float> transpose(const std::vector<float>& a, int rows, int cols) {
    std::vector<float> t(a.size());
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) t[(size_t)c * rows + r] = a[(size_t)r * cols + c];
    return t;
}

// keep_fp32: also keep each linear's fp32 weights as the exporter's [K, N].
HostModel random_model(const GPT2Config& c, uint64_t seed, bool keep_fp32 = false) {
    validate(c);
    HostModel m;
    m.cfg = c;
    const int d = c.d_model, ff = c.d_ff;
    uint64_t tid = 0;
    auto nxt = [&](size_t n) { return normal(n, 0.02f, seed * 0x100000001B3ull + (++tid)); };
    m.wte = nxt((size_t)c.vocab_size * d);
    m.wpe = nxt((size_t)c.max_seq_len * d);
    m.lnf_g.assign(d, 1.0f);
    m.lnf_b.assign(d, 0.0f);
    m.layers.resize(c.n_layers);
    // weights drawn directly in the exporter's transposed [N=out, K=in] layout
    auto linear = [&](int N, int K, std::vector<int32_t>& w, std::vector<float>& s, std::vector<float>& f) {
        const std::vector<float> wt = nxt((size_t)N * K);
        quantize_rows_host(wt, N, K, w, s);
        if (keep_fp32) f = transpose(wt, N, K);
    };
    for (auto& L : m.layers) {
        L.ln1_g.assign(d, 1.0f);
        L.ln1_b.assign(d, 0.0f);
        L.ln2_g.assign(d, 1.0f);
        L.ln2_b.assign(d, 0.0f);
        linear(3 * d, d, L.qkv_w, L.qkv_s, L.qkv_f);
        L.qkv_b = nxt(3 * d);
        linear(d, d, L.out_w, L.out_s, L.out_f);
        L.out_b = nxt(d);
        linear(ff, d, L.up_w, L.up_s, L.up_f);
        L.up_b = nxt(ff);
        linear(d, ff, L.down_w, L.down_s, L.down_f);
        L.down_b = nxt(d);
    }
    return m;
}

// want_fp32: also read {name}_weight_fp32.bin [K, N] (python/export_gpt2.py:48-57).
HostModel load_model(const std::string& dir, bool want_fp32 = false) {
    HostModel m;
    m.cfg = read_config(dir + "/config.json");
    const GPT2Config& c = m.cfg;
    validate(c);
    const int d = c.d_model, ff = c.d_ff;
    m.wte = read_bin<float>(dir + "/wte.bin", (size_t)c.vocab_size * d);
    m.wpe = read_bin<float>(dir + "/wpe.bin", (size_t)c.max_seq_len * d);
    m.lnf_g = read_bin<float>(dir + "/ln_f_gamma.bin", d);
    m.lnf_b = read_bin<float>(dir + "/ln_f_beta.bin", d);
    m.layers.resize(c.n_layers);
    for (int i = 0; i < c.n_layers; ++i) {
        char ld[64];
        std::snprintf(ld, sizeof(ld), "/layer_%02d/", i);
        const std::string p = dir + ld;
        auto& L = m.layers[i];
        L.ln1_g = read_bin<float>(p + "ln1_gamma.bin", d);
        L.ln1_b = read_bin<float>(p + "ln1_beta.bin", d);
        L.ln2_g = read_bin<float>(p + "ln2_gamma.bin", d);
        L.ln2_b = read_bin<float>(p + "ln2_beta.bin", d);
        L.qkv_w = read_bin<int32_t>(p + "qkv_weight.bin", (size_t)3 * d * d / 4);
        L.qkv_s = read_bin<float>(p + "qkv_scale.bin", 3 * d);
        L.qkv_b = read_bin<float>(p + "qkv_bias.bin", 3 * d);
        L.out_w = read_bin<int32_t>(p + "out_weight.bin", (size_t)d * d / 4);
        L.out_s = read_bin<float>(p + "out_scale.bin", d);
        L.out_b = read_bin<float>(p + "out_bias.bin", d);
        L.up_w = read_bin<int32_t>(p + "ffn_up_weight.bin", (size_t)ff * d / 4);
        L.up_s = read_bin<float>(p + "ffn_up_scale.bin", ff);
        L.up_b = read_bin<float>(p + "ffn_up_bias.bin", ff);
        L.down_w = read_bin<int32_t>(p + "ffn_down_weight.bin", (size_t)d * ff / 4);
        L.down_s = read_bin<float>(p + "ffn_down_scale.bin", d);
        L.down_b = read_bin<float>(p + "ffn_down_bias.bin", d);
        if (want_fp32) {
            L.qkv_f = read_bin<float>(p + "qkv_weight_fp32.bin", (size_t)d * 3 * d);
            L.out_f = read_bin<float>(p + "out_weight_fp32.bin", (size_t)d * d);
            L.up_f = read_bin<float>(p + "ffn_up_weight_fp32.bin", (size_t)d * ff);
            L.down_f = read_bin<float>(p + "ffn_down_weight_fp32.bin", (size_t)ff * d);
        }
    }
    return m;
}

}  // namespace

// ==================================================================== Impl
struct GPT2Engine::Impl {
    GPT2Config cfg{};
    GPT2EngineOptions opt;
    hipStream_t stream = nullptr;
    std::vector<void*> allocs;

    float *wte = nullptr, *wpe = nullptr, *lnf_g = nullptr, *lnf_b = nullptr;
    struct Layer {
        float *ln1_g, *ln1_b, *ln2_g, *ln2_b, *qkv_b, *out_b, *up_b, *down_b;
        QuantWeight qkv, out, up, down;
        float *qkv_f = nullptr, *out_f = nullptr, *up_f = nullptr, *down_f = nullptr;  // fp32 backend
    };
    std::vector<Layer> layers;
    QuantWeight head{};  // INT8 LM head (quantized wte), optional

    // activations, [max_batch, ...]
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr, *h = nullptr;
    float *logits = nullptr;
    int32_t* act_q = nullptr;
    float* act_s = nullptr;
    // fp32 backend: the vendor GEMM and its output rows [max_batch, max(3d, ff)]
    bool fp32 = false;
    std::unique_ptr<ie::VendorSgemm> blas;
    float* gemm_out = nullptr;

    // paged KV cache: per layer [P, bs, H, dh]; row b of the block table maps
    // its nbps logical blocks to physical blocks b * nbps + i
    static constexpr int kBlock = 16;
    int nbps = 0, phys_blocks = 0;
    size_t layer_elems = 0;
    char *kc = nullptr, *vc = nullptr;
    int *block_table = nullptr, *positions = nullptr, *ctx_lens = nullptr, *tokens = nullptr;
    float* ws = nullptr;
    size_t ws_bytes = 0;
    // fused head: per-row argmax keys [max_batch], zero between steps
    unsigned long long* head_keys = nullptr;
    unsigned* head_done = nullptr;  // the fused head's finishing-workgroup counter
    // Attention split plan of the current step (set by run_step): the
    // max_context_len and split count handed to the split kernel, as
    // ie_decode_attn would be called with them.
    struct AttnPlan {
        int max_ctx = 0, splits = 1;
    };
    AttnPlan plan;
    bool fused = false;  // fused step kernels apply to this model
    bool qkv_attn = false;  // the fused step's one-launch QKV + attention applies

    int pos = 0;  // host mirror: tokens in every active sequence
    int* host_tokens = nullptr;  // pinned [max_batch]
    // Greedy decode keeps one step in flight ahead of the host (see
    // GreedyPipe): each step's ids land in ring slot (position % 2), pinned
    // [2][max_batch] (written by the fused head's finalize kernel, else
    // copied), and ring_ev[slot] marks their arrival.
    int* host_ring = nullptr;
    hipEvent_t ring_ev[2] = {nullptr, nullptr};
    // top-k sampler: k values then k indices, written by the kernel into
    // pinned host memory
    float* host_topk_buf = nullptr;

    // Prefill scratch [rows, ...], rows = sequences x chunk tokens, grown on
    // first use (the decode step never touches it).
    struct PrefillBufs {
        int rows = 0;
        float *x = nullptr, *xn = nullptr, *qkv = nullptr, *q = nullptr, *attn = nullptr, *h = nullptr;
        float* act_s = nullptr;
        int32_t* act_q = nullptr;
        float* gemm_out = nullptr;  // fp32 backend
        int* ids = nullptr;  // pinned host mirror in host_ids
        int* host_ids = nullptr;
        int* row_slot = nullptr;  // cache slot of each row of the chunk (prefill_qkv)
    } pf;
    std::vector<void*> pf_allocs;

    // One captured decode step per (batch, attention split count).
    std::map<std::pair<int, int>, hipGraphExec_t> graphs;

    template <typename T>
    T* dev(size_t count) {
        void* p = nullptr;
        HIPC(hipMalloc(&p, std::max<size_t>(count, 1) * sizeof(T)));
        allocs.push_back(p);
        return static_cast<T*>(p);
    }
    template <typename T>
    T* upload(const std::vector<T>& v) {
        T* p = dev<T>(v.size());
        HIPC(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
        return p;
    }
    QuantWeight upload_q(const std::vector<int32_t>& w, const std::vector<float>& s, int N, int K) {
        QuantWeight q;
        q.packed = upload(w);
        q.scale = upload(s);
        q.N = N;
        q.K = K;
        return q;
    }

    void init(const HostModel& m, GPT2EngineOptions o) {
        cfg = m.cfg;
        opt = o;
        if (opt.max_batch < 1 || opt.max_batch > 16) throw std::runtime_error("max_batch must be 1..16");
        if (opt.kv_dtype != IE_KV_F32 && opt.kv_dtype != IE_KV_BF16) throw std::runtime_error("kv_dtype");
        HIPC(hipStreamCreate(&stream));
        const int d = cfg.d_model, ff = cfg.d_ff, V = cfg.vocab_size, B = opt.max_batch;
        fp32 = opt.backend == InferenceBackend::CUBLAS_FP32;
        if (fp32) {
            for (const auto& L : m.layers)
                if (L.qkv_f.empty() || L.out_f.empty() || L.up_f.empty() || L.down_f.empty())
                    throw std::runtime_error("fp32 backend: the model has no fp32 weights");
            blas.reset(new ie::VendorSgemm(stream));
            // vendor library calls stay out of graph capture
            opt.use_graph = false;
            opt.fuse = false;
        }
        wte = upload(m.wte);
        wpe = upload(m.wpe);
        lnf_g = upload(m.lnf_g);
        lnf_b = upload(m.lnf_b);
        for (const auto& L : m.layers) {
            Layer D{};
            D.ln1_g = upload(L.ln1_g);
            D.ln1_b = upload(L.ln1_b);
            D.ln2_g = upload(L.ln2_g);
            D.ln2_b = upload(L.ln2_b);
            D.qkv = upload_q(L.qkv_w, L.qkv_s, 3 * d, d);
            D.qkv_b = upload(L.qkv_b);
            D.out = upload_q(L.out_w, L.out_s, d, d);
            D.out_b = upload(L.out_b);
            D.up = upload_q(L.up_w, L.up_s, ff, d);
            D.up_b = upload(L.up_b);
            D.down = upload_q(L.down_w, L.down_s, d, ff);
            D.down_b = upload(L.down_b);
            if (fp32) {
                D.qkv_f = upload(L.qkv_f);
                D.out_f = upload(L.out_f);
                D.up_f = upload(L.up_f);
                D.down_f = upload(L.down_f);
            }
            layers.push_back(D);
        }
        if (opt.int8_lm_head) {
            std::vector<int32_t> hw;
            std::vector<float> hs;
            quantize_rows_host(m.wte, V, d, hw, hs);
            head = upload_q(hw, hs, V, d);
        }
        x = dev<float>((size_t)B * d);
        xn = dev<float>((size_t)B * d);
        qkv = dev<float>((size_t)B * 3 * d);
        q = dev<float>((size_t)B * d);
        attn = dev<float>((size_t)B * d);
        h = dev<float>((size_t)B * ff);
        logits = dev<float>((size_t)B * V);
        act_q = dev<int32_t>((size_t)B * std::max(d, ff) / 4);
        act_s = dev<float>(B);
        if (fp32) gemm_out = dev<float>((size_t)B * std::max(3 * d, ff));

        nbps = (cfg.max_seq_len + kBlock - 1) / kBlock;
        phys_blocks = B * nbps;
        layer_elems = (size_t)phys_blocks * kBlock * d;
        const size_t esz = opt.kv_dtype == IE_KV_BF16 ? 2 : 4;
        kc = dev<char>(layer_elems * esz * cfg.n_layers);
        vc = dev<char>(layer_elems * esz * cfg.n_layers);
        std::vector<int> table((size_t)B * nbps);
        std::iota(table.begin(), table.end(), 0);
        block_table = upload(table);
        positions = dev<int>(B);
        ctx_lens = dev<int>(B);
        tokens = dev<int>(B);
        const int S = ie_decode_num_splits(cfg.max_seq_len, kBlock, 0);
        ws_bytes = ie_decode_attn_workspace_bytes(B, cfg.n_heads, cfg.d_head, S);
        ws = dev<float>(ws_bytes / sizeof(float));
        fused = opt.fuse && (cfg.d_head == 64 || cfg.d_head == 128);
        for (int m = 1; m <= B && fused; ++m)
            fused = ie::gemv_fused_supported(m, d, ie::kSrcLnQuant, ie::kEpiQKV) &&
                    ie::gemv_fused_supported(m, d, ie::kSrcLnQuant, IE_EPI_BIAS_GELU) &&
                    ie::gemv_fused_supported(m, d, ie::kSrcQuant, IE_EPI_BIAS_RESIDUAL) &&
                    ie::gemv_fused_supported(m, ff, ie::kSrcQuant, IE_EPI_BIAS_RESIDUAL) &&
                    ie::gemv_fused_supported(m, d, ie::kSrcLnQuant, IE_EPI_PLAIN);
        qkv_attn = fused && ie::qkv_attn_supported(d, cfg.n_heads, cfg.d_head, kBlock);
        HIPC(hipHostMalloc(&host_tokens, sizeof(int) * B));
        HIPC(hipHostMalloc(&host_ring, sizeof(int) * 2 * B, hipHostMallocCoherent));
        for (auto& e : ring_ev) HIPC(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        head_keys = dev<unsigned long long>(B);
        HIPC(hipMemset(head_keys, 0, sizeof(unsigned long long) * B));
        head_done = dev<unsigned>(1);
        HIPC(hipMemset(head_done, 0, sizeof(unsigned)));
        HIPC(hipHostMalloc(&host_topk_buf, sizeof(float) * 2 * ie::kTopkMax, hipHostMallocCoherent));
        reset();
    }

    ~Impl() {  // best effort: a destructor has nowhere to report errors
        // the rocBLAS handle is bound to `stream` and may free its workspace
        // on it: release it while the stream and the buffers still exist
        blas.reset();
        for (auto& kv : graphs)
            if (kv.second) (void)hipGraphExecDestroy(kv.second);
        for (void* p : allocs) (void)hipFree(p);
        for (void* p : pf_allocs) (void)hipFree(p);
        if (pf.host_ids) (void)hipHostFree(pf.host_ids);
        if (host_tokens) (void)hipHostFree(host_tokens);
        if (host_ring) (void)hipHostFree(host_ring);
        for (auto& e : ring_ev)
            if (e) (void)hipEventDestroy(e);
        if (host_topk_buf) (void)hipHostFree(host_topk_buf);
        if (stream) (void)hipStreamDestroy(stream);
    }

    void reset() {
        pos = 0;
        std::vector<int> z(opt.max_batch, 0);
        HIPC(hipMemcpyAsync(positions, z.data(), sizeof(int) * z.size(), hipMemcpyHostToDevice, stream));
        HIPC(hipMemcpyAsync(ctx_lens, z.data(), sizeof(int) * z.size(), hipMemcpyHostToDevice, stream));
        HIPC(hipStreamSynchronize(stream));
    }

    void* layer_k(int l) { return kc + layer_elems * (opt.kv_dtype == IE_KV_BF16 ? 2 : 4) * l; }
    void* layer_v(int l) { return vc + layer_elems * (opt.kv_dtype == IE_KV_BF16 ? 2 : 4) * l; }

    // GEMV with its activation operand built from fp32 rows in the kernel.
    void fused_gemv(int B, const QuantWeight& w, int src, const float* xin, const float* g,
                    const float* b, int epi, const float* bias, const float* res, float* out,
                    const ie::GemvFusion* qkv_io = nullptr) {
        ie::GemmArgs a{};
        a.M = B; a.N = w.N; a.K = w.K;
        a.BT = w.packed; a.sB = w.scale;
        a.bias = bias; a.residual = res; a.C = out; a.epi = epi;
        ie::GemvFusion f = qkv_io ? *qkv_io : ie::GemvFusion{};
        f.src = src; f.x = xin; f.gamma = g; f.beta = b; f.eps = 1e-5f;
        ie::launch_gemv_fused(a, f, stream);
        IEC(ie::check_launch("fused gemv"));
    }

    // Whether a step's cache reads (all layers, B sequences at the plan's
    // longest context) exceed what the caches keep beside the weights: then
    // the fused attention streams them with non-temporal loads (GPT-2 Small
    // batch 16: 359.6 -> 340.6 us per step; batch 1, 28 MB, keeps plain
    // loads: 240.8 against 256.3 us with them).
    bool kv_stream_step(int B) const {
        const double bytes = 2.0 * cfg.n_layers * (double)B * plan.max_ctx * cfg.d_model *
                             (opt.kv_dtype == IE_KV_BF16 ? 2 : 4);
        return bytes > 64.0 * (1 << 20);
    }

    // The decode step with LayerNorm / quantizer prologues and the QKV-append
    // epilogue, and with a one-split attention plan the QKV projection and
    // the attention in one launch per (sequence, head): 4 launches per layer
    // (5 with more splits), plus the embedding and a two-launch head.  Same
    // operations and order as enqueue_step_unfused, so the same bits.
    void enqueue_step_fused(int B) {
        const int d = cfg.d_model, H = cfg.n_heads;
        hipStream_t s = stream;
        // With a one-split plan the first layer's QKV + attention launch
        // builds the embedding itself.
        const bool emb_fused = plan.splits == 1 && qkv_attn;
        if (!emb_fused) IEC(ie_embedding_batch(B, tokens, positions, d, wte, wpe, x, (ie_stream_t)s));
        for (int l = 0; l < cfg.n_layers; ++l) {
            const Layer& L = layers[l];
            ie::GemvFusion io{};
            io.q = q; io.kc = layer_k(l); io.vc = layer_v(l); io.kv_dtype = opt.kv_dtype;
            io.positions = positions; io.table = block_table; io.nbps = nbps; io.block_size = kBlock;
            io.ctx_lens = ctx_lens;
            if (plan.splits == 1 && qkv_attn) {
                // QKV projection and attention in one launch per (sequence, head)
                io.src = ie::kSrcLnQuant; io.x = x; io.gamma = L.ln1_g; io.beta = L.ln1_b; io.eps = 1e-5f;
                io.kv_stream = kv_stream_step(B);
                if (l == 0 && emb_fused) { io.ids = tokens; io.wte = wte; io.wpe = wpe; }
                ie::launch_qkv_attn(B, H, L.qkv.packed, L.qkv.scale, L.qkv_b, io, attn, s);
                IEC(ie::check_launch("qkv_attn"));
                fused_gemv(B, L.out, ie::kSrcQuant, attn, nullptr, nullptr, IE_EPI_BIAS_RESIDUAL, L.out_b, x, x);
                fused_gemv(B, L.up, ie::kSrcLnQuant, x, L.ln2_g, L.ln2_b, IE_EPI_BIAS_GELU, L.up_b, nullptr, h);
                fused_gemv(B, L.down, ie::kSrcQuant, h, nullptr, nullptr, IE_EPI_BIAS_RESIDUAL, L.down_b, x, x);
                continue;
            }
            fused_gemv(B, L.qkv, ie::kSrcLnQuant, x, L.ln1_g, L.ln1_b, ie::kEpiQKV, L.qkv_b, nullptr,
                       nullptr, &io);
            ie::DecodeArgs a{};
            a.B = B; a.H_q = H; a.H_kv = H; a.d = cfg.d_head;
            a.Q = q; a.k_cache = layer_k(l); a.v_cache = layer_v(l); a.kv_dtype = opt.kv_dtype;
            a.block_table = block_table; a.context_lens = ctx_lens;
            a.block_size = kBlock; a.num_blocks_per_seq = nbps;
            a.num_splits = plan.splits;
            a.blocks_per_split = ((plan.max_ctx + kBlock - 1) / kBlock + plan.splits - 1) / plan.splits;
            a.O = attn; a.workspace = ws;
            ie::launch_decode_attn(a, s);
            IEC(ie::check_launch("decode_attn"));
            fused_gemv(B, L.out, ie::kSrcQuant, attn, nullptr, nullptr, IE_EPI_BIAS_RESIDUAL, L.out_b, x, x);
            fused_gemv(B, L.up, ie::kSrcLnQuant, x, L.ln2_g, L.ln2_b, IE_EPI_BIAS_GELU, L.up_b, nullptr, h);
            fused_gemv(B, L.down, ie::kSrcQuant, h, nullptr, nullptr, IE_EPI_BIAS_RESIDUAL, L.down_b, x, x);
        }
        enqueue_head(B, true);
    }

    // Final LayerNorm, LM head and argmax over the hidden rows x [B, d]
    // (src/gpt2_engine.cu:612-627, 391-410; sampler.cu:10-14): logits
    // [B, V], argmax ids into `tokens`, and (advance, after a decode step)
    // every position moved on.  The fused step with the fp32 head does it in
    // one launch (LayerNorm + LM head + per-row argmax keys; its last
    // workgroup writes the ids, also into host_ring).
    // Whether the step's head is that fused one.
    bool head_writes_host(int B) const {
        return fused && !opt.int8_lm_head && ie::vocab_head_supported(B, cfg.d_model);
    }

    void enqueue_head(int B, bool advance) {
        const int d = cfg.d_model, V = cfg.vocab_size;
        ie_stream_t st = (ie_stream_t)stream;
        if (head_writes_host(B)) {
            ie::launch_vocab_head(B, x, lnf_g, lnf_b, 1e-5f, wte, logits, d, V, head_keys, head_done, tokens,
                                  positions, advance, host_ring, stream);
            IEC(ie::check_launch("vocab_head"));
            return;
        }
        if (fused) {
            if (opt.int8_lm_head) {
                fused_gemv(B, head, ie::kSrcLnQuant, x, lnf_g, lnf_b, IE_EPI_PLAIN, nullptr, nullptr, logits);
            } else {
                IEC(ie_layernorm(B, d, x, lnf_g, lnf_b, xn, 1e-5f, st));
                IEC(ie_vocab_proj(B, xn, wte, logits, d, V, st));
            }
        } else {
            IEC(ie_layernorm(B, d, x, lnf_g, lnf_b, xn, 1e-5f, st));
            if (opt.int8_lm_head) {
                IEC(ie_quantize_fp32_to_int8(B, d, xn, act_q, act_s, st));
                IEC(ie_int8_gemm(B, V, d, act_q, head.packed, act_s, head.scale, IE_EPI_PLAIN, nullptr, nullptr,
                                 logits, st));
            } else {
                IEC(ie_vocab_proj(B, xn, wte, logits, d, V, st));
            }
        }
        IEC(ie_argmax(B, logits, V, tokens, st));
        if (advance) {
            ie::launch_advance(B, positions, stream);
            IEC(ie::check_launch("advance"));
        }
    }

    // One linear of the unfused step or of prefill over M rows:
    // out = epilogue(in . W) as the INT8 path (the per-row activation
    // quantizer, then the INT8 GEMM with its epilogue, through the C ABI) or,
    // with the fp32 backend, a vendor fp32 GEMM on the [K, N] weights followed
    // by the same epilogue in fp32 (src/gpt2_engine.cu:530-610).
    void linear(int M, const QuantWeight& w, const float* wf, const float* in, int epi, const float* bias,
                const float* res, float* out, int32_t* aq, float* as, float* gout) {
        ie_stream_t st = (ie_stream_t)stream;
        if (fp32) {
            blas->rowmajor(M, w.N, w.K, in, wf, gout);
            ie::launch_fp32_epilogue(M, w.N, gout, bias, res, out, epi, stream);
            IEC(ie::check_launch("fp32 epilogue"));
            return;
        }
        IEC(ie_quantize_fp32_to_int8(M, w.K, in, aq, as, st));
        IEC(ie_int8_gemm(M, w.N, w.K, aq, w.packed, as, w.scale, epi, bias, res, out, st));
    }

    // Prefill's LayerNorm-fed projection: LayerNorm of pf.x [M, K], the
    // per-row quantizer, the INT8 GEMM.  With the INT8 backend at a width
    // launch_ln_quant takes, the LayerNorm and the quantizer are one launch
    // with the bytes of the pair; otherwise the C-ABI ops.
    void ln_linear(int M, const float* gamma, const float* beta, const QuantWeight& w, const float* wf, int epi,
                   const float* bias, float* out) {
        ie_stream_t st = (ie_stream_t)stream;
        if (!fp32 && ie::ln_quant_supported(w.K)) {
            ie::launch_ln_quant(M, w.K, pf.x, gamma, beta, 1e-5f, pf.act_q, pf.act_s, stream);
            IEC(ie::check_launch("ln_quant"));
            IEC(ie_int8_gemm(M, w.N, w.K, pf.act_q, w.packed, pf.act_s, w.scale, epi, bias, nullptr, out, st));
            return;
        }
        IEC(ie_layernorm(M, w.K, pf.x, gamma, beta, pf.xn, 1e-5f, st));
        linear(M, w, wf, pf.xn, epi, bias, nullptr, out, pf.act_q, pf.act_s, pf.gemm_out);
    }

    // Prefill's first LayerNorm, QKV projection and Q split + K/V append for
    // B x Pc rows at positions pos ..: with the INT8 backend at a width
    // launch_ln_quant takes, two launches (the LayerNorm + quantizer, then
    // the GEMM storing Q and the K/V rows itself, where prefill_qkv_write
    // would move them from pf.qkv); otherwise ln_linear into pf.qkv and
    // prefill_qkv_write.
    bool qkv_routed() const { return !fp32 && ie::ln_quant_supported(cfg.d_model); }

    void prefill_qkv(int B, int Pc, int l) {
        const Layer& L = layers[l];
        const int d = cfg.d_model, M = B * Pc;
        if (qkv_routed()) {  // pf.row_slot holds this chunk's slots
            ie::launch_ln_quant(M, d, pf.x, L.ln1_g, L.ln1_b, 1e-5f, pf.act_q, pf.act_s, stream);
            IEC(ie::check_launch("ln_quant"));
            ie::GemmArgs a{M, L.qkv.N, L.qkv.K, pf.act_q, L.qkv.packed, pf.act_s, L.qkv.scale, L.qkv_b,
                           nullptr, nullptr, ie::kEpiQKVRoute};
            a.route.q = pf.q;
            a.route.kc = layer_k(l);
            a.route.vc = layer_v(l);
            a.route.kv_dtype = opt.kv_dtype;
            a.route.row_slot = pf.row_slot;
            a.route.d = d;
            ie::launch_gemm_i8_qkv_route(a, stream);
            IEC(ie::check_launch("qkv_route"));
            return;
        }
        ln_linear(M, L.ln1_g, L.ln1_b, L.qkv, L.qkv_f, IE_EPI_BIAS, L.qkv_b, pf.qkv);
        ie::launch_prefill_qkv_write(B, Pc, pos, d, pf.qkv, block_table, nbps, kBlock, pf.q, layer_k(l),
                                     layer_v(l), opt.kv_dtype, stream);
        IEC(ie::check_launch("prefill_qkv_write"));
    }

    void enqueue_step(int B) {
        if (fused)
            enqueue_step_fused(B);
        else
            enqueue_step_unfused(B);
    }

    // One decode step for B sequences: reads tokens/positions on the device,
    // leaves logits, writes the argmax into tokens and advances positions.
    // Every operation goes through the public C ABI.
    void enqueue_step_unfused(int B) {
        const int d = cfg.d_model, H = cfg.n_heads;
        hipStream_t s = stream;
        ie_stream_t st = (ie_stream_t)s;
        IEC(ie_embedding_batch(B, tokens, positions, d, wte, wpe, x, st));
        for (int l = 0; l < cfg.n_layers; ++l) {
            const Layer& L = layers[l];
            IEC(ie_layernorm(B, d, x, L.ln1_g, L.ln1_b, xn, 1e-5f, st));
            linear(B, L.qkv, L.qkv_f, xn, IE_EPI_BIAS, L.qkv_b, nullptr, qkv, act_q, act_s, gemm_out);
            ie::launch_qkv_split_append(B, d, qkv, positions, block_table, nbps, kBlock, q, layer_k(l),
                                        layer_v(l), opt.kv_dtype, ctx_lens, s);
            IEC(ie::check_launch("qkv_split_append"));
            IEC(ie_decode_attn(B, H, H, cfg.d_head, q, layer_k(l), layer_v(l), opt.kv_dtype,
                               block_table, ctx_lens, plan.max_ctx, kBlock, nbps, attn, ws, ws_bytes, plan.splits,
                               st));
            linear(B, L.out, L.out_f, attn, IE_EPI_BIAS_RESIDUAL, L.out_b, x, x, act_q, act_s, gemm_out);
            IEC(ie_layernorm(B, d, x, L.ln2_g, L.ln2_b, xn, 1e-5f, st));
            linear(B, L.up, L.up_f, xn, IE_EPI_BIAS_GELU, L.up_b, nullptr, h, act_q, act_s, gemm_out);
            linear(B, L.down, L.down_f, h, IE_EPI_BIAS_RESIDUAL, L.down_b, x, x, act_q, act_s, gemm_out);
        }
        enqueue_head(B, true);
    }

    // Split plan for a step whose attention sees ctx tokens: one split per
    // kTokensPerSplit tokens (four waves share a split, so each walks about
    // six 16-token chunks), at most the workspace's 16; a single split writes
    // the output directly.  Computed from the host's position mirror, so the
    // captured graph for that plan can be replayed.
    static constexpr int kTokensPerSplit = 384;
    AttnPlan plan_for(int ctx) const {
        AttnPlan p;
        p.splits = std::max(1, std::min((ctx + kTokensPerSplit - 1) / kTokensPerSplit, 16));
        p.max_ctx = p.splits == 16 ? cfg.max_seq_len
                                   : std::min(p.splits * kTokensPerSplit, cfg.max_seq_len);
        return p;
    }

    void run_step(int B) {
        if (pos >= cfg.max_seq_len) throw std::runtime_error("context is full (max_seq_len reached)");
        plan = plan_for(pos + 1);
        if (opt.use_graph) {
            hipGraphExec_t& graph = graphs[{B, plan.splits}];
            if (!graph) {
                hipGraph_t g;
                HIPC(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
                try {
                    enqueue_step(B);
                } catch (...) {
                    hipGraph_t dummy = nullptr;
                    (void)hipStreamEndCapture(stream, &dummy);
                    if (dummy) (void)hipGraphDestroy(dummy);
                    throw;
                }
                HIPC(hipStreamEndCapture(stream, &g));
                const hipError_t e = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
                (void)hipGraphDestroy(g);
                if (e != hipSuccess) {
                    graph = nullptr;
                    HIPC(e);
                }
            }
            HIPC(hipGraphLaunch(graph, stream));
        } else {
            enqueue_step(B);
        }
        ++pos;
    }

    // Host token ids index wte rows on the device without a bound: reject
    // any outside [0, vocab_size) before they are uploaded.
    void check_ids(const int* t, size_t n) const {
        if (ie_check_token_ids((int)n, t, cfg.vocab_size) != IE_OK) throw std::runtime_error(ie_last_error());
    }

    // Whether the step at the current position would first have to capture
    // its graph (done on an idle stream).
    bool step_needs_capture(int B) const {
        if (!opt.use_graph) return false;
        auto it = graphs.find({B, plan_for(pos + 1).splits});
        return it == graphs.end() || !it->second;
    }

    // Greedy decode with one step in flight ahead of the host: the argmax of
    // a step is already in the device token buffer, where the next step's
    // embedding reads it, so step k + 1 is enqueued before the host waits
    // for step k's ids (copied to ring slot k % 2 behind step k; stream
    // order puts the copy before step k + 1 overwrites the buffer).  The GPU
    // then runs the steps back to back instead of idling for each host round
    // trip.  launch() enqueues a step if the caller's limits allow one more
    // (EOS, which only the host sees, is the one stop that cannot be known in
    // advance); wait() returns the oldest in-flight step's ids; finish()
    // undoes a step that was enqueued past the stop: the position mirror and
    // the device positions go back one, and the device token buffer gets the
    // ids the host kept (the cache row that step wrote is overwritten by the
    // next step or prompt at that position).
    struct GreedyPipe {
        Impl& I;
        int B;
        long launched = 0, waited = 0;
        int slots[2] = {0, 0};  // ring slot of each in-flight step, oldest first
        GreedyPipe(Impl& impl, int b) : I(impl), B(b) {}
        void launch() {
            if (I.step_needs_capture(B)) HIPC(hipStreamSynchronize(I.stream));
            const int slot = I.pos & 1;
            I.run_step(B);
            if (!I.head_writes_host(B))
                HIPC(hipMemcpyAsync(I.host_ring + slot * B, I.tokens, sizeof(int) * B, hipMemcpyDeviceToHost,
                                    I.stream));
            HIPC(hipEventRecord(I.ring_ev[slot], I.stream));
            slots[launched & 1] = slot;
            ++launched;
        }
        const int* wait() {
            const int slot = slots[waited & 1];
            HIPC(hipEventSynchronize(I.ring_ev[slot]));
            ++waited;
            return I.host_ring + slot * B;
        }
        void finish(const int* last_ids) {
            if (launched == waited) return;
            HIPC(hipStreamSynchronize(I.stream));
            I.pos -= (int)(launched - waited);
            ie::launch_set_positions(B, I.pos, I.positions, I.ctx_lens, I.stream);
            IEC(ie::check_launch("set_positions"));
            std::memcpy(I.host_tokens, last_ids, sizeof(int) * B);
            HIPC(hipMemcpyAsync(I.tokens, I.host_tokens, sizeof(int) * B, hipMemcpyHostToDevice, I.stream));
            HIPC(hipStreamSynchronize(I.stream));
            waited = launched;
        }
    };

    // Upload one token per sequence, run a step, fetch the argmax ids.
    // sync = false leaves the step in flight: the caller must synchronize the
    // stream before host_tokens is written again (the sampled loop's pick()
    // does, right after queueing the top-k behind the step).
    void step_tokens(const int* toks, int B, bool fetch, bool sync = true) {
        check_ids(toks, B);
        std::memcpy(host_tokens, toks, sizeof(int) * B);
        HIPC(hipMemcpyAsync(tokens, host_tokens, sizeof(int) * B, hipMemcpyHostToDevice, stream));
        run_step(B);
        if (fetch) HIPC(hipMemcpyAsync(host_tokens, tokens, sizeof(int) * B, hipMemcpyDeviceToHost, stream));
        if (sync) HIPC(hipStreamSynchronize(stream));
    }

    // ---- prefill ----
    static constexpr int kPrefillRows = 4096;  // rows (sequences x tokens) per chunk

    bool prefill_applies() const { return opt.prefill && (cfg.d_head == 64 || cfg.d_head == 128); }
    int prefill_chunk(int B) const {
        return opt.prefill_chunk > 0 ? opt.prefill_chunk : std::max(1, kPrefillRows / B);
    }

    void ensure_prefill(int rows) {
        if (rows <= pf.rows) return;
        HIPC(hipStreamSynchronize(stream));
        pf.rows = 0;
        for (void* p : pf_allocs) (void)hipFree(p);
        pf_allocs.clear();
        if (pf.host_ids) (void)hipHostFree(pf.host_ids);
        pf.host_ids = nullptr;
        const size_t R = rows, d = cfg.d_model, ff = cfg.d_ff;
        auto alloc = [&](size_t bytes) {
            void* p = nullptr;
            HIPC(hipMalloc(&p, std::max<size_t>(bytes, 16)));
            pf_allocs.push_back(p);
            return p;
        };
        pf.x = static_cast<float*>(alloc(R * d * 4));
        pf.xn = static_cast<float*>(alloc(R * d * 4));
        pf.qkv = static_cast<float*>(alloc(R * 3 * d * 4));
        pf.q = static_cast<float*>(alloc(R * d * 4));
        pf.attn = static_cast<float*>(alloc(R * d * 4));
        pf.h = static_cast<float*>(alloc(R * ff * 4));
        pf.act_q = static_cast<int32_t*>(alloc(R * std::max(d, ff)));
        pf.act_s = static_cast<float*>(alloc(R * 4));
        if (fp32) pf.gemm_out = static_cast<float*>(alloc(R * std::max(3 * d, ff) * 4));
        pf.ids = static_cast<int*>(alloc(R * 4));
        pf.row_slot = static_cast<int*>(alloc(R * 4));
        HIPC(hipHostMalloc(&pf.host_ids, R * sizeof(int)));
        pf.rows = rows;
    }

    // A prompt chunk through the model at once (the reference's prefill,
    // src/gpt2_engine.cu:660-676 with forward_layer's is_prefill branch,
    // :447-528): B sequences of P tokens (toks[b * P + t]) at positions
    // pos .. pos + P - 1, as M = B x chunk-row GEMMs and the causal prefill
    // attention over the paged cache, in chunks of prefill_chunk(B) tokens
    // per sequence (a later chunk attends to the earlier ones through the
    // cache).  Every operation goes through the public C ABI but these: each
    // LayerNorm and the quantizer of its output are one launch (same bytes,
    // ln_linear), and the Q split + K/V append is the QKV GEMM's epilogue
    // (prefill_qkv) or its own launch.  Leaves the
    // logits [B, V] of each sequence's last token, their argmax in `tokens`,
    // and positions at pos + P.  The reference prefills only a fresh session
    // and feeds a continuation through decode steps; here both prefill.
    void prefill(const int* toks, int B, int P) {
        if (B < 1 || B > opt.max_batch) throw std::runtime_error("batch out of range");
        if (P < 1) throw std::runtime_error("empty prompt");
        if (!prefill_applies()) throw std::runtime_error("prefill needs d_head 64 or 128");
        if (pos + P > cfg.max_seq_len) throw std::runtime_error("prompt does not fit the context");
        check_ids(toks, (size_t)B * P);
        const int d = cfg.d_model, H = cfg.n_heads, dh = cfg.d_head;
        const int chunk = std::min(P, prefill_chunk(B));
        ensure_prefill(B * chunk);
        ie_stream_t st = (ie_stream_t)stream;
        int Pc = 0;
        for (int c0 = 0; c0 < P; c0 += Pc) {
            Pc = std::min(chunk, P - c0);
            const int M = B * Pc;
            if (c0 > 0) HIPC(hipStreamSynchronize(stream));  // host_ids is about to be rewritten
            for (int b = 0; b < B; ++b)
                std::memcpy(pf.host_ids + (size_t)b * Pc, toks + (size_t)b * P + c0, sizeof(int) * Pc);
            HIPC(hipMemcpyAsync(pf.ids, pf.host_ids, sizeof(int) * M, hipMemcpyHostToDevice, stream));
            for (int b = 0; b < B; ++b)
                IEC(ie_embedding(pf.ids + (size_t)b * Pc, Pc, pos, d, wte, wpe, pf.x + (size_t)b * Pc * d, st));
            if (qkv_routed()) {
                ie::launch_prefill_row_slots(B, Pc, pos, block_table, nbps, kBlock, pf.row_slot, stream);
                IEC(ie::check_launch("prefill_row_slots"));
            }
            for (int l = 0; l < cfg.n_layers; ++l) {
                const Layer& L = layers[l];
                prefill_qkv(B, Pc, l);
                IEC(ie_prefill_attn(B, Pc, H, H, dh, pf.q, layer_k(l), layer_v(l), opt.kv_dtype, block_table, nbps,
                                    kBlock, pos, pf.attn, st));
                linear(M, L.out, L.out_f, pf.attn, IE_EPI_BIAS_RESIDUAL, L.out_b, pf.x, pf.x, pf.act_q, pf.act_s,
                       pf.gemm_out);
                ln_linear(M, L.ln2_g, L.ln2_b, L.up, L.up_f, IE_EPI_BIAS_GELU, L.up_b, pf.h);
                linear(M, L.down, L.down_f, pf.h, IE_EPI_BIAS_RESIDUAL, L.down_b, pf.x, pf.x, pf.act_q, pf.act_s,
                       pf.gemm_out);
            }
            pos += Pc;
        }
        // hidden row of each sequence's last token -> x [B, d]
        HIPC(hipMemcpy2DAsync(x, sizeof(float) * d, pf.x + (size_t)(Pc - 1) * d, sizeof(float) * d * Pc,
                              sizeof(float) * d, B, hipMemcpyDeviceToDevice, stream));
        ie::launch_set_positions(B, pos, positions, ctx_lens, stream);
        IEC(ie::check_launch("set_positions"));
        enqueue_head(B, false);
    }

    // Prompt of B sequences x P tokens through prefill (or, if disabled, one
    // decode step per position); the argmax ids end up in host_tokens.
    void run_prompt(const int* toks, int B, int P) {
        if (prefill_applies()) {
            prefill(toks, B, P);
            HIPC(hipMemcpyAsync(host_tokens, tokens, sizeof(int) * B, hipMemcpyDeviceToHost, stream));
            HIPC(hipStreamSynchronize(stream));
            return;
        }
        std::vector<int> col(B);
        for (int i = 0; i < P; ++i) {
            for (int b = 0; b < B; ++b) col[b] = toks[(size_t)b * P + i];
            step_tokens(col.data(), B, i + 1 == P);
        }
    }

    // Bytes one decode step streams for B sequences whose attention reads ctx
    // cached tokens each.
    double bytes_per_step(int B, double ctx) const {
        const double d = cfg.d_model, ff = cfg.d_ff, V = cfg.vocab_size;
        double w = cfg.n_layers * (3 * d * d + d * d + 2 * d * ff) * (fp32 ? 4.0 : 1.0);  // linear weights
        w += cfg.n_layers * 4.0 * (3 * d + d + ff + d) * (fp32 ? 1 : 2);   // biases (+ scales)
        w += cfg.n_layers * 4.0 * 4 * d;                                      // LayerNorm
        w += opt.int8_lm_head ? V * d + 4 * V : 4.0 * V * d;                  // LM head
        const double kv = 2.0 * cfg.n_layers * (double)B * ctx * d * (opt.kv_dtype == IE_KV_BF16 ? 2 : 4);
        return w + kv;
    }

    // tps counts the tokens the decode steps produced for sequences still
    // running (a sequence past its EOS is carried by the batch step but emits
    // nothing); mbu counts the bytes the timed steps streamed: the n steps
    // that ended at position pos read pos - n + 1 .. pos cached tokens, so
    // their mean context is pos - (n - 1) / 2.
    void fill_tail_metrics(InferenceMetrics& m, const std::vector<float>& itl, float decode_ms, int B,
                           long decode_tokens) {
        const int n = (int)itl.size();
        if (n > 0) {
            m.tpot_ms = decode_ms / n;
            m.tps = 1000.0f * decode_tokens / decode_ms;
            m.itl_min_ms = *std::min_element(itl.begin(), itl.end());
            m.itl_max_ms = *std::max_element(itl.begin(), itl.end());
            auto sorted = itl;
            std::sort(sorted.begin(), sorted.end());
            m.itl_p95_ms = n >= 20 ? sorted[(int)(n * 0.95)] : m.itl_max_ms;
            m.mbu = (float)(bytes_per_step(B, pos - (n - 1) / 2.0) * (1000.0 * n / decode_ms) / 8.0e12);
        }
        m.kv_cache_pct = 100.0f * ((pos + kBlock - 1) / kBlock) / nbps;
        size_t fr = 0, tot = 0;
        if (hipMemGetInfo(&fr, &tot) == hipSuccess) {
            m.vram_used_mb = (tot - fr) / (1024.0f * 1024.0f);
            m.vram_total_mb = tot / (1024.0f * 1024.0f);
        }
    }
};

using Clock = std::chrono::steady_clock;
static float ms_since(Clock::time_point t) {
    return std::chrono::duration<float, std::milli>(Clock::now() - t).count();
}

GPT2Engine::GPT2Engine(const std::string& model_dir, GPT2EngineOptions opt) : impl_(new Impl) {
    impl_->init(load_model(model_dir, opt.backend == InferenceBackend::CUBLAS_FP32), opt);
}

GPT2Engine::GPT2Engine(const std::string& model_dir, InferenceBackend backend) : impl_(new Impl) {
    GPT2EngineOptions opt;
    opt.backend = backend;
    impl_->init(load_model(model_dir, backend == InferenceBackend::CUBLAS_FP32), opt);
}

GPT2Engine::GPT2Engine(const GPT2Config& cfg, uint64_t seed, GPT2EngineOptions opt) : impl_(new Impl) {
    impl_->init(random_model(cfg, seed, opt.backend == InferenceBackend::CUBLAS_FP32), opt);
}

GPT2Engine::~GPT2Engine() = default;

void GPT2Engine::reset_session() { impl_->reset(); }
int GPT2Engine::session_tokens() const { return impl_->pos; }
const GPT2Config& GPT2Engine::config() const { return impl_->cfg; }
const float* GPT2Engine::logits_device() const { return impl_->logits; }
double GPT2Engine::step_bytes(int batch) const { return impl_->bytes_per_step(batch, impl_->pos + 1.0); }

void GPT2Engine::prefill(const int* tokens, int batch, int len) {
    impl_->prefill(tokens, batch, len);
    HIPC(hipStreamSynchronize(impl_->stream));
}

void GPT2Engine::step(const int* tokens, int batch) {
    if (batch < 1 || batch > impl_->opt.max_batch) throw std::runtime_error("batch out of range");
    impl_->step_tokens(tokens, batch, false);
}

// src/sampler.cu:16-45 for sequence 0's logits: the k largest on the device
// (ie_topk), then the reference's softmax and draw on the host
// (ie_top_k_draw, srand(seed) / rand()).  k above IE_TOPK_MAX takes the
// reference's own route, the whole row to the host, with the same order for
// equal values (lower index first) and the same draw.
static int sample_top_k_engine(const float* d_logits, int V, int k, float temperature, unsigned seed,
                               float* h_buf, hipStream_t s) {
    k = std::max(1, std::min(k, V));
    int token = 0;
    if (k <= ie::kTopkMax) {
        // The kernel writes values in words [0, k) and indices in [k, 2k)
        // straight into the pinned host buffer (no copy behind it); the
        // stream's completion makes them visible to the host.
        if (ie_topk(1, d_logits, V, k, h_buf, reinterpret_cast<int*>(h_buf + k), s) != IE_OK)
            throw std::runtime_error(ie_last_error());
        HIPC(hipStreamSynchronize(s));
        if (ie_top_k_draw(h_buf, reinterpret_cast<const int*>(h_buf + k), k, temperature, seed, &token) != IE_OK)
            throw std::runtime_error(ie_last_error());
        return token;
    }
    if (ie::host_top_k_token(d_logits, V, k, temperature, seed, s, &token) != IE_OK)
        throw std::runtime_error(ie_last_error());
    return token;
}

void GPT2Engine::generate(const std::vector<int>& prompt_tokens, int max_new_tokens, float temperature,
                          int top_k, bool greedy, std::function<void(int)> token_callback,
                          InferenceMetrics& metrics, bool reset_kv) {
    Impl& I = *impl_;
    metrics = InferenceMetrics{};
    metrics.max_tokens = max_new_tokens;
    metrics.generating = true;
    if (prompt_tokens.empty()) throw std::runtime_error("empty prompt");
    I.check_ids(prompt_tokens.data(), prompt_tokens.size());
    if (reset_kv) I.reset();
    // Seeds as the reference's loop passes them: 42 for the token after the
    // prompt, then 43, 44, ... (src/gpt2_engine.cu:707, 713, 747).
    unsigned sample_seed = 42u;
    bool first_pick = true;
    auto pick = [&]() -> int {
        if (greedy) return I.host_tokens[0];
        const unsigned seed = first_pick ? 42u : ++sample_seed;
        first_pick = false;
        return sample_top_k_engine(I.logits, I.cfg.vocab_size, top_k, temperature, seed, I.host_topk_buf,
                                   I.stream);
    };

    const auto t_total = Clock::now();
    // The prompt through prefill (src/gpt2_engine.cu:660-676), or with
    // prefill off one decode step per position (:680-698).
    I.run_prompt(prompt_tokens.data(), 1, (int)prompt_tokens.size());
    int next = pick();
    metrics.ttft_ms = ms_since(t_total);

    std::vector<float> itl;
    float decode_ms = 0.0f;
    if (greedy) {
        // The same loop with the next step enqueued before the host reads the
        // current one (GreedyPipe): the argmax is already on the device.
        // As the loop below, every emitted token is fed through a step (the
        // last one's result is not emitted).
        Impl::GreedyPipe pipe(I, 1);
        auto t = Clock::now();
        if (max_new_tokens > 0 && I.pos < I.cfg.max_seq_len) pipe.launch();
        for (int stepi = 0; stepi < max_new_tokens; ++stepi) {
            if (next == 50256) break;  // GPT-2 <|endoftext|>, src/gpt2_engine.cu:717
            token_callback(next);
            metrics.tokens_generated = stepi + 1;
            if (pipe.launched == pipe.waited) break;  // context full
            if (stepi + 1 < max_new_tokens && I.pos < I.cfg.max_seq_len) pipe.launch();
            next = *pipe.wait();
            const auto now = Clock::now();
            const float dt = std::chrono::duration<float, std::milli>(now - t).count();
            t = now;
            itl.push_back(dt);
            decode_ms += dt;
        }
        pipe.finish(&next);
    } else {
        for (int stepi = 0; stepi < max_new_tokens; ++stepi) {
            if (next == 50256) break;  // GPT-2 <|endoftext|>, src/gpt2_engine.cu:717
            token_callback(next);
            metrics.tokens_generated = stepi + 1;
            if (I.pos >= I.cfg.max_seq_len) break;
            const auto t = Clock::now();
            I.step_tokens(&next, 1, greedy, false);  // pick() synchronizes behind the top-k
            next = pick();
            const float dt = ms_since(t);
            itl.push_back(dt);
            decode_ms += dt;
        }
    }
    I.fill_tail_metrics(metrics, itl, decode_ms, 1, (long)itl.size());
    metrics.end_to_end_ms = ms_since(t_total);
    metrics.generating = false;
}

void GPT2Engine::generate_batch(const std::vector<std::vector<int>>& prompts, int max_new_tokens,
                                std::vector<std::vector<int>>& out, InferenceMetrics& metrics,
                                bool ignore_eos) {
    Impl& I = *impl_;
    const int B = (int)prompts.size();
    if (B < 1 || B > I.opt.max_batch) throw std::runtime_error("batch out of range");
    const size_t P = prompts[0].size();
    for (const auto& p : prompts) {
        if (p.size() != P || P == 0) throw std::runtime_error("prompts must share one non-zero length");
        I.check_ids(p.data(), P);
    }
    metrics = InferenceMetrics{};
    metrics.max_tokens = max_new_tokens;
    metrics.generating = true;
    I.reset();
    out.assign(B, {});
    std::vector<int> flat((size_t)B * P);
    for (int b = 0; b < B; ++b) std::copy(prompts[b].begin(), prompts[b].end(), flat.begin() + (size_t)b * P);
    const auto t_total = Clock::now();
    I.run_prompt(flat.data(), B, (int)P);
    metrics.ttft_ms = ms_since(t_total);
    std::vector<float> itl;
    float decode_ms = 0.0f;
    std::vector<char> done(B, 0);
    long decode_tokens = 0;
    // The argmax of the previous step is already in the device token buffer:
    // each step reads it directly, only the ids come back, and the next step
    // is enqueued before the host waits for the current one (GreedyPipe).
    Impl::GreedyPipe pipe(I, B);
    std::vector<int> cur(I.host_tokens, I.host_tokens + B);
    auto t = Clock::now();
    if (max_new_tokens > 1 && I.pos < I.cfg.max_seq_len) pipe.launch();
    for (int stepi = 0; stepi < max_new_tokens; ++stepi) {
        bool all_done = true;
        for (int b = 0; b < B; ++b) {
            const int tkn = cur[b];
            if (!done[b] && !ignore_eos && tkn == 50256) done[b] = 1;
            if (!done[b]) out[b].push_back(tkn);
            all_done = all_done && done[b];
        }
        metrics.tokens_generated = stepi + 1;
        // The step for this iteration was enqueued unless a limit other than
        // EOS ruled it out: stop here as the step-by-step loop would.
        if (all_done || pipe.launched == pipe.waited) break;
        if (stepi + 2 < max_new_tokens && I.pos < I.cfg.max_seq_len) pipe.launch();
        const int* ids = pipe.wait();
        // The timed step's tokens: one for each sequence still running when
        // it was enqueued (done[] does not yet see the ids it returned).
        for (int b = 0; b < B; ++b) decode_tokens += done[b] ? 0 : 1;
        std::copy(ids, ids + B, cur.begin());
        const auto now = Clock::now();
        const float dt = std::chrono::duration<float, std::milli>(now - t).count();
        t = now;
        itl.push_back(dt);
        decode_ms += dt;
    }
    pipe.finish(cur.data());
    std::copy(cur.begin(), cur.end(), I.host_tokens);
    I.fill_tail_metrics(metrics, itl, decode_ms, B, decode_tokens);
    metrics.end_to_end_ms = ms_since(t_total);
    metrics.generating = false;
}

void GPT2Engine::write_random_model(const std::string& dir, const GPT2Config& cfg, uint64_t seed) {
    const HostModel m = random_model(cfg, seed, true);
    ::mkdir(dir.c_str(), 0755);
    {
        std::ofstream f(dir + "/config.json");
        f << "{\n  \"n_layers\": " << cfg.n_layers << ",\n  \"n_heads\": " << cfg.n_heads
          << ",\n  \"d_model\": " << cfg.d_model << ",\n  \"d_ff\": " << cfg.d_ff
          << ",\n  \"vocab_size\": " << cfg.vocab_size << ",\n  \"max_seq_len\": " << cfg.max_seq_len
          << ",\n  \"d_head\": " << cfg.d_head << "\n}\n";
        if (!f) throw std::runtime_error("cannot write config.json");
    }
    write_bin(dir + "/wte.bin", m.wte);
    write_bin(dir + "/wpe.bin", m.wpe);
    write_bin(dir + "/ln_f_gamma.bin", m.lnf_g);
    write_bin(dir + "/ln_f_beta.bin", m.lnf_b);
    for (int i = 0; i < cfg.n_layers; ++i) {
        char ld[64];
        std::snprintf(ld, sizeof(ld), "/layer_%02d", i);
        const std::string p = dir + ld;
        ::mkdir(p.c_str(), 0755);
        const auto& L = m.layers[i];
        write_bin(p + "/ln1_gamma.bin", L.ln1_g);
        write_bin(p + "/ln1_beta.bin", L.ln1_b);
        write_bin(p + "/ln2_gamma.bin", L.ln2_g);
        write_bin(p + "/ln2_beta.bin", L.ln2_b);
        write_bin(p + "/qkv_weight.bin", L.qkv_w);
        write_bin(p + "/qkv_scale.bin", L.qkv_s);
        write_bin(p + "/qkv_bias.bin", L.qkv_b);
        write_bin(p + "/out_weight.bin", L.out_w);
        write_bin(p + "/out_scale.bin", L.out_s);
        write_bin(p + "/out_bias.bin", L.out_b);
        write_bin(p + "/ffn_up_weight.bin", L.up_w);
        write_bin(p + "/ffn_up_scale.bin", L.up_s);
        write_bin(p + "/ffn_up_bias.bin", L.up_b);
        write_bin(p + "/ffn_down_weight.bin", L.down_w);
        write_bin(p + "/ffn_down_scale.bin", L.down_s);
        write_bin(p + "/ffn_down_bias.bin", L.down_b);
        // python/export_gpt2.py:48-57: fp32 [K, N] for the vendor GEMM backend
        write_bin(p + "/qkv_weight_fp32.bin", L.qkv_f);
        write_bin(p + "/out_weight_fp32.bin", L.out_f);
        write_bin(p + "/ffn_up_weight_fp32.bin", L.up_f);
        write_bin(p + "/ffn_down_weight_fp32.bin", L.down_f);
    }
}
