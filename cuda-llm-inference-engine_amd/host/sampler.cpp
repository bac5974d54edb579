// sampler.cpp — host side of the reference's samplers (src/sampler.cu) over
// the device kernels: ie_top_k_draw (the softmax over the k selected logits
// and the rand() threshold, src/sampler.cu:28-44) and the reference's own
// entry points sample_argmax / sample_top_k (include/sampler.cuh) for callers
// linking against ie_compat.h.
#include <hip/hip_runtime.h>
#include <stdlib.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <mutex>
#include <numeric>
#include <vector>

#include "../csrc/ie_internal.h"
#include "ie_compat.h"

namespace {

// The reference's generator: glibc rand() (the TYPE_3 additive feedback
// generator behind random()), reseeded with srand(seed) only when the seed
// differs from the previous call's (src/sampler.cu:37-38); the process starts
// as if seeded with 1 and last_seed = 0.  Kept in a private state.
struct DrawRng {
    std::mutex mu;
    random_data rd{};
    char state[128] = {};
    unsigned last_seed = 0;
    DrawRng() { initstate_r(1u, state, sizeof(state), &rd); }
    float next(unsigned seed) {
        if (seed != last_seed) {
            srandom_r(seed, &rd);
            last_seed = seed;
        }
        int32_t v = 0;
        random_r(&rd, &v);
        return (float)v / (float)RAND_MAX;  // the reference divides by RAND_MAX converted to float
    }
};

DrawRng& draw_rng() {
    static DrawRng r;
    return r;
}

// src/sampler.cu:28-44, statement for statement in float arithmetic: the
// probabilities are normalised in place before the running sum.
int draw(const float* vals, const int* idx, int k, float temperature, float r) {
    const float max_val = vals[0];
    float sum = 0.0f;
    std::vector<float> probs(k);
    for (int i = 0; i < k; ++i) {
        probs[i] = expf((vals[i] - max_val) / temperature);
        sum += probs[i];
    }
    for (int i = 0; i < k; ++i) probs[i] /= sum;
    float cum = 0.0f;
    for (int i = 0; i < k; ++i) {
        cum += probs[i];
        if (r < cum) return idx[i];
    }
    return idx[k - 1];
}

// The pinned, coherent host buffer of the compat samplers, made by ie_init()
// (or by a sampler's first call when ie_init was not called) and kept for the
// process (the reference allocates a host vector per call): the selection
// kernels write k values then k indices (or the argmax index) straight into
// it, so no copy follows them.
struct CompatBufs {
    std::mutex mu;
    float* h_buf = nullptr;  // [2 kTopkMax] words
    bool ready() {
        if (!h_buf &&
            hipHostMalloc(&h_buf, sizeof(float) * 2 * ie::kTopkMax, hipHostMallocCoherent) != hipSuccess)
            h_buf = nullptr;
        return h_buf != nullptr;
    }
};

CompatBufs& compat_bufs() {
    static CompatBufs b;
    return b;
}

}  // namespace

namespace ie {
int host_top_k_token(const float* d_logits, int V, int k, float temperature, unsigned seed, hipStream_t s,
                     int* token) {
    std::vector<float> h(V);
    if (hipMemcpyAsync(h.data(), d_logits, sizeof(float) * V, hipMemcpyDeviceToHost, s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return fail(IE_ERR_HIP, "top_k: logits copy failed");
    std::vector<int> idx(V);
    std::iota(idx.begin(), idx.end(), 0);
    std::partial_sort(idx.begin(), idx.begin() + k, idx.end(),
                      [&](int a, int b) { return h[a] > h[b] || (h[a] == h[b] && a < b); });
    std::vector<float> vals(k);
    for (int i = 0; i < k; ++i) vals[i] = h[idx[i]];
    return ie_top_k_draw(vals.data(), idx.data(), k, temperature, seed, token);
}

int compat_sampler_init() {
    CompatBufs& b = compat_bufs();
    std::lock_guard<std::mutex> lock(b.mu);
    return b.ready() ? IE_OK : fail(IE_ERR_HIP, "ie_init: sampler buffer allocation failed");
}
}  // namespace ie

extern "C" int ie_top_k_draw(const float* vals, const int* idx, int k, float temperature, unsigned int seed,
                             int* token) {
    if (!vals || !idx || !token) return ie::fail(IE_ERR_INVALID, "top_k_draw: null pointer");
    if (k < 1) return ie::fail(IE_ERR_INVALID, "top_k_draw: k=%d < 1", k);
    if (!(temperature > 0.0f)) return ie::fail(IE_ERR_INVALID, "top_k_draw: temperature must be > 0");
    DrawRng& g = draw_rng();
    float r;
    {
        std::lock_guard<std::mutex> lock(g.mu);
        r = g.next(seed);
    }
    *token = draw(vals, idx, k, temperature, r);
    return IE_OK;
}

// src/sampler.cu:10-14: the first index of the maximum, on the device.
int sample_argmax(const float* d_logits, int vocab_size) {
    CompatBufs& b = compat_bufs();
    std::lock_guard<std::mutex> lock(b.mu);
    if (!b.ready()) {
        ie::fail(IE_ERR_HIP, "sample_argmax: buffer allocation failed");
        return -1;
    }
    int* h_idx = reinterpret_cast<int*>(b.h_buf);
    if (ie_argmax(1, d_logits, vocab_size, h_idx, nullptr) != IE_OK) return -1;
    if (hipStreamSynchronize(nullptr) != hipSuccess) {
        ie::fail(IE_ERR_HIP, "sample_argmax: synchronize failed");
        return -1;
    }
    return h_idx[0];
}

// src/sampler.cu:16-45: k clamped to the vocabulary as there; the selection
// on the device (k up to IE_TOPK_MAX), the draw on the host.
int sample_top_k(const float* d_logits, int vocab_size, int k, float temperature, unsigned int seed) {
    if (k > vocab_size) k = vocab_size;
    if (k > ie::kTopkMax) {
        int token = -1;
        if (!d_logits || vocab_size <= 0) {
            ie::fail(IE_ERR_INVALID, "sample_top_k: bad logits");
            return -1;
        }
        return ie::host_top_k_token(d_logits, vocab_size, k, temperature, seed, nullptr, &token) == IE_OK ? token
                                                                                                         : -1;
    }
    CompatBufs& b = compat_bufs();
    std::lock_guard<std::mutex> lock(b.mu);
    if (!b.ready()) {
        ie::fail(IE_ERR_HIP, "sample_top_k: buffer allocation failed");
        return -1;
    }
    if (ie_topk(1, d_logits, vocab_size, k, b.h_buf, reinterpret_cast<int*>(b.h_buf + k), nullptr) != IE_OK)
        return -1;
    if (hipStreamSynchronize(nullptr) != hipSuccess) {
        ie::fail(IE_ERR_HIP, "sample_top_k: synchronize failed");
        return -1;
    }
    int token = -1;
    if (ie_top_k_draw(b.h_buf, reinterpret_cast<const int*>(b.h_buf + k), k, temperature, seed, &token) != IE_OK)
        return -1;
    return token;
}
