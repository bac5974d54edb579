// compat_dropin.cpp — test program: the reference's own C++ entry points
// (include/ie_compat.h) called the way the reference's tests call them, from
// a plain C++ program that links libie_amd.so and nothing else of this
// repository.  Null stream, caller-owned device buffers, void returns.
//
//   INT8 GEMM: tests/test_int8_gemm.cu:15-94 — srand(42), A then B drawn as
//     rand()/RAND_MAX*2-1, B^T formed on the host, run_quantize_fp32_to_int8
//     on A and B^T, run_int8_gemm; plus the three epilogue entry points with a
//     bias and a residual drawn next.
//   Decode attention: tests/test_decode_attention.cu:48-140 — srand(42), Q,
//     then K and V interleaved, the paged cache built with an identity block
//     table, workspace [B, H_q, DA_MAX_SPLITS, d + 2], run_decode_attn.
//   run_layernorm in place (the engine's use, src/gpt2_engine.cu:459),
//   run_embedding, run_flash_attn_v2 (causal and not), sample_argmax and
//   sample_top_k.
//   run_layernorm_residual: tests/test_layernorm.cu:34-70 on its five shapes
//     (srand(42): x, residual, gamma in [0.8, 1.2], beta in [-0.1, 0.1]),
//     separate outputs, then again in place (out over x, residual_out over
//     the residual).
//   The K14 tile constants printed as benchmarks/int8_gemm_bench.cu:17 does.
//
// Every input and output is written to <out_dir>/<case>_<name>.bin (raw
// little-endian), and one line per case to <out_dir>/manifest.txt; the
// Python test (tests/test_gpu_compat_dropin.py) checks them against the
// oracle.  Exit status 0 unless a HIP call fails.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "ie_compat.h"

namespace {

std::string g_dir;
FILE* g_manifest = nullptr;

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "compat_dropin: %s: %s\n", what, hipGetErrorString(e));
        std::exit(3);
    }
}

template <typename T>
T* dalloc(size_t n) {
    void* p = nullptr;
    hip_ok(hipMalloc(&p, (n ? n : 1) * sizeof(T)), "hipMalloc");
    return static_cast<T*>(p);
}

template <typename T>
T* upload(const std::vector<T>& v) {
    T* p = dalloc<T>(v.size());
    hip_ok(hipMemcpy(p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
    return p;
}

template <typename T>
std::vector<T> download(const T* p, size_t n) {
    std::vector<T> v(n);
    hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
    hip_ok(hipMemcpy(v.data(), p, n * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return v;
}

template <typename T>
void save(const std::string& cs, const char* name, const std::vector<T>& v) {
    const std::string path = g_dir + "/" + cs + "_" + name + ".bin";
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(v.data(), sizeof(T), v.size(), f) != v.size()) {
        std::fprintf(stderr, "compat_dropin: cannot write %s\n", path.c_str());
        std::exit(4);
    }
    std::fclose(f);
}

float unit_draw() { return (float)rand() / RAND_MAX * 2.0f - 1.0f; }

// tests/test_int8_gemm.cu:15-94, plus the epilogue entry points.
void gemm_case(int M, int N, int K) {
    char cs[64];
    std::snprintf(cs, sizeof(cs), "gemm_%d_%d_%d", M, N, K);
    std::vector<float> A((size_t)M * K), B((size_t)K * N);
    srand(42);
    for (auto& a : A) a = unit_draw();
    for (auto& b : B) b = unit_draw();
    std::vector<float> BT((size_t)N * K);
    for (int k = 0; k < K; ++k)
        for (int n = 0; n < N; ++n) BT[(size_t)n * K + k] = B[(size_t)k * N + n];
    std::vector<float> bias(N), res((size_t)M * N);
    for (auto& x : bias) x = unit_draw();
    for (auto& x : res) x = unit_draw();

    float *dA = upload(A), *dBT = upload(BT), *dbias = upload(bias);
    int32_t* dAp = dalloc<int32_t>((size_t)M * (K / 4));
    int32_t* dBp = dalloc<int32_t>((size_t)N * (K / 4));
    float *dsA = dalloc<float>(M), *dsB = dalloc<float>(N);
    run_quantize_fp32_to_int8(M, K, dA, dAp, dsA);
    run_quantize_fp32_to_int8(N, K, dBT, dBp, dsB);
    hip_ok(hipDeviceSynchronize(), "quantize");
    float* dC = dalloc<float>((size_t)M * N);
    run_int8_gemm(M, N, K, dAp, dBp, dsA, dsB, dC);
    save(cs, "C_plain", download(dC, (size_t)M * N));
    run_int8_gemm_bias(M, N, K, dAp, dBp, dsA, dsB, dbias, dC);
    save(cs, "C_bias", download(dC, (size_t)M * N));
    run_int8_gemm_bias_gelu(M, N, K, dAp, dBp, dsA, dsB, dbias, dC);
    save(cs, "C_gelu", download(dC, (size_t)M * N));
    // residual aliased to C, as the reference engine passes its hidden state
    float* dR = upload(res);
    run_int8_gemm_bias_residual(M, N, K, dAp, dBp, dsA, dsB, dbias, dR, dR);
    save(cs, "C_residual", download(dR, (size_t)M * N));

    save(cs, "A", A);
    save(cs, "B", B);
    save(cs, "bias", bias);
    save(cs, "res", res);
    save(cs, "A_packed", download(dAp, (size_t)M * (K / 4)));
    save(cs, "scale_A", download(dsA, M));
    save(cs, "BT_packed", download(dBp, (size_t)N * (K / 4)));
    save(cs, "scale_B", download(dsB, N));
    std::fprintf(g_manifest, "gemm %s %d %d %d\n", cs, M, N, K);
    for (void* p : {(void*)dA, (void*)dBT, (void*)dbias, (void*)dAp, (void*)dBp, (void*)dsA,
                    (void*)dsB, (void*)dC, (void*)dR})
        hip_ok(hipFree(p), "hipFree");
}

// tests/test_decode_attention.cu:48-140 (the K13 side; the K11 comparison is
// the oracle's job).
void attn_case(int B, int H_q, int H_kv, int ctx, int d, int bs) {
    char cs[64];
    std::snprintf(cs, sizeof(cs), "attn_%d_%d_%d_%d_%d", B, H_q, H_kv, ctx, d);
    const int nbps = (ctx + bs - 1) / bs;
    const size_t q_size = (size_t)B * H_q * d, kv_total = (size_t)B * H_kv * ctx * d;
    const size_t cache = (size_t)B * nbps * bs * H_kv * d;
    std::vector<float> Q(q_size), K(kv_total), V(kv_total), kc(cache), vc(cache);
    std::vector<int> table((size_t)B * nbps), lens(B);
    srand(42);
    for (auto& q : Q) q = unit_draw();
    for (size_t i = 0; i < kv_total; ++i) {
        K[i] = unit_draw();
        V[i] = unit_draw();
    }
    for (int b = 0; b < B; ++b) {
        lens[b] = ctx;
        for (int blk = 0; blk < nbps; ++blk) {
            const int phys = b * nbps + blk;
            table[(size_t)b * nbps + blk] = phys;
            for (int t = 0; t < bs; ++t) {
                const int sp = blk * bs + t;
                for (int h = 0; h < H_kv; ++h)
                    for (int e = 0; e < d; ++e) {
                        const size_t idx = (((size_t)phys * bs + t) * H_kv + h) * d + e;
                        const size_t src = (((size_t)b * H_kv + h) * ctx + sp) * d + e;
                        kc[idx] = sp < ctx ? K[src] : 0.0f;
                        vc[idx] = sp < ctx ? V[src] : 0.0f;
                    }
            }
        }
    }
    float *dQ = upload(Q), *dkc = upload(kc), *dvc = upload(vc);
    int *dt = upload(table), *dl = upload(lens);
    float* dO = dalloc<float>(q_size);
    float* dws = dalloc<float>((size_t)B * H_q * DA_MAX_SPLITS * (d + 2));
    hip_ok(hipMemset(dO, 0, q_size * sizeof(float)), "hipMemset");
    run_decode_attn(B, H_q, H_kv, d, dQ, dkc, dvc, dt, dl, ctx, bs, nbps, dO, dws);
    save(cs, "O", download(dO, q_size));
    save(cs, "Q", Q);
    save(cs, "k_cache", kc);
    save(cs, "v_cache", vc);
    save(cs, "table", table);
    save(cs, "lens", lens);
    std::fprintf(g_manifest, "attn %s %d %d %d %d %d %d\n", cs, B, H_q, H_kv, ctx, d, bs);
    for (void* p : {(void*)dQ, (void*)dkc, (void*)dvc, (void*)dt, (void*)dl, (void*)dO, (void*)dws})
        hip_ok(hipFree(p), "hipFree");
}

// tests/test_layernorm.cu:34-70.
void layernorm_residual_case(int rows, int cols) {
    char cs[64];
    std::snprintf(cs, sizeof(cs), "lnr_%d_%d", rows, cols);
    const size_t n = (size_t)rows * cols;
    std::vector<float> x(n), res(n), gamma(cols), beta(cols);
    srand(42);
    for (auto& v : x) v = (float)rand() / RAND_MAX * 2.0f - 1.0f;
    for (auto& v : res) v = (float)rand() / RAND_MAX * 2.0f - 1.0f;
    for (auto& v : gamma) v = 0.8f + (float)rand() / RAND_MAX * 0.4f;
    for (auto& v : beta) v = (float)rand() / RAND_MAX * 0.2f - 0.1f;
    float *dx = upload(x), *dres = upload(res), *dg = upload(gamma), *db = upload(beta);
    float *dout = dalloc<float>(n), *dres_out = dalloc<float>(n);
    run_layernorm_residual(rows, cols, dx, dres, dg, db, dout, dres_out);
    save(cs, "out", download(dout, n));
    save(cs, "res_out", download(dres_out, n));
    run_layernorm_residual(rows, cols, dx, dres, dg, db, dx, dres);  // in place
    save(cs, "out_inplace", download(dx, n));
    save(cs, "res_out_inplace", download(dres, n));
    save(cs, "x", x);
    save(cs, "res", res);
    save(cs, "gamma", gamma);
    save(cs, "beta", beta);
    std::fprintf(g_manifest, "lnres %s %d %d\n", cs, rows, cols);
    for (void* p : {(void*)dx, (void*)dres, (void*)dg, (void*)db, (void*)dout, (void*)dres_out})
        hip_ok(hipFree(p), "hipFree");
}

void support_cases() {
    // run_layernorm in place: x and out are the same buffer
    const int rows = 4, cols = 768;
    std::vector<float> x((size_t)rows * cols), g(cols), b(cols);
    srand(7);
    for (auto& v : x) v = unit_draw() * 3.0f;
    for (auto& v : g) v = 1.0f + 0.1f * unit_draw();
    for (auto& v : b) v = 0.1f * unit_draw();
    float *dx = upload(x), *dg = upload(g), *db = upload(b);
    run_layernorm(rows, cols, dx, dg, db, dx);
    save("ln", "out", download(dx, x.size()));
    save("ln", "x", x);
    save("ln", "gamma", g);
    save("ln", "beta", b);
    std::fprintf(g_manifest, "layernorm ln %d %d\n", rows, cols);

    // run_embedding: 5 tokens from position 3
    const int V = 1000, S = 64, dm = 768, seq = 5, start = 3;
    std::vector<float> wte((size_t)V * dm), wpe((size_t)S * dm);
    for (auto& v : wte) v = unit_draw();
    for (auto& v : wpe) v = unit_draw();
    std::vector<int> ids = {0, 999, 17, 17, 512};
    float *dwte = upload(wte), *dwpe = upload(wpe), *demb = dalloc<float>((size_t)seq * dm);
    int* dids = upload(ids);
    run_embedding(dids, seq, start, dm, dwte, dwpe, demb);
    save("emb", "out", download(demb, (size_t)seq * dm));
    save("emb", "wte", wte);
    save("emb", "wpe", wpe);
    save("emb", "ids", ids);
    std::fprintf(g_manifest, "embedding emb %d %d %d %d %d\n", V, S, dm, seq, start);

    // run_flash_attn_v2 over [B, H, N, d], causal and not
    const int fB = 2, fH = 3, fN = 70, fd = 64;
    const size_t fs = (size_t)fB * fH * fN * fd;
    std::vector<float> fq(fs), fk(fs), fv(fs);
    for (size_t i = 0; i < fs; ++i) {
        fq[i] = unit_draw();
        fk[i] = unit_draw();
        fv[i] = unit_draw();
    }
    float *dq = upload(fq), *dk = upload(fk), *dv = upload(fv), *dfo = dalloc<float>(fs);
    for (int causal = 0; causal < 2; ++causal) {
        run_flash_attn_v2(fB, fH, fN, fd, dq, dk, dv, dfo, causal != 0);
        save(causal ? "fa_causal" : "fa_full", "O", download(dfo, fs));
    }
    save("fa", "Q", fq);
    save("fa", "K", fk);
    save("fa", "V", fv);
    std::fprintf(g_manifest, "flash fa %d %d %d %d\n", fB, fH, fN, fd);

    // samplers over one logits row
    const int n = 50257;
    std::vector<float> logits(n);
    for (auto& v : logits) v = unit_draw() * 4.0f;
    logits[31337] = 4.5f;  // the maximum, but not a dominant one for the draw
    float* dlog = upload(logits);
    std::vector<int> picks = {sample_argmax(dlog, n), sample_top_k(dlog, n, 40, 0.8f, 42u),
                              sample_top_k(dlog, n, 40, 0.8f, 42u), sample_top_k(dlog, n, 40, 0.8f, 43u)};
    save("samp", "logits", logits);
    save("samp", "picks", picks);
    std::fprintf(g_manifest, "sampler samp %d\n", n);
    for (void* p : {(void*)dx, (void*)dg, (void*)db, (void*)dwte, (void*)dwpe, (void*)demb, (void*)dids,
                    (void*)dq, (void*)dk, (void*)dv, (void*)dfo, (void*)dlog})
        hip_ok(hipFree(p), "hipFree");
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s <out_dir>\n", argv[0]);
        return 2;
    }
    g_dir = argv[1];
    g_manifest = std::fopen((g_dir + "/manifest.txt").c_str(), "w");
    if (!g_manifest) return 4;
    // benchmarks/int8_gemm_bench.cu:16-17
    std::printf("Tile: BM=%d BN=%d BK=%d | Thread tile: TM=%d TN=%d\n", I8_BM, I8_BN, I8_BK, I8_TM, I8_TN);
    std::fprintf(g_manifest, "i8consts k14 %d %d %d %d %d %d\n", I8_BM, I8_BN, I8_BK, I8_TM, I8_TN, I8_NTHREADS);
    // tests/test_int8_gemm.cu:97-101
    const int gemm_shapes[][3] = {{256, 256, 256}, {512, 512, 512}, {1024, 1024, 1024}, {2048, 2048, 2048},
                                  {512, 1024, 256}};
    for (const auto& s : gemm_shapes) gemm_case(s[0], s[1], s[2]);
    // tests/test_decode_attention.cu:144-151
    const int attn_shapes[][4] = {{1, 8, 8, 128}, {1, 16, 16, 512}, {4, 8, 8, 256},
                                  {1, 8, 8, 1024}, {1, 16, 4, 256}, {8, 32, 8, 1024}};
    for (const auto& s : attn_shapes) attn_case(s[0], s[1], s[2], s[3], 64, 16);
    support_cases();
    // tests/test_layernorm.cu:87-91
    const int ln_shapes[][2] = {{1, 768}, {128, 768}, {1, 256}, {64, 768}, {512, 768}};
    for (const auto& s : ln_shapes) layernorm_residual_case(s[0], s[1]);
    std::fclose(g_manifest);
    std::printf("compat_dropin: done\n");
    return 0;
}
