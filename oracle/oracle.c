/*
 * oracle.c — CPU restatement of the reference's quantized decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP library and
 * the CPU baseline that bench.py reports.  Never linked into the product.
 *
 * Built with -ffp-contract=off so every rounding step is the one written
 * here; where the reference's device compiler contracts a multiply-add (nvcc's
 * default -fmad=true), the contraction is written out explicitly with fmaf.
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------------
 * glibc rand(): rand() is random(), whose default state is the TYPE_3
 * additive feedback generator with a 128-byte state.  initstate_r with a
 * private 128-byte buffer selects the same generator without touching the
 * process-global state.  Draw expression: tests/test_int8_gemm.cu:25-28.
 * ---------------------------------------------------------------------- */
typedef struct {
    struct random_data rd;
    char state[128];
} orc_rng;

void* orc_rng_new(unsigned seed) {
    orc_rng* r = (orc_rng*)calloc(1, sizeof(orc_rng));
    if (!r) return NULL;
    initstate_r(seed, r->state, sizeof(r->state), &r->rd);
    srandom_r(seed, &r->rd);
    return r;
}

void orc_rng_free(void* rng) { free(rng); }

int orc_rng_next(void* rng) {
    int32_t v;
    random_r(&((orc_rng*)rng)->rd, &v);
    return (int)v;
}

static float draw_uniform(void* rng) {
    float x = (float)orc_rng_next(rng) / (float)RAND_MAX;
    return x * 2.0f - 1.0f;
}

void orc_rng_uniform(void* rng, float* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = draw_uniform(rng);
}

/* tests/test_decode_attention.cu:70-73: K and V drawn alternately. */
void orc_rng_uniform_pair(void* rng, float* a, float* b, long n) {
    for (long i = 0; i < n; ++i) {
        a[i] = draw_uniform(rng);
        b[i] = draw_uniform(rng);
    }
}

/* ------------------------------------------------------------------------
 * Quantizer, kernels/quantization/14_int8_gemm.cu:10-60.
 *   row_max = max |x|                                   (:21-34)
 *   scale   = row_max > 0 ? row_max / 127 : 1           (:36)
 *   inv     = 1 / scale                                 (:37)
 *   q       = (int8) clamp(rint(x * inv), -128, 127)    (:48-51)
 *   word    = q0 | q1<<8 | q2<<16 | q3<<24              (:53-58)
 * The maximum is exact in any order, so the block reduction is not restated.
 * ---------------------------------------------------------------------- */
static int8_t quant_one(float x, float inv) {
    float r = rintf(x * inv);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    return (int8_t)r;
}

int orc_quantize_fp32_to_int8(int rows, int cols, const float* input,
                              int32_t* output_packed, float* scales) {
    if (rows < 0 || cols < 0 || (cols % 4) != 0) return 1;
    const int pc = cols / 4;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* x = input + (size_t)r * cols;
        float m = 0.0f;
        for (int c = 0; c < cols; ++c) {
            float v = fabsf(x[c]);
            if (v > m) m = v;
        }
        float scale = (m > 0.0f) ? m / 127.0f : 1.0f;
        float inv = 1.0f / scale;
        scales[r] = scale;
        int32_t* o = output_packed + (size_t)r * pc;
        for (int i = 0; i < pc; ++i) {
            uint32_t w = 0;
            for (int j = 0; j < 4; ++j)
                w |= (uint32_t)(uint8_t)quant_one(x[4 * i + j], inv) << (8 * j);
            o[i] = (int32_t)w;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------
 * INT8 GEMM, NT layout: acc[i][j] = sum_k A[i][k] * BT[j][k]  (14_int8_gemm.cu
 * :96-140, each __dp4a adds four byte products).  Exact in int32 while
 * K * 128 * 128 < 2^31.
 * ---------------------------------------------------------------------- */
static void unpack_row(const int32_t* src, int K, int8_t* dst) {
    for (int k = 0; k < K; ++k)
        dst[k] = (int8_t)(((uint32_t)src[k >> 2]) >> (8 * (k & 3)));
}

static int gemm_args_ok(int M, int N, int K) {
    return M >= 0 && N >= 0 && K >= 0 && (K % 4) == 0 && K <= 131068;
}

int orc_int8_gemm_i32(int M, int N, int K, const int32_t* A_packed,
                      const int32_t* BT_packed, int32_t* acc) {
    if (!gemm_args_ok(M, N, K)) return 1;
    const int K4 = K / 4;
    int8_t* bt = (int8_t*)malloc((size_t)N * (K ? K : 1));
    if (!bt) return 2;
#pragma omp parallel for schedule(static)
    for (int j = 0; j < N; ++j) unpack_row(BT_packed + (size_t)j * K4, K, bt + (size_t)j * K);
#pragma omp parallel
    {
        int8_t* a = (int8_t*)malloc((size_t)(K ? K : 1));
#pragma omp for schedule(static)
        for (int i = 0; i < M; ++i) {
            unpack_row(A_packed + (size_t)i * K4, K, a);
            for (int j = 0; j < N; ++j) {
                const int8_t* b = bt + (size_t)j * K;
                int32_t s = 0;
                for (int k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)b[k];
                acc[(size_t)i * N + j] = s;
            }
        }
        free(a);
    }
    free(bt);
    return 0;
}

/* Epilogue, 14_int8_gemm.cu:142-169.  t = (float)acc * sA (:154, left to
 * right); Plain: t * sB.  For the bias forms the reference's compiler contracts
 * "t * sB + bias" into one fused multiply-add, written out here as fmaf; the
 * GELU inner "v + 0.044715 * v^3" likewise (:159-160). */
static float epilogue(int epi, int32_t acc, float sa, float sb, float bias,
                      float res) {
    float t = (float)acc * sa;
    switch (epi) {
        case 0:
            return t * sb;
        case 1:
            return fmaf(t, sb, bias);
        case 2: {
            float v = fmaf(t, sb, bias);
            float x3 = v * v * v;
            float u = 0.7978845608f * fmaf(0.044715f, x3, v);
            return 0.5f * v * (1.0f + tanhf(u));
        }
        default:
            return fmaf(t, sb, bias) + res;
    }
}

int orc_int8_gemm(int M, int N, int K, const int32_t* A_packed,
                  const int32_t* BT_packed, const float* scale_A,
                  const float* scale_B, int epi, const float* bias,
                  const float* residual, float* C) {
    if (!gemm_args_ok(M, N, K) || epi < 0 || epi > 3) return 1;
    if (epi >= 1 && !bias) return 1;
    if (epi == 3 && !residual) return 1;
    const int K4 = K / 4;
    int8_t* bt = (int8_t*)malloc((size_t)N * (K ? K : 1));
    int8_t* at = (int8_t*)malloc((size_t)M * (K ? K : 1));
    if (!bt || !at) {
        free(bt);
        free(at);
        return 2;
    }
#pragma omp parallel for schedule(static)
    for (int j = 0; j < N; ++j) unpack_row(BT_packed + (size_t)j * K4, K, bt + (size_t)j * K);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) unpack_row(A_packed + (size_t)i * K4, K, at + (size_t)i * K);
    /* every (row, column) output on its own: the threads share decode-sized M too */
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < N; ++j) {
            const int8_t* a = at + (size_t)i * K;
            const int8_t* b = bt + (size_t)j * K;
            int32_t s = 0;
            for (int k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)b[k];
            float bv = bias ? bias[j] : 0.0f;
            float rv = residual ? residual[(size_t)i * N + j] : 0.0f;
            C[(size_t)i * N + j] = epilogue(epi, s, scale_A[i], scale_B[j], bv, rv);
        }
    }
    free(at);
    free(bt);
    return 0;
}

void orc_gemm_f64(int M, int N, int K, const float* A, const float* B, double* C) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < M; ++i) {
        double* c = C + (size_t)i * N;
        for (int j = 0; j < N; ++j) c[j] = 0.0;
        for (int k = 0; k < K; ++k) {
            double a = A[(size_t)i * K + k];
            const float* b = B + (size_t)k * N;
            for (int j = 0; j < N; ++j) c[j] += a * (double)b[j];
        }
    }
}

/* ------------------------------------------------------------------------
 * Decode attention.
 * ---------------------------------------------------------------------- */
/* 13_decode_attn.cu:63: num_splits = clamp(max_kv_blocks / 4, 1, 16). */
int orc_decode_num_splits(int max_context_len, int block_size) {
    if (block_size <= 0) return 1;
    int nb = (max_context_len + block_size - 1) / block_size;
    int s = nb / 4;
    if (s < 1) s = 1;
    if (s > 16) s = 16;
    return s;
}

static inline float kv_load(const void* base, int dtype, size_t idx) {
    if (dtype == 0) return ((const float*)base)[idx];
    uint32_t bits = (uint32_t)((const uint16_t*)base)[idx] << 16;
    float f;
    memcpy(&f, &bits, sizeof(f));
    return f;
}

static int attn_args_ok(int B, int H_q, int H_kv, int d, int kv_dtype,
                        int block_size, int num_blocks_per_seq) {
    if (B < 0 || H_q <= 0 || H_kv <= 0 || d <= 0 || block_size <= 0) return 0;
    if (H_q % H_kv) return 0;
    if (kv_dtype != 0 && kv_dtype != 1) return 0;
    if (num_blocks_per_seq < 0) return 0;
    return 1;
}

int orc_decode_attn(int B, int H_q, int H_kv, int d, const float* Q,
                    const void* k_cache, const void* v_cache, int kv_dtype,
                    const int* block_table, const int* context_lens,
                    int max_context_len, int block_size,
                    int num_blocks_per_seq, int num_splits, float* O) {
    if (!attn_args_ok(B, H_q, H_kv, d, kv_dtype, block_size, num_blocks_per_seq)) return 1;
    const int G = H_q / H_kv;
    const float scale_f = 1.0f / sqrtf((float)d);           /* 13_decode_attn.cu:91 */
    const double scale = (double)scale_f;
    const int nb_max = (max_context_len + block_size - 1) / block_size;
    const int S = num_splits > 0 ? num_splits : orc_decode_num_splits(max_context_len, block_size);
    const int bps = S > 0 ? (nb_max + S - 1) / S : 0;       /* :65 */

#pragma omp parallel
    {
        double* o = (double*)malloc(sizeof(double) * (size_t)d);
        double* os = (double*)malloc(sizeof(double) * (size_t)d);
#pragma omp for collapse(2) schedule(dynamic)
        for (int b = 0; b < B; ++b) {
            for (int hq = 0; hq < H_q; ++hq) {
                const int kvh = hq / G;
                const int ctx = context_lens[b];
                const int nb = (ctx + block_size - 1) / block_size;
                const float* q = Q + ((size_t)b * H_q + hq) * d;
                const int* bt = block_table + (size_t)b * num_blocks_per_seq;
                double m_acc = -INFINITY, l_acc = 0.0;
                for (int i = 0; i < d; ++i) o[i] = 0.0;
                for (int s = 0; s < S; ++s) {
                    const int blk0 = s * bps;
                    int blk1 = blk0 + bps;
                    if (blk1 > nb) blk1 = nb;
                    if (blk0 >= nb) continue;                 /* empty split */
                    double m = -INFINITY, l = 0.0;
                    for (int i = 0; i < d; ++i) os[i] = 0.0;
                    for (int blk = blk0; blk < blk1; ++blk) {
                        const long long phys = bt[blk];
                        int ntok = ctx - blk * block_size;
                        if (ntok > block_size) ntok = block_size;
                        for (int t = 0; t < ntok; ++t) {
                            const size_t base =
                                ((size_t)(phys * block_size + t) * H_kv + kvh) * (size_t)d;
                            double dot = 0.0;
                            for (int i = 0; i < d; ++i)
                                dot += (double)q[i] * (double)kv_load(k_cache, kv_dtype, base + i);
                            const double sc = dot * scale;
                            const double mn = sc > m ? sc : m;
                            const double alpha = exp(m - mn);
                            const double p = exp(sc - mn);
                            for (int i = 0; i < d; ++i)
                                os[i] = os[i] * alpha + p * (double)kv_load(v_cache, kv_dtype, base + i);
                            l = l * alpha + p;
                            m = mn;
                        }
                    }
                    /* pass 2 merge, 13_decode_attn.cu:32-47 */
                    if (l_acc == 0.0) {
                        m_acc = m;
                        l_acc = l;
                        for (int i = 0; i < d; ++i) o[i] = os[i];
                    } else {
                        const double mn = m > m_acc ? m : m_acc;
                        const double a = exp(m_acc - mn), be = exp(m - mn);
                        for (int i = 0; i < d; ++i) o[i] = o[i] * a + os[i] * be;
                        l_acc = l_acc * a + l * be;
                        m_acc = mn;
                    }
                }
                float* out = O + ((size_t)b * H_q + hq) * d;
                for (int i = 0; i < d; ++i) out[i] = l_acc > 0.0 ? (float)(o[i] / l_acc) : 0.0f;
            }
        }
        free(o);
        free(os);
    }
    return 0;
}

int orc_decode_attn_f32(int B, int H_q, int H_kv, int d, const float* Q,
                        const void* k_cache, const void* v_cache, int kv_dtype,
                        const int* block_table, const int* context_lens,
                        int max_context_len, int block_size,
                        int num_blocks_per_seq, int num_splits, float* O) {
    enum { NW = 8 };
    if (!attn_args_ok(B, H_q, H_kv, d, kv_dtype, block_size, num_blocks_per_seq)) return 1;
    const int G = H_q / H_kv;
    const float scale = 1.0f / sqrtf((float)d);
    const int nb_max = (max_context_len + block_size - 1) / block_size;
    const int S = num_splits > 0 ? num_splits : orc_decode_num_splits(max_context_len, block_size);
    const int bps = S > 0 ? (nb_max + S - 1) / S : 0;

#pragma omp parallel
    {
        float* wo = (float*)malloc(sizeof(float) * (size_t)d * NW);
        float* so = (float*)malloc(sizeof(float) * (size_t)d);
        float* o = (float*)malloc(sizeof(float) * (size_t)d);
#pragma omp for collapse(2) schedule(dynamic)
        for (int b = 0; b < B; ++b) {
            for (int hq = 0; hq < H_q; ++hq) {
                const int kvh = hq / G;
                const int ctx = context_lens[b];
                const int nb = (ctx + block_size - 1) / block_size;
                const float* q = Q + ((size_t)b * H_q + hq) * d;
                const int* bt = block_table + (size_t)b * num_blocks_per_seq;
                float m_acc = -FLT_MAX, l_acc = 0.0f;
                for (int i = 0; i < d; ++i) o[i] = 0.0f;
                for (int s = 0; s < S; ++s) {
                    const int blk0 = s * bps;
                    int blk1 = blk0 + bps;
                    if (blk1 > nb) blk1 = nb;
                    if (blk0 >= nb) continue;
                    float wm[NW], wl[NW];
                    for (int w = 0; w < NW; ++w) {       /* :78-131, one warp's tokens */
                        float m = -FLT_MAX, l = 0.0f;
                        float* ow = wo + (size_t)w * d;
                        for (int i = 0; i < d; ++i) ow[i] = 0.0f;
                        for (int blk = blk0; blk < blk1; ++blk) {
                            const long long phys = bt[blk];
                            int ntok = ctx - blk * block_size;
                            if (ntok > block_size) ntok = block_size;
                            for (int t = w; t < ntok; t += NW) {
                                const size_t base =
                                    ((size_t)(phys * block_size + t) * H_kv + kvh) * (size_t)d;
                                float dot = 0.0f;
                                for (int i = 0; i < d; ++i)
                                    dot = fmaf(q[i], kv_load(k_cache, kv_dtype, base + i), dot);
                                const float sc = dot * scale;
                                const float mn = fmaxf(m, sc);
                                const float alpha = expf(m - mn);
                                const float p = expf(sc - mn);
                                for (int i = 0; i < d; ++i) ow[i] *= alpha;
                                l = fmaf(l, alpha, p);
                                m = mn;
                                for (int i = 0; i < d; ++i)
                                    ow[i] = fmaf(p, kv_load(v_cache, kv_dtype, base + i), ow[i]);
                            }
                        }
                        wm[w] = m;
                        wl[w] = l;
                    }
                    /* :150-176 warp merge */
                    float mm = wm[0], ml = wl[0];
                    for (int i = 0; i < d; ++i) so[i] = wo[i];
                    for (int w = 1; w < NW; ++w) {
                        if (wl[w] == 0.0f) continue;
                        const float mn = fmaxf(mm, wm[w]);
                        const float a = expf(mm - mn), be = expf(wm[w] - mn);
                        for (int i = 0; i < d; ++i) so[i] = so[i] * a + wo[(size_t)w * d + i] * be;
                        ml = ml * a + wl[w] * be;
                        mm = mn;
                    }
                    /* 13_decode_attn.cu:32-47 split merge */
                    if (ml == 0.0f) continue;
                    const float mn = fmaxf(m_acc, mm);
                    const float a = expf(m_acc - mn), be = expf(mm - mn);
                    for (int i = 0; i < d; ++i) o[i] = o[i] * a + so[i] * be;
                    l_acc = l_acc * a + ml * be;
                    m_acc = mn;
                }
                const float inv_l = l_acc > 0.0f ? 1.0f / l_acc : 0.0f;  /* :50-52 */
                float* out = O + ((size_t)b * H_q + hq) * d;
                for (int i = 0; i < d; ++i) out[i] = o[i] * inv_l;
            }
        }
        free(wo);
        free(so);
        free(o);
    }
    return 0;
}

/* ------------------------------------------------------------------------
 * Paged KV write, src/gpt2_engine.cu:321-346: token t of K/V [seq, H, dh]
 * lands at cache[((phys * bs + (pos % bs)) * H + h) * dh + d] with
 * pos = start_pos + t and phys = block_table[pos / bs].
 * ---------------------------------------------------------------------- */
int orc_kv_cache_write(const float* K_src, const float* V_src, float* k_cache,
                       float* v_cache, const int* block_table, int seq_len,
                       int start_pos, int n_heads, int d_head, int block_size) {
    if (seq_len < 0 || start_pos < 0 || n_heads <= 0 || d_head <= 0 || block_size <= 0) return 1;
    for (int t = 0; t < seq_len; ++t) {
        const int pos = start_pos + t;
        const long long phys = block_table[pos / block_size];
        const int off = pos % block_size;
        for (int h = 0; h < n_heads; ++h) {
            const size_t dst = ((size_t)(phys * block_size + off) * n_heads + h) * (size_t)d_head;
            const size_t src = ((size_t)t * n_heads + h) * (size_t)d_head;
            memcpy(k_cache + dst, K_src + src, sizeof(float) * (size_t)d_head);
            memcpy(v_cache + dst, V_src + src, sizeof(float) * (size_t)d_head);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------
 * Support ops.
 * ---------------------------------------------------------------------- */
/* 15_layernorm_residual.cu:59-103: mean = E[x], var = E[x^2] - mean^2,
 * out = gamma * (x - mean) * rsqrt(var + eps) + beta.  Accumulated in double
 * here (a checker, compared within a stated tolerance). */
void orc_layernorm(int rows, int cols, const float* x, const float* gamma,
                   const float* beta, float* out, float eps) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * cols;
        double s = 0.0, s2 = 0.0;
        for (int c = 0; c < cols; ++c) {
            s += xr[c];
            s2 += (double)xr[c] * xr[c];
        }
        const double mean = s / cols;
        const double var = s2 / cols - mean * mean;
        const double inv = 1.0 / sqrt(var + (double)eps);
        float* o = out + (size_t)r * cols;
        for (int c = 0; c < cols; ++c)
            o[c] = (float)((double)gamma[c] * ((double)xr[c] - mean) * inv + (double)beta[c]);
    }
}

/* 15_layernorm_residual.cu:6-57: y = x + residual in fp32 (one rounding),
 * residual_out = y, out = orc_layernorm(y).  residual_out may alias x or
 * residual (each element is read before it is written). */
void orc_layernorm_residual(int rows, int cols, const float* x, const float* residual,
                            const float* gamma, const float* beta, float* out,
                            float* residual_out, float eps) {
    for (size_t i = 0; i < (size_t)rows * cols; ++i) residual_out[i] = x[i] + residual[i];
    orc_layernorm(rows, cols, residual_out, gamma, beta, out, eps);
}

void orc_embedding(const int* token_ids, int seq_len, int start_pos,
                   int d_model, const float* wte, const float* wpe, float* out) {
    for (int t = 0; t < seq_len; ++t)
        for (int i = 0; i < d_model; ++i)
            out[(size_t)t * d_model + i] = wte[(size_t)token_ids[t] * d_model + i] +
                                           wpe[(size_t)(start_pos + t) * d_model + i];
}

void orc_vocab_proj(const float* hidden, const float* wte, float* logits, int d, int V) {
#pragma omp parallel for schedule(static)
    for (int j = 0; j < V; ++j) {
        double s = 0.0;
        const float* w = wte + (size_t)j * d;
        for (int k = 0; k < d; ++k) s += (double)hidden[k] * w[k];
        logits[j] = (float)s;
    }
}

int orc_argmax(const float* logits, int n) {
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (logits[i] > logits[best]) best = i;
    return best;
}

/* ------------------------------------------------------------------------
 * Top-k sampler, src/sampler.cu:16-45.
 *   k = min(k, V)                                                  (:21)
 *   indices ordered by logit descending, first k kept              (:22-25)
 *     (std::partial_sort leaves equal logits in unspecified order; here the
 *     lower index comes first, the order a stable sort gives)
 *   probs[i] = expf((h[idx[i]] - h[idx[0]]) / temperature), summed (:27-32)
 *   probs[i] /= sum                                                (:33)
 *   r = (float)rand() / RAND_MAX                                   (:35-37)
 *   first i with r < probs[0] + ... + probs[i], else idx[k-1]      (:38-44)
 * ---------------------------------------------------------------------- */
static const float* g_topk_row;

static int topk_cmp(const void* pa, const void* pb) {
    const int a = *(const int*)pa, b = *(const int*)pb;
    const float x = g_topk_row[a], y = g_topk_row[b];
    if (x > y) return -1;
    if (y > x) return 1;
    return a < b ? -1 : (a > b);
}

int orc_topk(int rows, int n, int k, const float* logits, float* vals, int* idx) {
    if (rows < 0 || n <= 0 || k < 1 || k > n) return 1;
    int* order = (int*)malloc(sizeof(int) * (size_t)n);
    if (!order) return 2;
    for (int r = 0; r < rows; ++r) {
        g_topk_row = logits + (size_t)r * n;
        for (int i = 0; i < n; ++i) order[i] = i;
        qsort(order, (size_t)n, sizeof(int), topk_cmp);
        for (int i = 0; i < k; ++i) {
            vals[(size_t)r * k + i] = g_topk_row[order[i]];
            idx[(size_t)r * k + i] = order[i];
        }
    }
    free(order);
    return 0;
}

float orc_rand_unit(void* rng) { return (float)orc_rng_next(rng) / (float)RAND_MAX; }

int orc_top_k_draw(const float* vals, const int* idx, int k, float temperature, float r) {
    float* probs = (float*)malloc(sizeof(float) * (size_t)k);
    if (!probs) return -1;
    const float max_val = vals[0];
    float sum = 0.0f;
    for (int i = 0; i < k; ++i) {
        probs[i] = expf((vals[i] - max_val) / temperature);
        sum += probs[i];
    }
    for (int i = 0; i < k; ++i) probs[i] /= sum;
    float cum = 0.0f;
    int out = idx[k - 1];
    for (int i = 0; i < k; ++i) {
        cum += probs[i];
        if (r < cum) {
            out = idx[i];
            break;
        }
    }
    free(probs);
    return out;
}
