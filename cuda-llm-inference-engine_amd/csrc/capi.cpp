// capi.cpp — the extern "C" boundary (include/ie_amd.h).
//
// Every entry point validates its arguments before touching HIP, so each
// rejection path is testable on a machine without a GPU, and no kernel ever
// sees a shape it was not written for (the reference's wrappers validate
// nothing: an unsupported GQA group is a silent no-op,
// kernels/decode/13_decode_attn.cu:107, and d != 64 overruns its buffers).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "ie_internal.h"

namespace {
thread_local char g_err[512] = "";

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int check_gemm(int M, int N, int K, const void* A, const void* BT, const float* sA,
               const float* sB, int epi, const float* bias, const float* residual,
               const void* C) {
    using ie::fail;
    if (M < 0 || N < 0 || K < 0) return fail(IE_ERR_INVALID, "int8_gemm: negative size M=%d N=%d K=%d", M, N, K);
    if (K % 4) return fail(IE_ERR_INVALID, "int8_gemm: K=%d is not a multiple of 4", K);
    // |acc| <= K * 128 * 128 must stay below 2^31.
    if (K > 131068) return fail(IE_ERR_UNSUPPORTED, "int8_gemm: K=%d overflows the int32 accumulator", K);
    if (epi < IE_EPI_PLAIN || epi > IE_EPI_I32) return fail(IE_ERR_INVALID, "int8_gemm: unknown epilogue %d", epi);
    const bool any_out = (size_t)M * N > 0;
    if (!any_out) return IE_OK;
    if (!C) return fail(IE_ERR_INVALID, "int8_gemm: C is null");
    if (K > 0 && (!A || !BT)) return fail(IE_ERR_INVALID, "int8_gemm: A or BT is null");
    if (!aligned(A, 4) || !aligned(BT, 4) || !aligned(C, 4))
        return fail(IE_ERR_INVALID, "int8_gemm: A, BT and C must be 4-byte aligned");
    if (epi != IE_EPI_I32 && (!sA || !sB)) return fail(IE_ERR_INVALID, "int8_gemm: scale_A or scale_B is null");
    if ((epi == IE_EPI_BIAS || epi == IE_EPI_BIAS_GELU || epi == IE_EPI_BIAS_RESIDUAL) && !bias)
        return fail(IE_ERR_INVALID, "int8_gemm: epilogue %d needs bias", epi);
    if (epi == IE_EPI_BIAS_RESIDUAL && !residual)
        return fail(IE_ERR_INVALID, "int8_gemm: epilogue BiasResidual needs residual");
    return IE_OK;
}
}  // namespace

namespace ie {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(IE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return IE_OK;
}

int check_decode_attn(int B, int H_q, int H_kv, int d, const float* Q, const void* k_cache, const void* v_cache,
                      int kv_dtype, const int* block_table, const int* context_lens, int max_context_len,
                      int block_size, int num_blocks_per_seq, const float* O, int num_splits, size_t* need_bytes,
                      int* splits) {
    *need_bytes = 0;
    *splits = 1;
    if (B < 0 || H_q <= 0 || H_kv <= 0 || d <= 0)
        return fail(IE_ERR_INVALID, "decode_attn: bad sizes B=%d H_q=%d H_kv=%d d=%d", B, H_q, H_kv, d);
    if (H_q % H_kv) return fail(IE_ERR_INVALID, "decode_attn: H_q=%d not a multiple of H_kv=%d", H_q, H_kv);
    const int G = H_q / H_kv;
    if (G != 1 && G != 2 && G != 4 && G != 8)
        return fail(IE_ERR_UNSUPPORTED, "decode_attn: group size %d not in {1,2,4,8}", G);
    if (d != 64 && d != 128) return fail(IE_ERR_UNSUPPORTED, "decode_attn: head dim %d not in {64,128}", d);
    if (kv_dtype != IE_KV_F32 && kv_dtype != IE_KV_BF16)
        return fail(IE_ERR_INVALID, "decode_attn: unknown kv dtype %d", kv_dtype);
    if (block_size <= 0) return fail(IE_ERR_INVALID, "decode_attn: block_size=%d", block_size);
    if (max_context_len < 0) return fail(IE_ERR_INVALID, "decode_attn: max_context_len=%d", max_context_len);
    const long long nb_max = ((long long)max_context_len + block_size - 1) / block_size;
    if (num_blocks_per_seq < nb_max)
        return fail(IE_ERR_INVALID, "decode_attn: num_blocks_per_seq=%d < ceil(max_context_len/block_size)=%lld",
                    num_blocks_per_seq, nb_max);
    if (B == 0) return IE_OK;
    if (!Q || !O || !block_table || !context_lens || (nb_max > 0 && (!k_cache || !v_cache)))
        return fail(IE_ERR_INVALID, "decode_attn: null pointer");
    if (!aligned(Q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(O, 4))
        return fail(IE_ERR_INVALID, "decode_attn: Q and the caches must be 16-byte aligned");
    if ((long long)B * H_kv > 65535LL * 65535LL || B > 65535 || H_kv > 65535)
        return fail(IE_ERR_UNSUPPORTED, "decode_attn: grid too large");
    *splits = ie_decode_num_splits(max_context_len, block_size, num_splits);
    *need_bytes = ie_decode_attn_workspace_bytes(B, H_q, d, *splits);
    return IE_OK;
}

}  // namespace ie

extern "C" {

const char* ie_last_error(void) { return g_err; }

int ie_version(void) { return 100; }

int ie_init(void) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return ie::fail(IE_ERR_HIP, "ie_init: %s", hipGetErrorString(e));
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return ie::fail(IE_ERR_HIP, "ie_init: %s", hipGetErrorString(e));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return ie::fail(IE_ERR_UNSUPPORTED, "ie_init: device %d is %s, the library is built for gfx950",
                        dev, p.gcnArchName);
    const int st = ie::compat_sampler_init();
    return st != IE_OK ? st : ie::decode_scratch_init();
}

int ie_quantize_fp32_to_int8(int rows, int cols, const float* input, int32_t* output_packed,
                             float* scales, ie_stream_t stream) {
    if (rows < 0 || cols < 0) return ie::fail(IE_ERR_INVALID, "quantize: negative size rows=%d cols=%d", rows, cols);
    if (cols % 4) return ie::fail(IE_ERR_INVALID, "quantize: cols=%d is not a multiple of 4", cols);
    if (rows == 0) return IE_OK;
    if (!input || !scales || (cols > 0 && !output_packed))
        return ie::fail(IE_ERR_INVALID, "quantize: null pointer");
    if (!aligned(input, 16) || !aligned(output_packed, 4) || !aligned(scales, 4))
        return ie::fail(IE_ERR_INVALID, "quantize: input must be 16-byte aligned");
    ie::launch_quantize(rows, cols, input, output_packed, scales, (hipStream_t)stream);
    return ie::check_launch("quantize");
}

int ie_int8_gemm_ex(int M, int N, int K, const int32_t* A_packed, const int32_t* BT_packed,
                    const float* scale_A, const float* scale_B, int epilogue, const float* bias,
                    const float* residual, void* C, int path, ie_stream_t stream) {
    int st = check_gemm(M, N, K, A_packed, BT_packed, scale_A, scale_B, epilogue, bias, residual, C);
    if (st != IE_OK) return st;
    if (path < IE_PATH_AUTO || path > IE_PATH_MFMA) return ie::fail(IE_ERR_INVALID, "int8_gemm: unknown path %d", path);
    if ((size_t)M * N == 0) return IE_OK;
    ie::GemmArgs a{M, N, K, A_packed, BT_packed, scale_A, scale_B, bias, residual, C, epilogue};
    if (path == IE_PATH_AUTO) path = (M <= ie::kGemvMaxM) ? IE_PATH_GEMV : IE_PATH_MFMA;
    if (path == IE_PATH_GEMV) {
        if (M > ie::kGemvMaxM) return ie::fail(IE_ERR_UNSUPPORTED, "int8_gemm: GEMV path takes M <= %d, got %d", ie::kGemvMaxM, M);
        ie::launch_gemv_i8(a, (hipStream_t)stream);
    } else {
        ie::launch_gemm_i8_mfma(a, (hipStream_t)stream);
    }
    return ie::check_launch("int8_gemm");
}

int ie_int8_gemm(int M, int N, int K, const int32_t* A_packed, const int32_t* BT_packed,
                 const float* scale_A, const float* scale_B, int epilogue, const float* bias,
                 const float* residual, float* C, ie_stream_t stream) {
    if (epilogue == IE_EPI_I32) return ie::fail(IE_ERR_INVALID, "int8_gemm: use ie_int8_gemm_ex for int32 output");
    return ie_int8_gemm_ex(M, N, K, A_packed, BT_packed, scale_A, scale_B, epilogue, bias, residual,
                           C, IE_PATH_AUTO, stream);
}

int ie_decode_num_splits(int max_context_len, int block_size, int num_splits) {
    if (block_size <= 0 || max_context_len < 0) return 1;
    const int nb = (int)(((long long)max_context_len + block_size - 1) / block_size);
    int s;
    if (num_splits <= 0) {
        s = nb / 4;  // kernels/decode/13_decode_attn.cu:63
        if (s > IE_DA_REF_MAX_SPLITS) s = IE_DA_REF_MAX_SPLITS;
    } else {
        s = num_splits < IE_DA_MAX_SPLITS ? num_splits : IE_DA_MAX_SPLITS;
        if (s > nb) s = nb;
    }
    return s < 1 ? 1 : s;
}

size_t ie_decode_attn_workspace_bytes(int B, int H_q, int d, int num_splits) {
    if (B < 0 || H_q < 0 || d < 0 || num_splits < 0) return 0;
    return (size_t)B * H_q * num_splits * (d + 2) * sizeof(float);
}

int ie_decode_attn(int B, int H_q, int H_kv, int d, const float* Q, const void* k_cache,
                   const void* v_cache, int kv_dtype, const int* block_table,
                   const int* context_lens, int max_context_len, int block_size,
                   int num_blocks_per_seq, float* O, float* workspace, size_t workspace_bytes,
                   int num_splits, ie_stream_t stream) {
    using ie::fail;
    size_t need = 0;
    int S = 1;
    const int st = ie::check_decode_attn(B, H_q, H_kv, d, Q, k_cache, v_cache, kv_dtype, block_table,
                                         context_lens, max_context_len, block_size, num_blocks_per_seq, O,
                                         num_splits, &need, &S);
    if (st != IE_OK || B == 0) return st;
    if (!workspace) return fail(IE_ERR_INVALID, "decode_attn: null pointer");
    if (!aligned(workspace, 4)) return fail(IE_ERR_INVALID, "decode_attn: workspace must be 4-byte aligned");
    if (workspace_bytes < need)
        return fail(IE_ERR_WORKSPACE, "decode_attn: workspace %zu bytes < %zu for %d splits", workspace_bytes, need, S);
    const long long nb_max = ((long long)max_context_len + block_size - 1) / block_size;
    ie::DecodeArgs a{};
    a.B = B; a.H_q = H_q; a.H_kv = H_kv; a.d = d;
    a.Q = Q; a.k_cache = k_cache; a.v_cache = v_cache; a.kv_dtype = kv_dtype;
    a.block_table = block_table; a.context_lens = context_lens;
    a.block_size = block_size; a.num_blocks_per_seq = num_blocks_per_seq;
    a.num_splits = S;
    a.blocks_per_split = (int)((nb_max + S - 1) / S);  // :65
    a.O = O; a.workspace = workspace;
    ie::launch_decode_attn(a, (hipStream_t)stream);
    return ie::check_launch("decode_attn");
}

int ie_prefill_attn(int B, int P, int H_q, int H_kv, int d, const float* Q, const void* k_cache,
                    const void* v_cache, int kv_dtype, const int* block_table, int num_blocks_per_seq,
                    int block_size, int start_pos, float* O, ie_stream_t stream) {
    using ie::fail;
    if (B < 0 || P < 0 || H_q <= 0 || H_kv <= 0 || d <= 0 || start_pos < 0)
        return fail(IE_ERR_INVALID, "prefill_attn: bad sizes B=%d P=%d H_q=%d H_kv=%d d=%d start=%d", B, P,
                    H_q, H_kv, d, start_pos);
    if (H_q % H_kv) return fail(IE_ERR_INVALID, "prefill_attn: H_q=%d not a multiple of H_kv=%d", H_q, H_kv);
    if (d != 64 && d != 128) return fail(IE_ERR_UNSUPPORTED, "prefill_attn: head dim %d not in {64,128}", d);
    if (kv_dtype != IE_KV_F32 && kv_dtype != IE_KV_BF16)
        return fail(IE_ERR_INVALID, "prefill_attn: unknown kv dtype %d", kv_dtype);
    if (block_size <= 0) return fail(IE_ERR_INVALID, "prefill_attn: block_size=%d", block_size);
    const long long nb = ((long long)start_pos + P + block_size - 1) / block_size;
    if (num_blocks_per_seq < nb)
        return fail(IE_ERR_INVALID, "prefill_attn: num_blocks_per_seq=%d < ceil((start_pos+P)/block_size)=%lld",
                    num_blocks_per_seq, nb);
    if (B == 0 || P == 0) return IE_OK;
    if (!Q || !O || !k_cache || !v_cache || !block_table) return fail(IE_ERR_INVALID, "prefill_attn: null pointer");
    if (!aligned(Q, 16) || !aligned(O, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
        return fail(IE_ERR_INVALID, "prefill_attn: Q, O and the caches must be 16-byte aligned");
    if ((long long)((P + 15) / 16) * H_q * B > 0x7fffffffLL)
        return fail(IE_ERR_UNSUPPORTED, "prefill_attn: grid too large (ceil(P/16) x H_q x B > 2^31 - 1)");
    ie::PrefillArgs a{};
    a.B = B; a.P = P; a.H_q = H_q; a.H_kv = H_kv; a.d = d;
    a.Q = Q; a.k = k_cache; a.v = v_cache; a.kv_dtype = kv_dtype;
    a.paged = true; a.block_table = block_table; a.num_blocks_per_seq = num_blocks_per_seq;
    a.block_size = block_size; a.start_pos = start_pos; a.causal = true; a.O = O;
    ie::launch_prefill_attn(a, (hipStream_t)stream);
    return ie::check_launch("prefill_attn");
}

int ie_flash_attn(int B, int H, int N, int d, const float* Q, const float* K, const float* V, float* O,
                  int causal, ie_stream_t stream) {
    using ie::fail;
    if (B < 0 || H <= 0 || N < 0 || d <= 0)
        return fail(IE_ERR_INVALID, "flash_attn: bad sizes B=%d H=%d N=%d d=%d", B, H, N, d);
    if (d != 64 && d != 128) return fail(IE_ERR_UNSUPPORTED, "flash_attn: head dim %d not in {64,128}", d);
    if (B == 0 || N == 0) return IE_OK;
    if (!Q || !K || !V || !O) return fail(IE_ERR_INVALID, "flash_attn: null pointer");
    if (!aligned(Q, 16) || !aligned(K, 16) || !aligned(V, 16) || !aligned(O, 16))
        return fail(IE_ERR_INVALID, "flash_attn: Q, K, V and O must be 16-byte aligned");
    if ((long long)((N + 15) / 16) * H * B > 0x7fffffffLL)
        return fail(IE_ERR_UNSUPPORTED, "flash_attn: grid too large (ceil(N/16) x H x B > 2^31 - 1)");
    // O is written while other workgroups still read Q, K and V.
    const uintptr_t bytes = (uintptr_t)B * H * N * d * sizeof(float);
    const uintptr_t o0 = (uintptr_t)O, o1 = o0 + bytes;
    for (const float* in : {Q, K, V}) {
        const uintptr_t i0 = (uintptr_t)in, i1 = i0 + bytes;
        if (o0 < i1 && i0 < o1) return fail(IE_ERR_INVALID, "flash_attn: O overlaps Q, K or V");
    }
    ie::PrefillArgs a{};
    a.B = B; a.P = N; a.H_q = H; a.H_kv = H; a.d = d;
    a.Q = Q; a.k = K; a.v = V; a.kv_dtype = IE_KV_F32;
    a.paged = false; a.block_size = 1; a.causal = causal != 0; a.O = O;
    ie::launch_prefill_attn(a, (hipStream_t)stream);
    return ie::check_launch("flash_attn");
}

int ie_kv_cache_write(const float* K_src, const float* V_src, void* k_cache, void* v_cache,
                      int kv_dtype, const int* block_table, int seq_len, int start_pos,
                      int n_heads, int d_head, int block_size, ie_stream_t stream) {
    using ie::fail;
    if (seq_len < 0 || start_pos < 0 || n_heads <= 0 || d_head <= 0 || block_size <= 0)
        return fail(IE_ERR_INVALID, "kv_cache_write: bad sizes");
    if (kv_dtype != IE_KV_F32 && kv_dtype != IE_KV_BF16) return fail(IE_ERR_INVALID, "kv_cache_write: unknown kv dtype");
    if (seq_len == 0) return IE_OK;
    if (!K_src || !V_src || !k_cache || !v_cache || !block_table) return fail(IE_ERR_INVALID, "kv_cache_write: null pointer");
    ie::launch_kv_write(K_src, V_src, k_cache, v_cache, kv_dtype, block_table, seq_len, start_pos,
                        n_heads, d_head, block_size, (hipStream_t)stream);
    return ie::check_launch("kv_cache_write");
}

int ie_kv_cache_append_batch(int B, const float* K_src, const float* V_src, void* k_cache,
                             void* v_cache, int kv_dtype, const int* block_table,
                             int num_blocks_per_seq, const int* positions, int n_heads,
                             int d_head, int block_size, ie_stream_t stream) {
    using ie::fail;
    if (B < 0 || n_heads <= 0 || d_head <= 0 || block_size <= 0 || num_blocks_per_seq <= 0)
        return fail(IE_ERR_INVALID, "kv_cache_append_batch: bad sizes");
    if (kv_dtype != IE_KV_F32 && kv_dtype != IE_KV_BF16)
        return fail(IE_ERR_INVALID, "kv_cache_append_batch: unknown kv dtype");
    if (B == 0) return IE_OK;
    if (!K_src || !V_src || !k_cache || !v_cache || !block_table || !positions)
        return fail(IE_ERR_INVALID, "kv_cache_append_batch: null pointer");
    ie::launch_kv_append_batch(B, K_src, V_src, k_cache, v_cache, kv_dtype, block_table,
                               num_blocks_per_seq, positions, n_heads, d_head, block_size,
                               (hipStream_t)stream);
    return ie::check_launch("kv_cache_append_batch");
}

int ie_layernorm(int rows, int cols, const float* x, const float* gamma, const float* beta,
                 float* out, float eps, ie_stream_t stream) {
    if (rows < 0 || cols <= 0) return ie::fail(IE_ERR_INVALID, "layernorm: bad sizes");
    if (rows == 0) return IE_OK;
    if (!x || !gamma || !beta || !out) return ie::fail(IE_ERR_INVALID, "layernorm: null pointer");
    ie::launch_layernorm(rows, cols, x, gamma, beta, out, eps, (hipStream_t)stream);
    return ie::check_launch("layernorm");
}

int ie_layernorm_residual(int rows, int cols, const float* x, const float* residual, const float* gamma,
                          const float* beta, float* out, float* residual_out, float eps, ie_stream_t stream) {
    if (rows < 0 || cols <= 0) return ie::fail(IE_ERR_INVALID, "layernorm_residual: bad sizes");
    if (rows == 0) return IE_OK;
    if (!x || !residual || !gamma || !beta || !out || !residual_out)
        return ie::fail(IE_ERR_INVALID, "layernorm_residual: null pointer");
    ie::launch_layernorm_residual(rows, cols, x, residual, gamma, beta, out, residual_out, eps,
                                  (hipStream_t)stream);
    return ie::check_launch("layernorm_residual");
}

int ie_embedding(const int* token_ids, int seq_len, int start_pos, int d_model, const float* wte,
                 const float* wpe, float* out, ie_stream_t stream) {
    if (seq_len < 0 || start_pos < 0 || d_model <= 0) return ie::fail(IE_ERR_INVALID, "embedding: bad sizes");
    if (seq_len == 0) return IE_OK;
    if (!token_ids || !wte || !wpe || !out) return ie::fail(IE_ERR_INVALID, "embedding: null pointer");
    ie::launch_embedding(token_ids, seq_len, start_pos, d_model, wte, wpe, out, (hipStream_t)stream);
    return ie::check_launch("embedding");
}

int ie_embedding_batch(int B, const int* token_ids, const int* positions, int d_model,
                       const float* wte, const float* wpe, float* out, ie_stream_t stream) {
    if (B < 0 || d_model <= 0) return ie::fail(IE_ERR_INVALID, "embedding_batch: bad sizes");
    if (B == 0) return IE_OK;
    if (!token_ids || !positions || !wte || !wpe || !out)
        return ie::fail(IE_ERR_INVALID, "embedding_batch: null pointer");
    ie::launch_embedding_batch(B, token_ids, positions, d_model, wte, wpe, out, (hipStream_t)stream);
    return ie::check_launch("embedding_batch");
}

int ie_vocab_proj(int rows, const float* hidden, const float* wte, float* logits, int d, int V,
                  ie_stream_t stream) {
    if (rows < 0 || rows > 16 || d <= 0 || V < 0 || (d % 4))
        return ie::fail(IE_ERR_INVALID, "vocab_proj: rows must be 0..16 and d a multiple of 4");
    if (rows == 0 || V == 0) return IE_OK;
    if (!hidden || !wte || !logits) return ie::fail(IE_ERR_INVALID, "vocab_proj: null pointer");
    if (!aligned(hidden, 16) || !aligned(wte, 16)) return ie::fail(IE_ERR_INVALID, "vocab_proj: 16-byte alignment");
    ie::launch_vocab_proj(rows, hidden, wte, logits, d, V, (hipStream_t)stream);
    return ie::check_launch("vocab_proj");
}

int ie_argmax(int rows, const float* logits, int n, int* out_idx, ie_stream_t stream) {
    if (rows < 0 || n <= 0) return ie::fail(IE_ERR_INVALID, "argmax: bad sizes");
    if (rows == 0) return IE_OK;
    if (!logits || !out_idx) return ie::fail(IE_ERR_INVALID, "argmax: null pointer");
    ie::launch_argmax(rows, logits, n, out_idx, (hipStream_t)stream);
    return ie::check_launch("argmax");
}

int ie_topk(int rows, const float* logits, int n, int k, float* out_vals, int* out_idx, ie_stream_t stream) {
    if (rows < 0 || n <= 0) return ie::fail(IE_ERR_INVALID, "topk: bad sizes");
    if (k < 1 || k > n || k > ie::kTopkMax)
        return ie::fail(IE_ERR_INVALID, "topk: k=%d outside [1, min(n=%d, %d)]", k, n, ie::kTopkMax);
    if (rows == 0) return IE_OK;
    if (!logits || !out_vals || !out_idx) return ie::fail(IE_ERR_INVALID, "topk: null pointer");
    ie::launch_topk(rows, logits, n, k, out_vals, out_idx, (hipStream_t)stream);
    return ie::check_launch("topk");
}

int ie_check_token_ids(int n, const int* ids, int vocab_size) {
    if (n < 0 || vocab_size <= 0) return ie::fail(IE_ERR_INVALID, "token ids: n=%d vocab_size=%d", n, vocab_size);
    if (n > 0 && !ids) return ie::fail(IE_ERR_INVALID, "token ids: null pointer");
    for (int i = 0; i < n; ++i)
        if (ids[i] < 0 || ids[i] >= vocab_size)
            return ie::fail(IE_ERR_INVALID, "token id %d at index %d is outside [0, %d)", ids[i], i, vocab_size);
    return IE_OK;
}

}  // extern "C"
