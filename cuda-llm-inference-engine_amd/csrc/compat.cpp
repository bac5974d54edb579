// compat.cpp — the reference's C++ launch signatures (include/ie_compat.h)
// on top of the C ABI.  Null stream, void return; a rejected call prints why
// and leaves its outputs untouched.
#include "ie_compat.h"

#include <cstdio>

namespace {
void report(const char* fn, int st) {
    if (st != IE_OK) std::fprintf(stderr, "ie_amd: %s rejected (%d): %s\n", fn, st, ie_last_error());
}
}  // namespace

// kernels/quantization/14_int8_gemm.cuh:20-23
void run_quantize_fp32_to_int8(int rows, int cols, const float* input, int32_t* output_packed,
                               float* scales) {
    report("run_quantize_fp32_to_int8",
           ie_quantize_fp32_to_int8(rows, cols, input, output_packed, scales, nullptr));
}

// kernels/quantization/14_int8_gemm.cuh:27-32
void run_int8_gemm(int M, int N, int K, const int32_t* A_packed, const int32_t* BT_packed,
                   const float* scale_A, const float* scale_B, float* C) {
    report("run_int8_gemm", ie_int8_gemm(M, N, K, A_packed, BT_packed, scale_A, scale_B,
                                         IE_EPI_PLAIN, nullptr, nullptr, C, nullptr));
}

// kernels/quantization/14_int8_gemm.cuh:38-44
void run_int8_gemm_bias(int M, int N, int K, const int32_t* A_packed, const int32_t* BT_packed,
                        const float* scale_A, const float* scale_B, const float* bias, float* C) {
    report("run_int8_gemm_bias", ie_int8_gemm(M, N, K, A_packed, BT_packed, scale_A, scale_B,
                                              IE_EPI_BIAS, bias, nullptr, C, nullptr));
}

// kernels/quantization/14_int8_gemm.cuh:46-53
void run_int8_gemm_bias_gelu(int M, int N, int K, const int32_t* A_packed,
                             const int32_t* BT_packed, const float* scale_A,
                             const float* scale_B, const float* bias, float* C) {
    report("run_int8_gemm_bias_gelu", ie_int8_gemm(M, N, K, A_packed, BT_packed, scale_A, scale_B,
                                                   IE_EPI_BIAS_GELU, bias, nullptr, C, nullptr));
}

// kernels/quantization/14_int8_gemm.cuh:55-64
void run_int8_gemm_bias_residual(int M, int N, int K, const int32_t* A_packed,
                                 const int32_t* BT_packed, const float* scale_A,
                                 const float* scale_B, const float* bias, const float* residual,
                                 float* C) {
    report("run_int8_gemm_bias_residual",
           ie_int8_gemm(M, N, K, A_packed, BT_packed, scale_A, scale_B, IE_EPI_BIAS_RESIDUAL, bias,
                        residual, C, nullptr));
}

// kernels/decode/13_decode_attn.cuh:192-199.  The caller's workspace is the
// reference's [B, H_q, DA_MAX_SPLITS, d + 2] floats, so the reference split
// rule (at most DA_MAX_SPLITS splits) is used.
void run_decode_attn(int B, int H_q, int H_kv, int d, const float* Q, const float* k_cache,
                     const float* v_cache, const int* block_table, const int* context_lens,
                     int max_context_len, int block_size, int num_blocks_per_seq, float* O,
                     float* workspace) {
    const size_t ws = ie_decode_attn_workspace_bytes(B, H_q, d, DA_MAX_SPLITS);
    report("run_decode_attn",
           ie_decode_attn(B, H_q, H_kv, d, Q, k_cache, v_cache, IE_KV_F32, block_table,
                          context_lens, max_context_len, block_size, num_blocks_per_seq, O,
                          workspace, ws, 0, nullptr));
}

// kernels/flash_attention/10_flash_attn_v2.cuh:7-9
void run_flash_attn_v2(int B, int H, int N, int d, const float* Q, const float* K, const float* V,
                       float* O, bool causal) {
    report("run_flash_attn_v2", ie_flash_attn(B, H, N, d, Q, K, V, O, causal ? 1 : 0, nullptr));
}

// kernels/layernorm/15_layernorm_residual.cuh (run_layernorm)
void run_layernorm(int rows, int cols, const float* x, const float* gamma, const float* beta,
                   float* out, float eps) {
    report("run_layernorm", ie_layernorm(rows, cols, x, gamma, beta, out, eps, nullptr));
}

// kernels/layernorm/15_layernorm_residual.cuh:7-15
void run_layernorm_residual(int rows, int cols, const float* x, const float* residual, const float* gamma,
                            const float* beta, float* out, float* residual_out, float eps) {
    report("run_layernorm_residual",
           ie_layernorm_residual(rows, cols, x, residual, gamma, beta, out, residual_out, eps, nullptr));
}

// kernels/layernorm/15_embed.cuh
void run_embedding(const int* token_ids, int seq_len, int start_pos, int d_model,
                   const float* wte, const float* wpe, float* out) {
    report("run_embedding", ie_embedding(token_ids, seq_len, start_pos, d_model, wte, wpe, out, nullptr));
}
