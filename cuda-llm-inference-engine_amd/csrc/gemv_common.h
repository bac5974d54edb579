// gemv_common.h — pieces of the INT8 GEMV shared by gemv_i8.hip and the
// engine's fused QKV projection + attention (qkv_attn.hip): epilogue operand
// loads, the QKV-append store, the fused LayerNorm / quantizer prologue that
// builds an int8 activation row in LDS, and the dot4 / DPP row reduction.
// Both files use them, so the same row gives the same bits in either.
#pragma once

#include <hip/hip_runtime.h>

#include "device_util.h"
#include "epilogue.h"
#include "ie_internal.h"

namespace ie {
namespace {

// Epilogue operands of one output element (scale of its column, bias,
// residual), loaded before the dot products so their latency hides behind
// the weight stream instead of following it.
struct EpiIn {
    float sb = 0.0f, bias = 0.0f, res = 0.0f;
};
template <int EPI>
__device__ __forceinline__ EpiIn epi_load(int m, int n, int N, const float* __restrict__ sB,
                                          const float* bias, const float* residual) {
    EpiIn e;
    if constexpr (EPI != IE_EPI_I32) e.sb = sB[n];
    if constexpr (EPI != IE_EPI_I32 && EPI != IE_EPI_PLAIN) e.bias = bias[n];
    if constexpr (EPI == IE_EPI_BIAS_RESIDUAL) e.res = residual[(size_t)m * N + n];
    return e;
}

// Cache slot of the token each row appends (kEpiQKV): row m writes at
// positions[m] through its block-table row.  The lookups are wave-uniform
// (scalar loads), so they wait on nothing but themselves.
template <int ROWS>
__device__ __forceinline__ void qkv_slots(const GemvFusion& f, int M, size_t (&slot)[ROWS]) {
#pragma unroll
    for (int m = 0; m < ROWS; ++m) {
        slot[m] = 0;
        if (m < M) {
            const int pos = f.positions[m];
            const int blk = pos / f.block_size;
            slot[m] = (size_t)f.table[(size_t)m * f.nbps + blk] * f.block_size + (pos - blk * f.block_size);
        }
    }
}

// Output store of every GEMV kernel: the GEMM epilogues, or (kEpiQKV) the
// bias epilogue routed as the reference's qkv_split + kv_cache_write
// (src/gpt2_engine.cu:292-315, 321-346) would place it: Q [M, d], K and V at
// cache slot `slot` of row m, and ctx_lens[m] = positions[m] + 1.
template <int EPI>
__device__ __forceinline__ void gemv_store(void* C, int m, int n, int N, int32_t acc, float sa,
                                           const EpiIn& e, size_t slot, const GemvFusion& f) {
    if constexpr (EPI == kEpiQKV) {
        const float v = epilogue_value<IE_EPI_BIAS>(acc, sa, e.sb, e.bias, 0.0f);
        const int d = N / 3;
        if (n < d) {
            f.q[(size_t)m * d + n] = v;
            if (n == 0) f.ctx_lens[m] = f.positions[m] + 1;
        } else {
            const bool is_k = n < 2 * d;
            const size_t i = slot * d + (is_k ? n - d : n - 2 * d);
            void* base = is_k ? f.kc : f.vc;
            if (f.kv_dtype == IE_KV_BF16)
                static_cast<uint16_t*>(base)[i] = f32_to_bf16_rne(v);
            else
                static_cast<float*>(base)[i] = v;
        }
    } else {
        store_epilogue_v<EPI>(C, (size_t)m * N + n, acc, sa, e.sb, e.bias, e.res);
    }
}

// One wave builds one int8 activation row of K bytes in LDS (K / 4 words at
// dst) from fp32 row xr: optionally LayerNorm (ln_* as the standalone
// LayerNorm), then the per-row quantizer (quant_scale / quant_word, as
// quant.hip).  So the bytes equal those of the standalone LayerNorm +
// quantizer pair, and do not depend on M or on which kernel stages the row.
// Split into a load phase and a compute phase, so a wave can have several
// rows' loads in flight before it computes any of them.  The LayerNorm's
// gamma/beta (the same for every row) are loaded with the first row
// (ln_load), not after the row's mean and variance: that would be a second
// memory round trip on the prologue's critical path.
template <int K>
struct LnVec {
    float4 g[K / 256], b[K / 256];
};

template <int K, int SRC>
__device__ __forceinline__ void ln_load(const GemvFusion& f, LnVec<K>& p, int lane) {
    if constexpr (SRC == kSrcLnQuant) {
        const float4* g4 = reinterpret_cast<const float4*>(f.gamma);
        const float4* b4 = reinterpret_cast<const float4*>(f.beta);
#pragma unroll
        for (int i = 0; i < K / 256; ++i) {
            p.g[i] = g4[lane + 64 * i];
            p.b[i] = b4[lane + 64 * i];
        }
    }
}

template <int K>
__device__ __forceinline__ void stage_load(const float* __restrict__ xr, float4 (&v)[K / 256], int lane) {
    static_assert(K % 256 == 0, "a lane stages whole float4s");
    const float4* x4 = reinterpret_cast<const float4*>(xr);
#pragma unroll
    for (int i = 0; i < K / 256; ++i) v[i] = x4[lane + 64 * i];
}

template <int K, int SRC>
__device__ __forceinline__ void stage_compute(float4 (&v)[K / 256], const GemvFusion& f, const LnVec<K>& p,
                                              int32_t* dst, float* scale, int lane) {
    constexpr int NV = K / 256;
    if constexpr (SRC == kSrcLnQuant) {
        float s = 0.0f, s2 = 0.0f, mean, rs;
#pragma unroll
        for (int i = 0; i < NV; ++i) ln_accum(v[i], s, s2);
        ln_finish(s, s2, K, f.eps, mean, rs);
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = ln_apply(v[i], p.g[i], p.b[i], mean, rs);
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)),
                             fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    mx = wave_max(mx);
    const float sc = quant_scale(mx);
    const float inv = 1.0f / sc;
#pragma unroll
    for (int i = 0; i < NV; ++i) dst[lane + 64 * i] = quant_word(v[i], inv);
    if (lane == 0) *scale = sc;
}

template <int K, int SRC>
__device__ __forceinline__ void stage_row(const float* __restrict__ xr, const GemvFusion& f,
                                          int32_t* dst, float* scale, int lane) {
    float4 v[K / 256];
    LnVec<K> p;
    stage_load<K>(xr, v, lane);
    ln_load<K, SRC>(f, p, lane);
    stage_compute<K, SRC>(v, f, p, dst, scale, lane);
}

// Rows m >= M of a fused prologue: zero bytes (their outputs are not stored).
template <int K>
__device__ __forceinline__ void zero_row(int32_t* dst, float* scale, int lane) {
#pragma unroll
    for (int i = 0; i < K / 256; ++i) dst[lane + 64 * i] = 0;
    if (lane == 0) *scale = 0.0f;
}

// Shared tail: reduce each row's 16 lane partials with DPP and store.
template <int MT, int EPI>
__device__ __forceinline__ void gemv_finish(const int32_t (&acc)[MT], int li, int n, bool row_ok,
                                            int M, int N, const float* sA, const EpiIn& e,
                                            const size_t (&slot)[MT], void* C,
                                            const GemvFusion& f) {
    int32_t mine = 0;
    size_t my_slot = 0;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int32_t t = row16_sum(acc[m]);
        if (li == m) {
            mine = t;
            my_slot = slot[m];
        }
    }
    if (row_ok && li < M) {
        float sa = 0.0f;
        if constexpr (EPI != IE_EPI_I32) sa = sA[li];
        gemv_store<EPI>(C, li, n, N, mine, sa, e, my_slot, f);
    }
}

template <int MT>
__device__ __forceinline__ void dot_chunk(int32_t (&acc)[MT], const i32x4 wv, const i32x4* a_lds,
                                          int stride, int c) {
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const i32x4 av = a_lds[m * stride + c];
        int32_t s = acc[m];
        s = dot4_i8(wv.x, av.x, s);
        s = dot4_i8(wv.y, av.y, s);
        s = dot4_i8(wv.z, av.z, s);
        s = dot4_i8(wv.w, av.w, s);
        acc[m] = s;
    }
}

}  // namespace
}  // namespace ie
