// gemv_i8.hip — INT8 GEMV for decode-sized M (1..16) on gfx950.
//
// Computes the same sum as the reference's K14 dp4a GEMM
// (kernels/quantization/14_int8_gemm.cu:96-140) followed by its epilogue
// (:142-169), for C[M,N] = A[M,K] * BT[N,K]^T with M <= 16.
//
// The weights BT dominate the traffic (N*K bytes, read once), so the kernel is
// laid out for HBM streaming:
//   * a workgroup owns 16 output features; each wave owns 4 of them and each
//     16-lane DPP row owns one, so a wave's load instruction fetches 4 rows x
//     256 contiguous bytes with 16-byte vector loads;
//   * activations (M*K bytes, tiny) are staged in LDS in 2 KiB-of-K chunks and
//     read back with 16-byte LDS loads, so the weight stream is the only
//     global traffic;
//   * v_dot4_i32_i8 accumulates four byte products per instruction in exact
//     int32 (sum order does not matter for integers);
//   * the 16 partial sums of a feature are combined with four DPP row
//     rotations (no LDS round trip), then lane m of the row stores output m.
// Requires K % 16 == 0 and 16-byte aligned A/BT; other shapes use the generic
// kernel at the end of this file.
#include <algorithm>

#include "device_util.h"
#include "epilogue.h"
#include "ie_internal.h"

namespace ie {
namespace {

constexpr int kRowsPerWG = 16;
constexpr int kChunk = 128;  // 16-byte columns of A per LDS chunk (2 KiB of K)

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
// rows' loads in flight before it computes any of them.
template <int K>
__device__ __forceinline__ void stage_load(const float* __restrict__ xr, float4 (&v)[K / 256], int lane) {
    static_assert(K % 256 == 0, "a lane stages whole float4s");
    const float4* x4 = reinterpret_cast<const float4*>(xr);
#pragma unroll
    for (int i = 0; i < K / 256; ++i) v[i] = x4[lane + 64 * i];
}

template <int K, int SRC>
__device__ __forceinline__ void stage_compute(float4 (&v)[K / 256], const GemvFusion& f, int32_t* dst,
                                              float* scale, int lane) {
    constexpr int NV = K / 256;
    if constexpr (SRC == kSrcLnQuant) {
        float s = 0.0f, s2 = 0.0f, mean, rs;
#pragma unroll
        for (int i = 0; i < NV; ++i) ln_accum(v[i], s, s2);
        ln_finish(s, s2, K, f.eps, mean, rs);
        const float4* g4 = reinterpret_cast<const float4*>(f.gamma);
        const float4* b4 = reinterpret_cast<const float4*>(f.beta);
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = ln_apply(v[i], g4[lane + 64 * i], b4[lane + 64 * i], mean, rs);
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
    stage_load<K>(xr, v, lane);
    stage_compute<K, SRC>(v, f, dst, scale, lane);
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

// K known at compile time (K16 = K / 16 sixteen-byte chunks per row).  Each
// wave walks groups of G x 4 rows; all weight loads of a group (G * K16 / 16
// per lane, 12 for the GPT-2 shapes) are issued together, and the next
// group's loads are issued before the current group is reduced, so every lane
// keeps 12-24 16-byte HBM reads in flight.  The first group's loads are issued
// before the activation block A[M, K] is staged in LDS, so the staging
// latency hides behind them.
//
// With SRC != kSrcInt8 wave w builds activation row w itself (stage_row) while
// the first weight loads are in flight, and the row scales come from LDS.
//
// NT: weight loads are non-temporal (streamed past the caches).  Used for
// weight matrices too large to stay cache-resident between calls; measured
// 10% faster at K = 8192, N = 28672.
template <int MT, int EPI, int K16, int SRC = kSrcInt8, bool NT = false>
__global__ __launch_bounds__(256) void gemv_i8_fixed_kernel(
    int M, int N, const int32_t* __restrict__ A, const int32_t* __restrict__ BT,
    const float* __restrict__ sA, const float* __restrict__ sB, const float* bias,
    const float* residual, void* C, GemvFusion f) {
    constexpr int CPL = K16 / 16;                             // chunks per lane per row
    constexpr int G = CPL >= 12 ? 1 : (12 + CPL - 1) / CPL;   // row groups per pass
    static_assert(CPL <= 32, "fixed-K GEMV covers K <= 8192");
    static_assert(SRC == kSrcInt8 || MT <= 4, "one staging wave per row");
    __shared__ i32x4 a_lds[MT * K16];
    __shared__ float s_sa[MT];
    const int lane = threadIdx.x & 63;
    const int li = lane & 15;
    const int wave_global = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int step = gridDim.x * 4 * (4 * G);
    const i32x4* w4 = reinterpret_cast<const i32x4*>(BT);

    i32x4 wv[G][CPL];
    auto load_group = [&](int r0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int n = r0 + g * 4 + (lane >> 4);
            const i32x4* w = w4 + (size_t)min(n, N - 1) * K16 + li;
#pragma unroll
            for (int t = 0; t < CPL; ++t) {
                if constexpr (NT)
                    wv[g][t] = __builtin_nontemporal_load(w + 16 * t);
                else
                    wv[g][t] = w[16 * t];
            }
        }
    };
    // Epilogue operands of a pass's rows are requested ahead of its weights.
    EpiIn ein[G];
    auto load_epi = [&](int r) {
#pragma unroll
        for (int g = 0; g < G; ++g)
            ein[g] = epi_load<EPI>(min(li, M - 1), min(r + g * 4 + (lane >> 4), N - 1), N, sB, bias,
                                   residual);
    };
    size_t slot[MT];
    if constexpr (EPI == kEpiQKV) qkv_slots<MT>(f, M, slot);
    int r0 = wave_global * (4 * G);
    if (r0 < N) {
        load_epi(r0);
        load_group(r0);
    }

    if constexpr (SRC == kSrcInt8) {
        const i32x4* a4 = reinterpret_cast<const i32x4*>(A);
        for (int i = threadIdx.x; i < MT * K16; i += 256) {
            const int m = i / K16;
            const int mm = m < M ? m : M - 1;
            a_lds[i] = a4[(size_t)mm * K16 + (i - m * K16)];
        }
    } else {
        const int w = threadIdx.x >> 6;
        if (w < MT) {
            int32_t* dst = reinterpret_cast<int32_t*>(a_lds + w * K16);
            if (w < M)
                stage_row<K16 * 16, SRC>(f.x + (size_t)w * K16 * 16, f, dst, &s_sa[w], lane);
            else
                zero_row<K16 * 16>(dst, &s_sa[w], lane);
        }
    }
    __syncthreads();
    const float* sa_src = SRC == kSrcInt8 ? sA : s_sa;

    for (; r0 < N; r0 += step) {
        if constexpr (CPL > 16)
            if (r0 != wave_global * (4 * G)) load_group(r0);
        int32_t acc[G][MT];
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int m = 0; m < MT; ++m) acc[g][m] = 0;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int t = 0; t < CPL; ++t) dot_chunk<MT>(acc[g], wv[g][t], a_lds, K16, li + 16 * t);
        // Next pass in flight during the reduce (K <= 4096: 12-16 loads per
        // lane; at K = 8192 one pass already keeps 32 loads per lane in flight).
        if constexpr (CPL <= 16)
            if (r0 + step < N) load_group(r0 + step);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int n = r0 + g * 4 + (lane >> 4);
            gemv_finish<MT, EPI>(acc[g], li, n, n < N, M, N, sa_src, ein[g], slot, C, f);
        }
        if (r0 + step < N) load_epi(r0 + step);
    }
}

// Any K % 16 == 0: activations staged in LDS in 2 KiB-of-K chunks.
template <int MT, int EPI>
__global__ __launch_bounds__(256) void gemv_i8_kernel(
    int M, int N, int K, const int32_t* __restrict__ A,
    const int32_t* __restrict__ BT, const float* __restrict__ sA,
    const float* __restrict__ sB, const float* bias, const float* residual,
    void* C) {
    __shared__ i32x4 a_lds[MT * kChunk];
    const int lane = threadIdx.x & 63;
    const int li = lane & 15;
    const int n = blockIdx.x * kRowsPerWG + (threadIdx.x >> 6) * 4 + (lane >> 4);
    const bool row_ok = n < N;
    const int K16 = K >> 4;
    const i32x4* w = reinterpret_cast<const i32x4*>(BT) + (size_t)(row_ok ? n : 0) * K16;
    const i32x4* a4 = reinterpret_cast<const i32x4*>(A);

    int32_t acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0;

    for (int c0 = 0; c0 < K16; c0 += kChunk) {
        const int cw = min(kChunk, K16 - c0);
        __syncthreads();
        for (int i = threadIdx.x; i < MT * cw; i += 256) {
            const int m = i / cw;
            const int c = i - m * cw;
            const int mm = m < M ? m : M - 1;  // padded rows re-read a real row
            a_lds[m * kChunk + c] = a4[(size_t)mm * K16 + c0 + c];
        }
        __syncthreads();
        if (row_ok) {
#pragma unroll 8
            for (int c = li; c < cw; c += 16) dot_chunk<MT>(acc, w[c0 + c], a_lds, kChunk, c);
        }
    }
    const size_t no_slot[MT] = {};
    gemv_finish<MT, EPI>(acc, li, n, row_ok, M, N, sA,
                         epi_load<EPI>(min(li, M - 1), row_ok ? n : N - 1, N, sB, bias, residual),
                         no_slot, C, GemvFusion{});
}

// 5 <= M <= 16: v_mfma_i32_16x16x64_i8 with the activations (M padded to 16
// rows) as the A operand and 16 weight rows as the B operand.  A workgroup
// owns 16 output features and its four waves split K four ways (so even
// N = 768 spreads over 48 workgroups), each adding its int32 tile into LDS at
// the end (exact).  Lane l feeds weight row n0 + l % 16, K-bytes
// 16 * (l / 16) .. +16 of each 64-byte K step, so one 16-byte load per lane
// per MFMA streams 1 KiB of weights; dot4 would need 4 instructions per weight
// byte at M = 16, which caps it below HBM speed.  Accumulator v of lane l is
// C[4 * (l / 16) + v][n0 + l % 16].  For K <= 4096 the activation block is
// staged in LDS (or built there by the fused prologue); beyond that each lane
// reads its A fragment straight from global memory (the block is L2-resident).
// Weight loads run U steps ahead of the MFMAs.  With the activations read
// from global memory (K > 4096), NG groups of 16 output features share each
// activation fragment: one A load feeds NG MFMAs, so the activations cost
// 1/NG of the weights' L2 and address traffic instead of as much again.
template <int EPI, int K64, int SRC = kSrcInt8, bool NT = false, int NG = 1>
__global__ __launch_bounds__(256) void gemv_i8_mfma16_kernel(
    int M, int N, const int8_t* __restrict__ A, const int8_t* __restrict__ BT,
    const float* __restrict__ sA, const float* __restrict__ sB, const float* bias,
    const float* residual, void* C, GemvFusion f) {
    constexpr int K = K64 * 64;
    static_assert(K64 % 4 == 0, "four waves split K");
    constexpr int KW = K64 / 4;                // K steps per wave
    constexpr bool A_LDS = K <= 4096;
    static_assert(A_LDS || SRC == kSrcInt8, "fused prologues stage A in LDS");
    static_assert(NG == 1 || (!A_LDS && EPI != kEpiQKV), "feature groups share global activations");
    // weight steps in flight per lane: the largest divisor of KW up to 8
    // (up to 4 with several feature groups, whose loads multiply by NG)
    constexpr int UMAX = NG > 1 ? 4 : 8;
    constexpr int U = KW <= UMAX ? KW : KW % UMAX == 0 ? UMAX : KW % 6 == 0 && UMAX >= 6 ? 6 : KW % 4 == 0 ? 4 : 2;
    static_assert(KW % U == 0, "whole batches");
    __shared__ i32x4 a_lds[A_LDS ? 16 * K / 16 : 1];
    __shared__ float s_sa[16];
    __shared__ i32x4 red[3][NG][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, kq = lane >> 4;
    const int n0 = blockIdx.x * 16 * NG;
    const int kb = wave * KW;  // first K step of this wave

    auto ldw = [&](const int8_t* p) {
        if constexpr (NT)
            return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
        else
            return *reinterpret_cast<const i32x4*>(p);
    };
    // Epilogue operands of this lane's outputs (rows 4 kq + v, column n0 +
    // col; only wave 0 stores) requested ahead of the weights.
    EpiIn ein[NG][4];
    size_t slot[16];
    if (wave == 0) {
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                ein[g][v] = epi_load<EPI>(min(4 * kq + v, M - 1), min(n0 + 16 * g + col, N - 1), N, sB, bias,
                                          residual);
        if constexpr (EPI == kEpiQKV) qkv_slots<16>(f, M, slot);
    }
    const int8_t* w[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) w[g] = BT + (size_t)min(n0 + 16 * g + col, N - 1) * K + kq * 16;
    const int8_t* arow = A + (size_t)min(col, M - 1) * K + kq * 16;  // global A (K > 4096)
    i32x4 wv[U][NG], ag[A_LDS ? 1 : U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
        for (int g = 0; g < NG; ++g) wv[u][g] = ldw(w[g] + (size_t)(kb + u) * 64);
        if constexpr (!A_LDS) ag[u] = *reinterpret_cast<const i32x4*>(arow + (size_t)(kb + u) * 64);
    }

    if constexpr (A_LDS) {
        if constexpr (SRC == kSrcInt8) {
            for (int i = threadIdx.x; i < 16 * (K / 16); i += 256) {
                const int m = i / (K / 16);
                const int mm = m < M ? m : M - 1;
                a_lds[i] = reinterpret_cast<const i32x4*>(A + (size_t)mm * K)[i - m * (K / 16)];
            }
        } else {
            // Wave w builds rows w, w + 4, w + 8, w + 12: RB rows' loads go out
            // together (4 at K <= 1024, 2 at larger K for registers), so the
            // rows cost one memory round trip per batch, not one each.
            constexpr int RB = K <= 1024 ? 4 : 2;
#pragma unroll
            for (int m0 = 0; m0 < 16; m0 += 4 * RB) {
                float4 v[RB][K / 256];
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const int m = m0 + 4 * r + wave;
                    if (m < M) stage_load<K>(f.x + (size_t)m * K, v[r], lane);
                }
#pragma unroll
                for (int r = 0; r < RB; ++r) {
                    const int m = m0 + 4 * r + wave;
                    int32_t* dst = reinterpret_cast<int32_t*>(a_lds + m * (K / 16));
                    if (m < M)
                        stage_compute<K, SRC>(v[r], f, dst, &s_sa[m], lane);
                    else
                        zero_row<K>(dst, &s_sa[m], lane);
                }
            }
        }
        __syncthreads();
    }
    const float* sa_src = SRC == kSrcInt8 ? sA : s_sa;

    // Two accumulators alternate so consecutive MFMAs do not wait on each
    // other; their integer sum is exact.
    i32x4 acc[NG], acc1[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) acc[g] = acc1[g] = i32x4{0, 0, 0, 0};
#pragma unroll 1
    for (int k0 = 0; k0 < KW; k0 += U) {
        i32x4 av[U], cur[U][NG];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if constexpr (A_LDS)
                av[u] = a_lds[col * (K / 16) + (kb + k0 + u) * 4 + kq];
            else
                av[u] = ag[u];
#pragma unroll
            for (int g = 0; g < NG; ++g) cur[u][g] = wv[u][g];
        }
        // next batch's weights (and global A fragments) in flight during the MFMAs
        if (k0 + U < KW) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
#pragma unroll
                for (int g = 0; g < NG; ++g) wv[u][g] = ldw(w[g] + (size_t)(kb + k0 + U + u) * 64);
                if constexpr (!A_LDS) ag[u] = *reinterpret_cast<const i32x4*>(arow + (size_t)(kb + k0 + U + u) * 64);
            }
        }
#pragma unroll
        for (int u = 0; u < U; u += 2)
#pragma unroll
            for (int g = 0; g < NG; ++g) {
                acc[g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u], cur[u][g], acc[g], 0, 0, 0);
                if (u + 1 < U)
                    acc1[g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u + 1], cur[u + 1][g], acc1[g], 0, 0, 0);
            }
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        acc[g] += acc1[g];
        if (wave > 0) red[wave - 1][g][lane] = acc[g];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        acc[g] += red[0][g][lane];
        acc[g] += red[1][g][lane];
        acc[g] += red[2][g][lane];
    }
#pragma unroll
    for (int g = 0; g < NG; ++g) {
    const int n = n0 + 16 * g + col;
    if (n < N) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int m = 4 * kq + v;
            if (m < M) {
                float sa = 0.0f;
                if constexpr (EPI != IE_EPI_I32) sa = sa_src[m];
                size_t sl = 0;
                if constexpr (EPI == kEpiQKV) {
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (kq == q) sl = slot[4 * q + v];
                }
                gemv_store<EPI>(C, m, n, N, acc[g][v], sa, ein[g][v], sl, f);
            }
        }
    }
    }
}

// K = 8192, 2 <= M <= 16: the MFMA GEMV made persistent.  One workgroup per
// CU stages the 16 x K activation block (rows past M repeat row M - 1) in LDS
// once, 128 KiB, and walks 16-feature groups g = blockIdx.x, + gridDim.x, ...;
// its four waves split each group's K four ways and add their int32 tiles in
// LDS (exact), as the per-group kernel does.  The activations cost 32 MiB of
// L2 reads in all instead of as much as the weights, and each wave's weight
// loads run U steps ahead across group boundaries, so the stream does not
// drain between groups.
template <int EPI, int K64, bool NT, int NW>
__global__ __launch_bounds__(64 * NW) void gemv_i8_mfma16_persist_kernel(
    int M, int N, const int8_t* __restrict__ A, const int8_t* __restrict__ BT, const float* __restrict__ sA,
    const float* __restrict__ sB, const float* bias, const float* residual, void* C) {
    constexpr int K = K64 * 64;
    constexpr int KW = K64 / NW;  // K steps per wave and group
    constexpr int U = 8;          // weight steps in flight per lane
    static_assert(KW % U == 0, "whole batches per group");
    constexpr int NB = KW / U;   // batches per group
    __shared__ i32x4 a_lds[16 * K / 16];
    __shared__ i32x4 red[NW - 1][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, kq = lane >> 4;
    const int kb = wave * KW;
    const int ngroups = (N + 15) / 16;
    const int mine = (int)blockIdx.x < ngroups ? (ngroups - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 0;
    const int nbat = mine * NB;

    auto ldw = [&](const int8_t* p) {
        if constexpr (NT)
            return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
        else
            return *reinterpret_cast<const i32x4*>(p);
    };
    // weights of batch bi: group blockIdx.x + (bi / NB) gridDim.x, steps
    // kb + (bi % NB) U .. + U
    auto wrow = [&](int bi) {
        const int g = (int)blockIdx.x + (bi / NB) * (int)gridDim.x;
        return BT + (size_t)min(g * 16 + col, N - 1) * K + kq * 16 + (size_t)(kb + (bi % NB) * U) * 64;
    };
    i32x4 wv[U];
    if (nbat > 0) {
        const int8_t* w = wrow(0);
#pragma unroll
        for (int u = 0; u < U; ++u) wv[u] = ldw(w + (size_t)u * 64);
    }
    for (int i = threadIdx.x; i < 16 * (K / 16); i += 64 * NW) {
        const int m = i / (K / 16);
        a_lds[i] = reinterpret_cast<const i32x4*>(A + (size_t)min(m, M - 1) * K)[i - m * (K / 16)];
    }
    __syncthreads();

    i32x4 acc = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    EpiIn ein[4];
#pragma unroll 1
    for (int bi = 0; bi < nbat; ++bi) {
        const int g = (int)blockIdx.x + (bi / NB) * (int)gridDim.x;
        if (bi % NB == 0 && wave == 0) {
            // the group's epilogue operands, requested with its first weights
#pragma unroll
            for (int v = 0; v < 4; ++v)
                ein[v] = epi_load<EPI>(min(4 * kq + v, M - 1), min(g * 16 + col, N - 1), N, sB, bias, residual);
        }
        i32x4 cur[U];
#pragma unroll
        for (int u = 0; u < U; ++u) cur[u] = wv[u];
        if (bi + 1 < nbat) {  // next batch, possibly the next group's, in flight
            const int8_t* w = wrow(bi + 1);
#pragma unroll
            for (int u = 0; u < U; ++u) wv[u] = ldw(w + (size_t)u * 64);
        }
        const int kk = kb + (bi % NB) * U;
#pragma unroll
        for (int u = 0; u < U; u += 2) {
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_lds[col * (K / 16) + (kk + u) * 4 + kq], cur[u], acc, 0,
                                                        0, 0);
            acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_lds[col * (K / 16) + (kk + u + 1) * 4 + kq], cur[u + 1],
                                                         acc1, 0, 0, 0);
        }
        if (bi % NB == NB - 1) {  // group done (uniform across the workgroup)
            acc += acc1;
            if (wave > 0) red[wave - 1][lane] = acc;
            __syncthreads();
            if (wave == 0) {
#pragma unroll
                for (int w = 0; w < NW - 1; ++w) acc += red[w][lane];
                const int n = g * 16 + col;
                if (n < N) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int m = 4 * kq + v;
                        if (m < M) {
                            float sa = 0.0f;
                            if constexpr (EPI != IE_EPI_I32) sa = sA[m];
                            gemv_store<EPI>(C, m, n, N, acc[v], sa, ein[v], 0, GemvFusion{});
                        }
                    }
                }
            }
            __syncthreads();  // red is rewritten by the next group
            acc = i32x4{0, 0, 0, 0};
            acc1 = i32x4{0, 0, 0, 0};
        }
    }
}

// Any K % 4 == 0 and any alignment: one thread per output element.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(
    int M, int N, int K, const int32_t* __restrict__ A,
    const int32_t* __restrict__ BT, const float* __restrict__ sA,
    const float* __restrict__ sB, const float* bias, const float* residual,
    void* C) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)M * N) return;
    const int m = (int)(idx / N);
    const int n = (int)(idx - (size_t)m * N);
    const int K4 = K >> 2;
    const int32_t* a = A + (size_t)m * K4;
    const int32_t* b = BT + (size_t)n * K4;
    int32_t s = 0;
    for (int k = 0; k < K4; ++k) s = dot4_i8(a[k], b[k], s);
    float sa = 0.0f, sb = 0.0f;
    if constexpr (EPI != IE_EPI_I32) {
        sa = sA[m];
        sb = sB[n];
    }
    store_epilogue<EPI>(C, idx, s, sa, sb, bias, residual, n);
}

// Weight matrices at least this large are streamed with non-temporal loads
// (a quarter of the 256 MiB MALL: larger ones do not stay resident anyway).
constexpr size_t kStreamWeightBytes = 64ull << 20;

template <int MT, int EPI, int K16, int SRC = kSrcInt8>
void launch_fixed(const GemmArgs& a, hipStream_t s, const GemvFusion& f = GemvFusion{}) {
    constexpr int CPL = K16 / 16;
    constexpr int G = CPL >= 12 ? 1 : (12 + CPL - 1) / CPL;
    const int rows_per_wg = 4 * 4 * G;
    const bool nt = (size_t)a.N * K16 * 16 >= kStreamWeightBytes;
    // Streaming shapes: one workgroup per CU walking row groups (each wave
    // keeps a whole group's loads in flight); measured faster than one
    // workgroup per 16 rows, which re-stages the activations in every
    // workgroup and leaves a partial last wave of workgroups.
    const int cap = nt ? num_cus() : 2048;
    const unsigned blocks = (unsigned)min((a.N + rows_per_wg - 1) / rows_per_wg, cap);
    if (nt)
        gemv_i8_fixed_kernel<MT, EPI, K16, SRC, true><<<blocks, 256, 0, s>>>(
            a.M, a.N, a.A, a.BT, a.sA, a.sB, a.bias, a.residual, a.C, f);
    else
        gemv_i8_fixed_kernel<MT, EPI, K16, SRC, false><<<blocks, 256, 0, s>>>(
            a.M, a.N, a.A, a.BT, a.sA, a.sB, a.bias, a.residual, a.C, f);
}

template <int EPI, int K64, int SRC = kSrcInt8, int NG = 1>
void launch_mfma16(const GemmArgs& a, hipStream_t s, const GemvFusion& f = GemvFusion{}) {
    const unsigned blocks = (unsigned)((a.N + 16 * NG - 1) / (16 * NG));
    const bool nt = (size_t)a.N * K64 * 64 >= kStreamWeightBytes;
    auto* k = nt ? gemv_i8_mfma16_kernel<EPI, K64, SRC, true, NG> : gemv_i8_mfma16_kernel<EPI, K64, SRC, false, NG>;
    k<<<blocks, 256, 0, s>>>(a.M, a.N, reinterpret_cast<const int8_t*>(a.A),
                             reinterpret_cast<const int8_t*>(a.BT), a.sA, a.sB, a.bias, a.residual,
                             a.C, f);
}

template <int EPI, int K64>
void launch_mfma16_persist(const GemmArgs& a, hipStream_t s) {
    constexpr int NW = 8;  // 8 waves split each group's K: measured ahead of 4 and 16
    const unsigned blocks = (unsigned)std::min((a.N + 15) / 16, num_cus());
    const bool nt = (size_t)a.N * K64 * 64 >= kStreamWeightBytes;
    auto* k = nt ? gemv_i8_mfma16_persist_kernel<EPI, K64, true, NW> : gemv_i8_mfma16_persist_kernel<EPI, K64, false, NW>;
    k<<<blocks, 64 * NW, 0, s>>>(a.M, a.N, reinterpret_cast<const int8_t*>(a.A),
                                         reinterpret_cast<const int8_t*>(a.BT), a.sA, a.sB, a.bias, a.residual, a.C);
}

template <int EPI, int K, int SRC>
void launch_fused(const GemmArgs& a, const GemvFusion& f, hipStream_t s) {
    if (a.M <= 1) launch_fixed<1, EPI, K / 16, SRC>(a, s, f);
    else if (a.M <= 2) launch_fixed<2, EPI, K / 16, SRC>(a, s, f);
    else if (a.M <= 4) launch_fixed<4, EPI, K / 16, SRC>(a, s, f);
    else launch_mfma16<EPI, K / 64, SRC>(a, s, f);
}

template <int MT, int EPI>
void launch_mt(const GemmArgs& a, hipStream_t s) {
    if constexpr (MT > 4) {
        if (a.K == 768) return launch_mfma16<EPI, 12>(a, s);
        if (a.K == 3072) return launch_mfma16<EPI, 48>(a, s);
    }
    // K = 8192: one row streams best with dot4; from two rows on, the dot4
    // work per pass (no cross-pass prefetch at this K) outlasts the loads, so
    // the MFMA kernel takes over.
    if (a.K == 8192) {
        if constexpr (MT == 1) {
            return launch_fixed<1, EPI, 512>(a, s);
        } else {
            // Measured at N = 8192 and 28672, M = 2..16 (fraction of HBM peak):
            // many groups and M >= 5, the persistent kernel (N = 28672, M = 16:
            // 0.48 -> 0.60); around N = 8192, two feature groups per workgroup
            // (M = 16: 0.41 -> 0.49, M = 2: 0.53 -> 0.57); otherwise one.
            if (a.N >= 16384 && a.M >= 5) return launch_mfma16_persist<EPI, 128>(a, s);
            if (a.N >= 8192 && a.N < 16384) return launch_mfma16<EPI, 128, kSrcInt8, 2>(a, s);
            return launch_mfma16<EPI, 128>(a, s);
        }
    }
    // Specialised K: the GPT-2 widths.
    if constexpr (MT <= 4) {
        if (a.K == 768) return launch_fixed<MT, EPI, 48>(a, s);
        if (a.K == 3072) return launch_fixed<MT, EPI, 192>(a, s);
    }
    const dim3 grid((a.N + kRowsPerWG - 1) / kRowsPerWG);
    gemv_i8_kernel<MT, EPI><<<grid, 256, 0, s>>>(a.M, a.N, a.K, a.A, a.BT, a.sA, a.sB, a.bias,
                                                  a.residual, a.C);
}

template <int EPI>
struct GemvLaunch {
    static void run(const GemmArgs& a, hipStream_t s) {
        if (a.M <= 1) launch_mt<1, EPI>(a, s);
        else if (a.M <= 2) launch_mt<2, EPI>(a, s);
        else if (a.M <= 4) launch_mt<4, EPI>(a, s);
        else if (a.M <= 8) launch_mt<8, EPI>(a, s);
        else launch_mt<16, EPI>(a, s);
    }
};

template <int EPI>
struct GenericLaunch {
    static void run(const GemmArgs& a, hipStream_t s) {
        const size_t total = (size_t)a.M * a.N;
        const unsigned blocks = (unsigned)((total + 255) / 256);
        gemm_i8_generic_kernel<EPI><<<blocks, 256, 0, s>>>(a.M, a.N, a.K, a.A, a.BT, a.sA,
                                                           a.sB, a.bias, a.residual, a.C);
    }
};

bool vec_ok(const GemmArgs& a) {
    return (a.K % 16) == 0 && ((uintptr_t)a.A % 16) == 0 && ((uintptr_t)a.BT % 16) == 0;
}

}  // namespace

// Compute units of the current device (256 on MI355X), looked up once.
int num_cus() {
    static const int n = [] {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
            v = 256;
        return v;
    }();
    return n;
}

void launch_gemv_i8(const GemmArgs& a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    if (vec_ok(a))
        dispatch_epilogue<GemvLaunch>(a.epi, a, s);
    else
        dispatch_epilogue<GenericLaunch>(a.epi, a, s);
}

// The decode step's combinations at the GPT-2 widths: LayerNorm-fed QKV
// (append epilogue), FFN-up (GELU) and INT8 LM head (plain) at K = d = 768;
// quantizer-fed attention-out (K = 768) and FFN-down (K = 3072) with the
// residual epilogue.
bool gemv_fused_supported(int M, int K, int src, int epi) {
    if (M < 1 || M > kGemvMaxM) return false;
    if (src == kSrcLnQuant)
        return K == 768 && (epi == kEpiQKV || epi == IE_EPI_BIAS_GELU || epi == IE_EPI_PLAIN);
    if (src == kSrcQuant) return (K == 768 || K == 3072) && epi == IE_EPI_BIAS_RESIDUAL;
    return false;
}

void launch_gemv_fused(const GemmArgs& a, const GemvFusion& f, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    if (f.src == kSrcLnQuant) {
        if (a.epi == kEpiQKV) return launch_fused<kEpiQKV, 768, kSrcLnQuant>(a, f, s);
        if (a.epi == IE_EPI_BIAS_GELU) return launch_fused<IE_EPI_BIAS_GELU, 768, kSrcLnQuant>(a, f, s);
        return launch_fused<IE_EPI_PLAIN, 768, kSrcLnQuant>(a, f, s);
    }
    if (a.K == 768) return launch_fused<IE_EPI_BIAS_RESIDUAL, 768, kSrcQuant>(a, f, s);
    launch_fused<IE_EPI_BIAS_RESIDUAL, 3072, kSrcQuant>(a, f, s);
}

// Used by the MFMA path for shapes its vector loads cannot cover.
void launch_gemm_i8_generic(const GemmArgs& a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    dispatch_epilogue<GenericLaunch>(a.epi, a, s);
}

}  // namespace ie
