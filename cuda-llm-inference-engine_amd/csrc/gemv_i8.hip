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
//
// Kernels by shape: gemv_i8_fixed_kernel (dot4, M <= 4, K <= 3072 and the
// fused GPT-2 prologues), gemv_i8_mfma16_kernel (MFMA, 5 <= M <= 16,
// K <= 4096), gemv_i8_burst_kernel (K = 768 / 3072 with N >= 16384 and
// M <= 8: the LM head), and at K = 8192 gemv_i8_parted_kernel (4-feature
// items, M <= 4 or N >= 16384) and gemv_i8_slice_kernel (16-feature groups
// split over K, the rest); gemv_i8_kernel covers any other K.
#include <algorithm>

#include "device_util.h"
#include "epilogue.h"
#include "gemv_common.h"
#include "ie_internal.h"

namespace ie {
namespace {

constexpr int kRowsPerWG = 16;
constexpr int kChunk = 128;  // 16-byte columns of A per LDS chunk (2 KiB of K)

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
template <int MT, int EPI, int K16, int SRC = kSrcInt8, bool NT = false, int GF = 0, int NW = 4>
__global__ __launch_bounds__(64 * NW) void gemv_i8_fixed_kernel(
    int M, int N, const int32_t* __restrict__ A, const int32_t* __restrict__ BT,
    const float* __restrict__ sA, const float* __restrict__ sB, const float* bias,
    const float* residual, void* C, GemvFusion f) {
    constexpr int CPL = K16 / 16;                             // chunks per lane per row
    constexpr int G = GF > 0 ? GF : CPL >= 12 ? 1 : (12 + CPL - 1) / CPL;   // row groups per pass
    static_assert(CPL <= 32, "fixed-K GEMV covers K <= 8192");
    static_assert(SRC == kSrcInt8 || MT <= NW, "one staging wave per row");
    __shared__ i32x4 a_lds[MT * K16];
    __shared__ float s_sa[MT];
    const int lane = threadIdx.x & 63;
    const int li = lane & 15;
    const int wave_global = blockIdx.x * NW + (threadIdx.x >> 6);
    const int step = gridDim.x * NW * (4 * G);
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
        for (int i = threadIdx.x; i < MT * K16; i += 64 * NW) {
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

// 5 <= M <= 16, K <= 4096: v_mfma_i32_16x16x64_i8 with the activations (M
// padded to 16 rows) as the A operand and 16 weight rows as the B operand.  A
// workgroup owns 16 output features and its NWV waves (4, or 8 at long K)
// split K (so even N = 768 spreads over 48 workgroups), each adding its int32
// tile into LDS at the end (exact).  Lane l feeds weight row n0 + l % 16, K-bytes
// 16 * (l / 16) .. +16 of each 64-byte K step, so one 16-byte load per lane
// per MFMA streams 1 KiB of weights; dot4 would need 4 instructions per weight
// byte at M = 16, which caps it below HBM speed.  Accumulator v of lane l is
// C[4 * (l / 16) + v][n0 + l % 16].  The activation block is staged in LDS
// (or built there by the fused prologue); weight loads run U steps ahead of
// the MFMAs.
template <int EPI, int K64, int SRC = kSrcInt8, bool NT = false, int NWV = 4, int RS = 16, int FW = 16>
__global__ __launch_bounds__(64 * NWV) void gemv_i8_mfma16_kernel(
    int M, int N, const int8_t* __restrict__ A, const int8_t* __restrict__ BT,
    const float* __restrict__ sA, const float* __restrict__ sB, const float* bias,
    const float* residual, void* C, GemvFusion f) {
    constexpr int K = K64 * 64;
    // Workgroup (x, y) takes rows y RS .. y RS + RS - 1 (the MFMA tile keeps
    // 16 rows; rows past the workgroup's are never stored, and a row's sums
    // do not depend on the others, so every split gives the same bits).
    if constexpr (RS < 16) {
        static_assert(EPI != kEpiQKV, "QKV rows carry cache slots");
        const int m0 = blockIdx.y * RS;
        M = min(M - m0, RS);
        if (A) A += (size_t)m0 * K;
        if (sA) sA += m0;
        if (residual) residual += (size_t)m0 * N;
        C = static_cast<char*>(C) + (size_t)m0 * N * 4;
        if (f.x) f.x += (size_t)m0 * K;
    }
    static_assert(K64 % NWV == 0, "the waves split K evenly");
    static_assert(K <= 4096, "the activation block fits LDS");
    constexpr int KW = K64 / NWV;  // K steps per wave
    // weight steps in flight per lane: the largest divisor of KW up to 8
    constexpr int U = KW <= 8 ? KW : KW % 8 == 0 ? 8 : KW % 6 == 0 ? 6 : KW % 4 == 0 ? 4 : 2;
    static_assert(KW % U == 0, "whole batches");
    __shared__ i32x4 a_lds[16 * K / 16];
    __shared__ float s_sa[16];
    __shared__ i32x4 red[NWV - 1][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, kq = lane >> 4;
    // FW < 16 features per workgroup (so a small N still covers every CU):
    // columns FW .. 15 re-read feature FW - 1 (the same lines, fetched once)
    // and are not stored.
    static_assert(FW == 16 || (FW < 16 && EPI != kEpiQKV), "QKV rows keep 16 features");
    const int n0 = blockIdx.x * FW;
    const int kb = wave * KW;  // first K step of this wave

    auto ldw = [&](const int8_t* p) {
        if constexpr (NT)
            return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
        else
            return *reinterpret_cast<const i32x4*>(p);
    };
    // Epilogue operands of this lane's outputs (rows 4 kq + v, column n0 +
    // col; only wave 0 stores) requested ahead of the weights.
    EpiIn ein[4];
    size_t slot[16];
    if (wave == 0) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
            ein[v] = epi_load<EPI>(min(4 * kq + v, M - 1), min(n0 + col, N - 1), N, sB, bias, residual);
        if constexpr (EPI == kEpiQKV) qkv_slots<16>(f, M, slot);
    }
    const int8_t* w = BT + (size_t)min(n0 + min(col, FW - 1), N - 1) * K + kq * 16;
    i32x4 wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) wv[u] = ldw(w + (size_t)(kb + u) * 64);

    if constexpr (SRC == kSrcInt8) {
        for (int i = threadIdx.x; i < 16 * (K / 16); i += 64 * NWV) {
            const int m = i / (K / 16);
            const int mm = m < M ? m : M - 1;
            a_lds[i] = reinterpret_cast<const i32x4*>(A + (size_t)mm * K)[i - m * (K / 16)];
        }
    } else {
        // Wave w builds rows w, w + NWV, ...: RB rows' loads go out together
        // (4 at K <= 1024, 2 at larger K for registers), so the rows cost one
        // memory round trip per batch, not one each.
        constexpr int RB = K <= 1024 ? 4 : 2;
        LnVec<K> p;
#pragma unroll
        for (int m0 = 0; m0 < 16; m0 += NWV * RB) {
            float4 v[RB][K / 256];
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const int m = m0 + NWV * r + wave;
                if (m < M) stage_load<K>(f.x + (size_t)m * K, v[r], lane);
            }
            if (m0 == 0) ln_load<K, SRC>(f, p, lane);
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const int m = m0 + NWV * r + wave;
                int32_t* dst = reinterpret_cast<int32_t*>(a_lds + m * (K / 16));
                if (m < M)
                    stage_compute<K, SRC>(v[r], f, p, dst, &s_sa[m], lane);
                else
                    zero_row<K>(dst, &s_sa[m], lane);
            }
        }
    }
    __syncthreads();
    const float* sa_src = SRC == kSrcInt8 ? sA : s_sa;

    // Two accumulators alternate so consecutive MFMAs do not wait on each
    // other; their integer sum is exact.
    i32x4 acc = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
#pragma unroll 1
    for (int k0 = 0; k0 < KW; k0 += U) {
        i32x4 av[U], cur[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            av[u] = a_lds[col * (K / 16) + (kb + k0 + u) * 4 + kq];
            cur[u] = wv[u];
        }
        // next batch's weights in flight during the MFMAs
        if (k0 + U < KW) {
#pragma unroll
            for (int u = 0; u < U; ++u) wv[u] = ldw(w + (size_t)(kb + k0 + U + u) * 64);
        }
#pragma unroll
        for (int u = 0; u < U; u += 2) {
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u], cur[u], acc, 0, 0, 0);
            if (u + 1 < U) acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[u + 1], cur[u + 1], acc1, 0, 0, 0);
        }
    }
    acc += acc1;
    if (wave > 0) red[wave - 1][lane] = acc;
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < NWV - 1; ++w) acc += red[w][lane];
    const int n = n0 + col;
    if (n < N && col < FW) {
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
                gemv_store<EPI>(C, m, n, N, acc[v], sa, ein[v], sl, f);
            }
        }
    }
}

// K = 8192, 2 <= M <= 16: one wave per (16-feature group, K slice).
//
// The weights are the only HBM stream, so the rate is set by how many of
// their loads each CU keeps in flight.  A workgroup of 8 waves (one per CU:
// the activation block fills its LDS) gives each wave one group's K range of
// 8192 / KS bytes, KS = 2^ks_log slices per group chosen by the launcher so
// that every wave of the GPU has work.  A wave streams its range through a
// ring of R register sets of U 16-byte loads: set r is refilled right after
// its MFMAs, so (R - 1) U loads stay in flight while one set is consumed, and
// no register copy forces an early wait.  MFMA operands as in the kernels
// above: lane (col, kq) supplies feature col's and activation row col's
// K-bytes 64 s + 16 kq .. + 16 of step s.  The M activation rows sit in LDS
// with rows padded to K + 16 bytes, so the 16 lanes reading one K chunk of 16
// rows fall on distinct banks; rows past M read row M - 1 (results
// discarded).  KS > 1: a group's slices are waves of one workgroup that add
// their int32 tiles in LDS (exact), and each wave has at most one group (the
// launcher sizes the grid so).  KS = 1: waves walk groups g, g + 8 gridDim.x,
// ... and store each as it completes.
// MR: activation rows staged (8 when M <= 8: LDS rows 8-15 then hold
// whatever they held, and only feed results that are not stored).
template <int EPI, bool NT, int R, int MR = 16>
__global__ __launch_bounds__(512) void gemv_i8_slice_kernel(int M, int N, int ks_log, const int8_t* __restrict__ A,
                                                            const int8_t* __restrict__ BT,
                                                            const float* __restrict__ sA,
                                                            const float* __restrict__ sB, const float* bias,
                                                            const float* residual, void* C) {
    constexpr int K = 8192, U = 8, LDA = K + 16;
    constexpr int SB_LOG = 4;  // log2(128 / U)
    __shared__ __attribute__((aligned(16))) int8_t a_lds[16 * LDA];
    __shared__ i32x4 red[8][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kq = lane >> 4;
    const int ks = 1 << ks_log;
    const int slice = wave & (ks - 1), gslot = wave >> ks_log;
    const int nb_log = SB_LOG - ks_log;  // batches of U steps per item: 128 / ks / U (>= R)
    const int nb = 1 << nb_log;
    const int ngroups = (N + 15) / 16;
    const int gstride = (int)gridDim.x * (8 >> ks_log);
    const int g0 = (int)blockIdx.x + (int)gridDim.x * gslot;
    const int nitems = g0 < ngroups ? (ngroups - 1 - g0) / gstride + 1 : 0;
    const int total = nitems << nb_log;  // this wave's batches
    const int kbyte0 = slice * (K >> ks_log);

    auto ldw = [&](const int8_t* p) {
        if constexpr (NT)
            return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
        else
            return *reinterpret_cast<const i32x4*>(p);
    };
    // first weight byte of batch b: item b >> nb_log, steps (b & (nb - 1)) U ..
    auto wptr = [&](int b) {
        const int g = g0 + (b >> nb_log) * gstride;
        return BT + (size_t)min(g * 16 + col, N - 1) * K + kbyte0 + (b & (nb - 1)) * (U * 64) + kq * 16;
    };

    // Issue order: activation rows, row scales, then the ring's first R
    // batches; loads retire in order, so the LDS stores below wait only for
    // the rows.  Rows past M repeat row M - 1 (never stored): unconditional
    // loads, which a conditional one per row would serialise (each branch
    // waited for its load).
    i32x4 stage[MR];
#pragma unroll
    for (int j = 0; j < MR; ++j) stage[j] = reinterpret_cast<const i32x4*>(A + (size_t)min(j, M - 1) * K)[threadIdx.x];
    float sa[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) sa[v] = EPI != IE_EPI_I32 ? sA[min(4 * kq + v, M - 1)] : 0.0f;
    // (unconditional: a wave without a group loads valid rows it never uses,
    // and the compiler can count every set as issued)
    i32x4 w[R][U];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int8_t* p = wptr(r);
#pragma unroll
        for (int u = 0; u < U; ++u) w[r][u] = ldw(p + u * 64);
    }
#pragma unroll
    for (int j = 0; j < MR; ++j) reinterpret_cast<i32x4*>(a_lds + j * LDA)[threadIdx.x] = stage[j];
    __syncthreads();

    auto finish = [&](int g, const i32x4& acc) {
        const int n = g * 16 + col;
        EpiIn e[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) e[v] = epi_load<EPI>(min(4 * kq + v, M - 1), min(n, N - 1), N, sB, bias, residual);
        if (n < N) {
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (4 * kq + v < M) gemv_store<EPI>(C, 4 * kq + v, n, N, acc[v], sa[v], e[v], 0, GemvFusion{});
        }
    };

    // Two accumulators alternate so consecutive MFMAs do not wait on each
    // other; their integer sum is exact.
    i32x4 acc0 = {0, 0, 0, 0}, acc1 = {0, 0, 0, 0};
    const int8_t* arow = a_lds + min(col, M - 1) * LDA + kbyte0 + kq * 16;
    // One pass over the R sets: MFMAs on set r (batch b + r), then, if REFILL,
    // set r reloaded with batch b + r + R.  total is a multiple of R (ks <= 4),
    // so every body but the last refills all its sets, and the waits count
    // the R - 1 sets issued after each one.
    auto body = [&](int b, auto refill) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int bi = b + r;
            const int8_t* ap = arow + (bi & (nb - 1)) * (U * 64);
#pragma unroll
            for (int u = 0; u < U; u += 2) {
                acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const i32x4*>(ap + u * 64), w[r][u],
                                                             acc0, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(*reinterpret_cast<const i32x4*>(ap + (u + 1) * 64),
                                                             w[r][u + 1], acc1, 0, 0, 0);
            }
            if constexpr (decltype(refill)::value) {
                const int8_t* p = wptr(bi + R);
#pragma unroll
                for (int u = 0; u < U; ++u) w[r][u] = ldw(p + u * 64);
            }
            if (ks_log == 0 && (bi & (nb - 1)) == nb - 1) {
                finish(g0 + (bi >> nb_log) * gstride, acc0 + acc1);
                acc0 = acc1 = i32x4{0, 0, 0, 0};
            }
        }
    };
    int b = 0;
#pragma unroll 1
    for (; b + R < total; b += R) body(b, std::true_type{});
    if (total > 0) body(b, std::false_type{});
    if (ks_log > 0) {
        acc0 += acc1;
        if (slice > 0 && nitems > 0) red[wave][lane] = acc0;
        __syncthreads();
        if (slice == 0 && nitems > 0) {
            for (int t = 1; t < ks; ++t) acc0 += red[wave + t][lane];
            finish(g0, acc0);
        }
    }
}

// K = 8192, M <= 4 MB: the MFMA GEMV over 4-feature items, K in four parts.
//
// The weight stream runs fastest when each load instruction reads a few rows
// with long runs, one row set finished before the next starts (4 rows x 256
// bytes per wave instruction, walked row set by row set, streams about 15%
// faster than the 16 rows x 64 bytes of a 16-feature MFMA fragment).  So here
// the 16 columns of v_mfma_i32_16x16x64_i8 are 4 features x 4 K-parts and its
// 16 rows are 4 activation rows x the same 4 parts: column c is feature c / 4,
// part c % 4 (row r likewise), and at step s (256 K-bytes) lane (c, q)
// supplies bytes 256 s + 16 (4 q + c % 4) .. + 16 of its feature (B) and of
// its activation row (A).  Row r and column c pair equal K positions exactly
// when r % 4 == c % 4; those entries hold each part's int32 sum, the rest are
// discarded, and the four parts (the four lanes of a quad) are added with
// DPP at the end (exact).  A wave instruction loads 4 rows x 256 contiguous
// bytes, 64 contiguous bytes per lane quad.  MB blocks of 4 activation rows
// each take one MFMA per weight fragment.
//
// One item = 4 features x all of K = 32 steps = R (4) batches of U (8)
// loads: one pass over the register ring.  Waves walk items b + gridDim.x w,
// + 8 gridDim.x, ...; each pass refills the ring with the next item's
// weights, so the stream does not drain between items, and requests the next
// item's epilogue operands after storing the current one's, so no wait
// covers more than the loads issued before it.
template <int EPI, bool NT, int MB>
__global__ __launch_bounds__(512) void gemv_i8_parted_kernel(int M, int N, const int8_t* __restrict__ A,
                                                             const int8_t* __restrict__ BT,
                                                             const float* __restrict__ sA,
                                                             const float* __restrict__ sB, const float* bias,
                                                             const float* residual, void* C) {
    // LDS rows padded to K + 64 bytes: the 16 lanes reading one step's
    // fragments (4 rows x 4 parts) fall on distinct banks.
    constexpr int K = 8192, U = 8, R = 4, LDA = K + 64;
    static_assert(R * U * 256 == K, "one item per ring pass");
    __shared__ __attribute__((aligned(16))) int8_t a_lds[4 * MB * LDA];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, q = lane >> 4;
    const int part = col & 3, f = col >> 2;
    const int nitems_all = (N + 3) / 4;
    const int stride = (int)gridDim.x * 8;
    const int i0 = (int)blockIdx.x + (int)gridDim.x * wave;
    const int nitems = i0 < nitems_all ? (nitems_all - 1 - i0) / stride + 1 : 0;

    auto ldw = [&](const int8_t* p) {
        if constexpr (NT)
            return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
        else
            return *reinterpret_cast<const i32x4*>(p);
    };
    const int kofs = (4 * q + part) * 16;  // this lane's 16 bytes within a step
    const int8_t* bt = opaque_global(BT);
    auto wrow = [&](int t) {  // feature f of the wave's item t
        return bt + (size_t)min(4 * (i0 + t * stride) + f, N - 1) * K + kofs;
    };
    // The lane's output of an item: block part (when part < MB), row
    // 4 part + q of C, feature f; the epilogue operands are read clamped.
    const int out_m = 4 * part + q;
    const bool out_ok = part < MB && out_m < M;
    const int m_c = min(out_m, M - 1);
    auto out_n = [&](int t) { return 4 * (i0 + t * stride) + f; };

    // Issue order: activation rows, the first item's weights, its epilogue
    // operands; the LDS stores wait only for the rows.  Rows past M repeat
    // row M - 1 (never used for a stored result): unconditional loads, which
    // a conditional one per row would serialise (each branch waited for its
    // load: N = K = 8192, M = 4 12.43 -> 11.95 us).
    i32x4 stage[4 * MB];
#pragma unroll
    for (int j = 0; j < 4 * MB; ++j)
        stage[j] = reinterpret_cast<const i32x4*>(A + (size_t)min(j, M - 1) * K)[threadIdx.x];
    i32x4 w[R][U];
    {
        const int8_t* p = wrow(0);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int u = 0; u < U; ++u) w[r][u] = ldw(p + (r * U + u) * 256);
    }
    const float sa = EPI != IE_EPI_I32 ? sA[m_c] : 0.0f;
    EpiIn e = epi_load<EPI>(m_c, min(out_n(0), N - 1), N, sB, bias, residual);
#pragma unroll
    for (int j = 0; j < 4 * MB; ++j) reinterpret_cast<i32x4*>(a_lds + j * LDA)[threadIdx.x] = stage[j];
    __syncthreads();

    // A operand of block j: activation row 4 j + f (clamped to M - 1; those
    // rows' results are never stored), the same 16 bytes as B.
    const int8_t* arow[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) arow[j] = a_lds + min(4 * j + f, M - 1) * LDA + kofs;

    auto pass = [&](int t, auto refill) {
        i32x4 acc[MB][2];
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[j][0] = acc[j][1] = i32x4{0, 0, 0, 0};
        const int8_t* pn = wrow(t + 1);
        // The activation fragments are the same for every item; an opaque
        // zero offset keeps the compiler from hoisting all 32 of them into
        // registers, where they would crowd out the ring.
        int aofs = 0;
        asm volatile("" : "+v"(aofs));
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int s = r * U + u;
#pragma unroll
                for (int j = 0; j < MB; ++j)
                    acc[j][u & 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        *reinterpret_cast<const i32x4*>(arow[j] + aofs + s * 256), w[r][u], acc[j][u & 1], 0, 0, 0);
            }
            if constexpr (decltype(refill)::value) {
#pragma unroll
                for (int u = 0; u < U; ++u) w[r][u] = ldw(pn + (r * U + u) * 256);
            }
            // keep each set's refill right behind its MFMAs (the compiler
            // would otherwise sink all refills to the end of the pass)
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
        }
        // acc[j][.][v] of lane (c, q) is row 4 q + v of block j: part v of
        // activation row 4 j + q.  Keep v = c % 4 (the matching part), add
        // the quad's four parts; then lane (part, f, q) takes block part.
        int32_t mine = 0;
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            const i32x4 x4 = acc[j][0] + acc[j][1];
            int32_t x = part == 0 ? x4[0] : part == 1 ? x4[1] : part == 2 ? x4[2] : x4[3];
            x += __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xf, 0xf, false);  // quad_perm [1, 0, 3, 2]
            x += __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xf, 0xf, false);  // quad_perm [2, 3, 0, 1]
            mine = part == j ? x : mine;
        }
        const int n = out_n(t);
        if (out_ok && n < N) gemv_store<EPI>(C, out_m, n, N, mine, sa, e, 0, GemvFusion{});
        if constexpr (decltype(refill)::value) e = epi_load<EPI>(m_c, min(out_n(t + 1), N - 1), N, sB, bias, residual);
    };
    if (nitems > 0) {
        int t = 0;
#pragma unroll 1
        for (; t + 1 < nitems; ++t) pass(t, std::true_type{});
        pass(t, std::false_type{});
    }
}

// K = 256 S <= 3072 (the GPT-2 widths), M <= 4 MB: the 4-feature-item MFMA
// GEMV above without a ring.  An item is only S load steps, so each wave
// takes IPW consecutive items (4 IPW rows, one contiguous run of weights),
// issues all their loads and epilogue operands at once, then computes item by
// item; the workgroups are small (4 waves, M x K bytes of LDS) and all
// resident at once, so a GEMV of any width is one memory round trip plus its
// transfer (the 768 x 50257 LM head: 38.6 MB in flight together).
template <int EPI, bool NT, int MB, int S, int IPW>
__global__ __launch_bounds__(256) void gemv_i8_burst_kernel(int M, int N, const int8_t* __restrict__ A,
                                                            const int8_t* __restrict__ BT,
                                                            const float* __restrict__ sA,
                                                            const float* __restrict__ sB, const float* bias,
                                                            const float* residual, void* C) {
    constexpr int K = 256 * S, LDA = K + 64;  // padded rows: conflict-free reads
    constexpr int CH = 4 * MB * (K / 16);      // 16-byte chunks of the activation block
    __shared__ __attribute__((aligned(16))) int8_t a_lds[4 * MB * LDA];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, q = lane >> 4;
    const int part = col & 3, f = col >> 2;
    const int nitems_all = (N + 3) / 4;
    const int i0 = ((int)blockIdx.x * 4 + wave) * IPW;
    const int kofs = (4 * q + part) * 16;
    const int out_m = 4 * part + q;
    const bool out_ok = part < MB && out_m < M;
    const int m_c = min(out_m, M - 1);

    auto ldw = [&](const int8_t* p) {
        if constexpr (NT)
            return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
        else
            return *reinterpret_cast<const i32x4*>(p);
    };
    // Issue order: activation rows (rows past M repeat row M - 1), every
    // item's weights (rows past N repeat row N - 1), epilogue operands.
    constexpr int SPT = (CH + 255) / 256;  // staging chunks per thread
    i32x4 stage[SPT];
#pragma unroll
    for (int c = 0; c < SPT; ++c) {
        const int ch = threadIdx.x + 256 * c;
        if (CH % 256 == 0 || ch < CH) {
            const int r = ch / (K / 16);
            stage[c] = reinterpret_cast<const i32x4*>(A + (size_t)min(r, M - 1) * K)[ch - r * (K / 16)];
        }
    }
    i32x4 w[IPW][S];
#pragma unroll
    for (int it = 0; it < IPW; ++it) {
        const int8_t* p = BT + (size_t)min(4 * (i0 + it) + f, N - 1) * K + kofs;
#pragma unroll
        for (int s = 0; s < S; ++s) w[it][s] = ldw(p + s * 256);
    }
    const float sa = EPI != IE_EPI_I32 ? sA[m_c] : 0.0f;
    EpiIn e[IPW];
#pragma unroll
    for (int it = 0; it < IPW; ++it) e[it] = epi_load<EPI>(m_c, min(4 * (i0 + it) + f, N - 1), N, sB, bias, residual);
#pragma unroll
    for (int c = 0; c < SPT; ++c) {
        const int ch = threadIdx.x + 256 * c;
        if (CH % 256 == 0 || ch < CH) {
            const int r = ch / (K / 16);
            reinterpret_cast<i32x4*>(a_lds + r * LDA)[ch - r * (K / 16)] = stage[c];
        }
    }
    __syncthreads();

    const int8_t* arow[MB];
#pragma unroll
    for (int j = 0; j < MB; ++j) arow[j] = a_lds + min(4 * j + f, M - 1) * LDA + kofs;
#pragma unroll
    for (int it = 0; it < IPW; ++it) {
        if (i0 + it >= nitems_all) continue;  // uniform: past the last item
        i32x4 acc[MB][2];
#pragma unroll
        for (int j = 0; j < MB; ++j) acc[j][0] = acc[j][1] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int j = 0; j < MB; ++j)
                acc[j][s & 1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                    *reinterpret_cast<const i32x4*>(arow[j] + s * 256), w[it][s], acc[j][s & 1], 0, 0, 0);
        // diagonal entries (row part == column part), summed over the quad
        int32_t mine = 0;
#pragma unroll
        for (int j = 0; j < MB; ++j) {
            const i32x4 x4 = acc[j][0] + acc[j][1];
            int32_t x = part == 0 ? x4[0] : part == 1 ? x4[1] : part == 2 ? x4[2] : x4[3];
            x += __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xf, 0xf, false);  // quad_perm [1, 0, 3, 2]
            x += __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xf, 0xf, false);  // quad_perm [2, 3, 0, 1]
            mine = part == j ? x : mine;
        }
        const int n = 4 * (i0 + it) + f;
        if (out_ok && n < N) gemv_store<EPI>(C, out_m, n, N, mine, sa, e[it], 0, GemvFusion{});
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
// The 16-row MFMA GEMV splits its rows over several workgroups only for
// weights up to this size: each row block re-reads the weights, which for
// these stay in the caches.
constexpr size_t kRowSplitWeightBytes = 8ull << 20;

template <int MT, int EPI, int K16, int SRC = kSrcInt8, int GF = 0, int NW = 4>
void launch_fixed(const GemmArgs& a, hipStream_t s, const GemvFusion& f = GemvFusion{}) {
    constexpr int CPL = K16 / 16;
    constexpr int G = GF > 0 ? GF : CPL >= 12 ? 1 : (12 + CPL - 1) / CPL;
    const int rows_per_wg = NW * 4 * G;
    const bool nt = (size_t)a.N * K16 * 16 >= kStreamWeightBytes;
    // Streaming shapes: one workgroup per CU walking row groups (each wave
    // keeps a whole group's loads in flight); measured faster than one
    // workgroup per 16 rows, which re-stages the activations in every
    // workgroup and leaves a partial last wave of workgroups.
    const int cap = nt ? num_cus() : 2048;
    const unsigned blocks = (unsigned)min((a.N + rows_per_wg - 1) / rows_per_wg, cap);
    if (nt)
        gemv_i8_fixed_kernel<MT, EPI, K16, SRC, true, GF, NW><<<blocks, 64 * NW, 0, s>>>(
            a.M, a.N, a.A, a.BT, a.sA, a.sB, a.bias, a.residual, a.C, f);
    else
        gemv_i8_fixed_kernel<MT, EPI, K16, SRC, false, GF, NW><<<blocks, 64 * NW, 0, s>>>(
            a.M, a.N, a.A, a.BT, a.sA, a.sB, a.bias, a.residual, a.C, f);
}

template <int EPI, int K64, int SRC = kSrcInt8>
void launch_mfma16(const GemmArgs& a, hipStream_t s, const GemvFusion& f = GemvFusion{}) {
    const unsigned blocks = (unsigned)((a.N + 15) / 16);
    const bool nt = (size_t)a.N * K64 * 64 >= kStreamWeightBytes;
    // 8 waves at K = 3072 (the fused prologue stages the 16 rows in one round
    // trip instead of two, and each wave's K range is one batch of loads):
    // M = 16, N = 768 GEMV 0.048 -> 0.055 of HBM peak, GPT-2 batch-16 decode
    // 30088 -> 30684 tok/s; K = 768 (12 steps) keeps 4.
    constexpr int NWV = (K64 % 8 == 0 && K64 >= 32) ? 8 : 4;
    // Rows per workgroup: 4 when the weights stay cached (each row block
    // re-reads them): a workgroup then stages 4 activation rows, not 16, and
    // a CU keeps only so many bytes in flight (GPT-2 batch-16 decode step
    // 413.7 -> 368.7 us, same bits; 1, 2 and 8 rows measured slower).  QKV
    // epilogue rows carry cache slots and keep 16.
    auto go = [&](auto rsc, auto fwc) {
        constexpr int RS = decltype(rsc)::value, FW = decltype(fwc)::value;
        auto* k = nt ? gemv_i8_mfma16_kernel<EPI, K64, SRC, true, NWV, RS, FW>
                     : gemv_i8_mfma16_kernel<EPI, K64, SRC, false, NWV, RS, FW>;
        k<<<dim3((unsigned)((a.N + FW - 1) / FW), (unsigned)((a.M + RS - 1) / RS)), 64 * NWV, 0, s>>>(
            a.M, a.N, reinterpret_cast<const int8_t*>(a.A), reinterpret_cast<const int8_t*>(a.BT), a.sA, a.sB,
            a.bias, a.residual, a.C, f);
    };
    if constexpr (EPI != kEpiQKV)
        if ((size_t)a.N * K64 * 64 <= kRowSplitWeightBytes) {
            // 12 features per workgroup when 16 leave CUs idle and 12 fill
            // them (N = 768, 16 rows: 192 -> 256 workgroups)
            const long long rb = (a.M + 3) / 4, cus = num_cus();
            if ((long long)blocks * rb < cus && (long long)((a.N + 11) / 12) * rb <= cus)
                return go(std::integral_constant<int, 4>{}, std::integral_constant<int, 12>{});
            return go(std::integral_constant<int, 4>{}, std::integral_constant<int, 16>{});
        }
    go(std::integral_constant<int, 16>{}, std::integral_constant<int, 16>{});
}

template <int EPI>
void launch_slice(const GemmArgs& a, hipStream_t s) {
    const int groups = (a.N + 15) / 16;
    const int cus = num_cus();
    // K slices per group: the most that still give every wave at most one
    // group (groups x KS <= 8 waves x CUs), up to 4 (the kernel's ring needs
    // a multiple of R = 4 batches per wave).
    int ks_log = 0;
    while (ks_log < 2 && (long long)groups * (2 << ks_log) <= 8LL * cus) ++ks_log;
    const unsigned blocks = ks_log == 0 ? (unsigned)std::min(groups, cus) : (unsigned)((groups << ks_log) + 7) / 8;
    // Plain loads: a wave instruction here reads 16 rows x 64 bytes, half of
    // each 128-byte line, a pattern that streams slower with non-temporal
    // loads (M = 8 / 16 at N = 8192: 0.58 / 0.556 -> 0.589 / 0.566 of HBM
    // peak).  A ring of 2 sets of 8 loads: measured level with 4 sets.  Only
    // 9 <= M <= 16 come here (16 staged rows).
    auto* k = gemv_i8_slice_kernel<EPI, false, 2>;
    k<<<blocks, 512, 0, s>>>(a.M, a.N, ks_log, reinterpret_cast<const int8_t*>(a.A),
                             reinterpret_cast<const int8_t*>(a.BT), a.sA, a.sB, a.bias, a.residual, a.C);
}

template <int EPI>
void launch_parted(const GemmArgs& a, hipStream_t s) {
    const int items = (a.N + 3) / 4;
    const unsigned blocks = (unsigned)std::min(items, num_cus());
    const bool nt = (size_t)a.N * 8192 >= kStreamWeightBytes;
    auto go = [&](auto mb) {
        constexpr int MB = decltype(mb)::value;
        auto* k = nt ? gemv_i8_parted_kernel<EPI, true, MB> : gemv_i8_parted_kernel<EPI, false, MB>;
        k<<<blocks, 512, 0, s>>>(a.M, a.N, reinterpret_cast<const int8_t*>(a.A), reinterpret_cast<const int8_t*>(a.BT),
                                 a.sA, a.sB, a.bias, a.residual, a.C);
    };
    if (a.M <= 4) go(std::integral_constant<int, 1>{});
    else if (a.M <= 8) go(std::integral_constant<int, 2>{});
    else go(std::integral_constant<int, 4>{});
}

template <int EPI, int S>
void launch_burst(const GemmArgs& a, hipStream_t s) {
    constexpr int IPW = S <= 3 ? 8 : 2;  // 24 loads of weights per lane in flight
    const int items = (a.N + 3) / 4;
    const unsigned blocks = (unsigned)((items + 4 * IPW - 1) / (4 * IPW));
    // Non-temporal weight loads from 16 MiB up (the burst kernel takes N >=
    // 16384): the 768 x 50257 LM head 8.87 -> 8.31 us with its weights
    // rotated through 1 GiB, 3072 x 16390 10.8 -> 9.9 us, and the GPT-2 decode
    // step with the INT8 LM head 225.9 -> 223.2 us (batch 1) and 336.4 ->
    // 334.6 us (batch 16), where plain loads would leave the head in the MALL.
    const bool nt = (size_t)a.N * (256 * S) >= ((size_t)16 << 20);
    auto go = [&](auto mb) {
        constexpr int MB = decltype(mb)::value;
        auto* k = nt ? gemv_i8_burst_kernel<EPI, true, MB, S, IPW> : gemv_i8_burst_kernel<EPI, false, MB, S, IPW>;
        k<<<blocks, 256, 0, s>>>(a.M, a.N, reinterpret_cast<const int8_t*>(a.A), reinterpret_cast<const int8_t*>(a.BT),
                                 a.sA, a.sB, a.bias, a.residual, a.C);
    };
    if (a.M <= 4) go(std::integral_constant<int, 1>{});
    else if (a.M <= 8) go(std::integral_constant<int, 2>{});
    else go(std::integral_constant<int, 4>{});
}

// One decode row (M = 1): 16 rows per workgroup (one group of 4 rows per
// wave) and, at K = 3072 or N <= 1024, one-wave workgroups, so more CUs
// share the few hundred KB of weights and each wave's dot and epilogue chain
// is shorter (GPT-2 Small batch-1 decode step 272 -> 252 us; 64 rows per
// 4-wave workgroup before; one-wave workgroups for the 768 x 768 attention
// output projection: 247.5 -> 246.5 us).  M = 2 / 3-4: one group of 4 rows
// per wave as well, on the MT waves that stage the activation rows (8 / 16
// rows per workgroup; 64 before: batch 2 / 3 / 4 decode step 272 / 304 /
// 309 -> 253 / 279 / 282 us, same bits).
template <int EPI, int K, int SRC>
void launch_fused(const GemmArgs& a, const GemvFusion& f, hipStream_t s) {
    if (a.M <= 1 && (K == 3072 || a.N <= 1024)) launch_fixed<1, EPI, K / 16, SRC, 1, 1>(a, s, f);
    else if (a.M <= 1) launch_fixed<1, EPI, K / 16, SRC, 1, 4>(a, s, f);
    else if (a.M <= 2) launch_fixed<2, EPI, K / 16, SRC, 1, 2>(a, s, f);
    else if (a.M <= 4) launch_fixed<4, EPI, K / 16, SRC, 1, 4>(a, s, f);
    else launch_mfma16<EPI, K / 64, SRC>(a, s, f);
}

template <int MT, int EPI>
void launch_mt(const GemmArgs& a, hipStream_t s) {
    // Wide GPT-2-width GEMVs (the 768 x 50257 LM head): all of a wave's
    // loads at once (M = 1 / 4 / 8: 0.49 / 0.44 / 0.39 -> 0.52 / 0.51 / 0.49
    // of HBM peak per graph-replayed launch; slower on the narrow shapes,
    // whose time is launch latency).  At 9 <= M <= 16 it takes K = 3072
    // (N = 16390, weights rotated through 1 GiB: 18.3 -> 13.5 us at M = 16
    // against the MFMA GEMV); at K = 768 the MFMA GEMV stays, whose plain
    // loads keep an LM head in the MALL between decode steps (GPT-2 batch-16
    // step with the INT8 head 337.0 -> 334.6 us, although a standalone
    // launch on rotated weights is 2% slower).
    if (a.N >= 16384) {
        if (a.K == 768 && a.M <= 8) return launch_burst<EPI, 3>(a, s);
        if (a.K == 3072) return launch_burst<EPI, 12>(a, s);
    }
    if constexpr (MT > 4) {
        if (a.K == 768) return launch_mfma16<EPI, 12>(a, s);
        if (a.K == 3072) return launch_mfma16<EPI, 48>(a, s);
    }
    // K = 8192 (measured at N = 8192 and 28672, M = 1..16, fraction of HBM
    // peak on one box): the 4-feature-item kernel for M <= 8 (N = 28672:
    // M = 1 0.76 -> 0.79 against dot4, M = 4 0.62 -> 0.79 against the 16-row
    // MFMA kernels; N = 8192, rotated weights: M = 5 / 8 13.94 / 14.31 ->
    // 13.15 / 13.59 us against the K-sliced kernel) and for any M once each
    // wave has two items or more (N >= 16384; N = 28672, M = 16: 0.64 ->
    // 0.69); below that, at 9 <= M <= 16, the K-sliced 16-feature kernel,
    // whose activation staging costs a quarter as much per wave (N = 8192,
    // M = 16: 14.9 against 16.9 us).
    if (a.K == 8192) {
        if (a.M <= 8 || a.N >= 16384) return launch_parted<EPI>(a, s);
        return launch_slice<EPI>(a, s);
    }
    // Specialised K: the GPT-2 widths, with the decode step's grouping (one
    // 4-row group per wave; one-wave workgroups at N <= 1024 and at K = 3072
    // for M <= 2): M = 1 / 2 / 4 at 768 x 2304 3.83 / 3.92 / 4.17 -> 2.82 /
    // 2.87 / 2.97 us, 3072 x 768 3.48 / 3.80 -> 3.01 / 3.63 us (M = 4 keeps
    // four waves, level at 4.42 us), same bits; the step built from the C ABI
    // 466 -> 451 us at batch 1, 546 -> 497 us at batch 4.
    if constexpr (MT <= 4) {
        if (a.K == 768 && a.N <= 1024) return launch_fixed<MT, EPI, 48, kSrcInt8, 1, 1>(a, s);
        if (a.K == 768) return launch_fixed<MT, EPI, 48, kSrcInt8, 1, 4>(a, s);
        if (a.K == 3072 && MT <= 2) return launch_fixed<MT, EPI, 192, kSrcInt8, 1, 1>(a, s);
        if (a.K == 3072) return launch_fixed<MT, EPI, 192, kSrcInt8, 1, 4>(a, s);
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
