// gemm_i8_stream.hip — INT8 GEMM for mid-size problems (prefill-sized M, a
// few hundred to a few thousand rows, GPT-2-sized N and K) on gfx950.
//
// Same result as the reference's K14 kernel (kernels/quantization/
// 14_int8_gemm.cu:65-170): exact int32 K-sum, then the dequant epilogue.
//
// At these sizes a 256x256 (or 128x128) LDS-tiled workgroup leaves most of the
// 256 CUs idle and spends its time in the per-step barrier, so here every wave
// is independent: it owns a 32 x (32 * NB) block of C, held as NB
// v_mfma_i32_32x32x32_i8 accumulators, and streams its A and B fragments
// straight from global memory into registers one K-group ahead, with no LDS
// and no barrier.  A K-group is 128 bytes of K = four MFMA K-steps:
//   * lane l owns row l % 32 of the A block (and of each B block) and half
//     h = l / 32 of the group's 128 bytes: one 64-byte contiguous run, read
//     as four 16-byte loads, so the two lanes of a row cover its 128-byte
//     line;
//   * MFMA step s of the group takes chunk s of each lane's run: K-bytes
//     128u + 16s (h = 0) and 128u + 64 + 16s (h = 1).  A and B use the same
//     lane -> K map, so the four steps sum exactly the group's 128 bytes, in
//     whatever order; the int32 result is the K-sum bit for bit.
// Accumulator v of lane l is C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32] of its
// 32x32 block.  Rows past M or N read the last valid row (results discarded).
// When there are few blocks and a long K loop, 2 or 4 waves share a block,
// each walking a contiguous range of its K-groups, and add their int32 tiles
// in LDS (exact, so the result is the same bits).
// Requirements (checked by the launcher): K % 128 == 0, 16-byte aligned A, BT.
#include "device_util.h"
#include "epilogue.h"
#include "ie_internal.h"

namespace ie {
namespace {

constexpr int KG = 128;  // K bytes per group

template <int NB>
struct Group {
    i32x4 a[4];
    i32x4 b[NB][4];
};

template <int NB>
__device__ __forceinline__ void load_group(Group<NB>& g, const int8_t* arow,
                                           const int8_t* const (&brow)[NB], int k0) {
#pragma unroll
    for (int s = 0; s < 4; ++s) g.a[s] = *reinterpret_cast<const i32x4*>(arow + k0 + 16 * s);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int s = 0; s < 4; ++s) g.b[j][s] = *reinterpret_cast<const i32x4*>(brow[j] + k0 + 16 * s);
}

template <int NB>
__device__ __forceinline__ void mfma_group(const Group<NB>& g, i32x16 (&acc)[NB]) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int j = 0; j < NB; ++j)
            acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(g.a[s], g.b[j][s], acc[j], 0, 0, 0);
}

// KS waves per workgroup share one C block and split its K-groups into KS
// contiguous ranges (KS = 1: the whole K loop on one wave); their int32
// tiles are added in LDS, which is exact, so the result does not depend on
// KS.  blockIdx.x walks N blocks fastest so consecutive workgroups share
// their A rows in L2.
template <int EPI, int NB, int KS>
__global__ __launch_bounds__(64 * KS) void gemm_i8_stream_kernel(
    int M, int N, int K, const int8_t* __restrict__ A, const int8_t* __restrict__ BT,
    const float* __restrict__ sA, const float* __restrict__ sB, const float* bias,
    const float* residual, void* C) {
    const int lane = threadIdx.x & 63;
    const int wave = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 31, h = lane >> 5;
    const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32 * NB;
    const int8_t* arow = A + (size_t)min(m0 + r, M - 1) * K + 64 * h;
    const int8_t* brow[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) brow[j] = BT + (size_t)min(n0 + 32 * j + r, N - 1) * K + 64 * h;

    i32x16 acc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][v] = 0;

    const int ngt = K / KG;
    const int g0 = (int)((long long)ngt * wave / KS), g1 = (int)((long long)ngt * (wave + 1) / KS);
    // Ping-pong over groups: group u+1 (clamped to the last group of the
    // range, a cache hit) is always in flight while group u runs.  (A
    // four-deep ring measured slower: a wave load touches 32 rows' cache
    // lines, so the address path, not latency, is what more requests in
    // flight run into.)
    if (g1 > g0) {
        Group<NB> ga, gb;
        load_group(ga, arow, brow, g0 * KG);
        int u = g0;
        while (true) {
            load_group(gb, arow, brow, min(u + 1, g1 - 1) * KG);
            mfma_group(ga, acc);
            if (++u >= g1) break;
            load_group(ga, arow, brow, min(u + 1, g1 - 1) * KG);
            mfma_group(gb, acc);
            if (++u >= g1) break;
        }
    }
    if constexpr (KS > 1) {
        // waves 1..KS-1 hand their tiles to wave 0 through LDS
        __shared__ i32x16 red[KS - 1][NB][64];
        if (wave > 0) {
#pragma unroll
            for (int j = 0; j < NB; ++j) red[wave - 1][j][lane] = acc[j];
        }
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int w = 0; w < KS - 1; ++w)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[j] += red[w][j][lane];
    }

    // Every operand the stores need (scales, bias, residual; clamped
    // indices) is gathered first and consumed once in straight-line code:
    // loaded inside the branchy store loop, each would wait for all earlier
    // stores (vmcnt counts stores, and C may alias them).
    const int cbase = n0 + r;
    const int rbase = m0 + 4 * h;
    constexpr bool HAS_BIAS = EPI == IE_EPI_BIAS || EPI == IE_EPI_BIAS_GELU || EPI == IE_EPI_BIAS_RESIDUAL;
    constexpr bool HAS_RES = EPI == IE_EPI_BIAS_RESIDUAL;
    float sa[16] = {}, sb[NB] = {}, bv[NB] = {}, rv[16][NB] = {};
    if constexpr (EPI != IE_EPI_I32) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int n = min(cbase + 32 * j, N - 1);
            sb[j] = sB[n];
            if constexpr (HAS_BIAS) bv[j] = bias[n];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = min(rbase + 8 * (v >> 2) + (v & 3), M - 1);
            sa[v] = sA[m];
            if constexpr (HAS_RES) {
#pragma unroll
                for (int j = 0; j < NB; ++j) rv[v][j] = residual[(size_t)m * N + min(cbase + 32 * j, N - 1)];
            }
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            asm volatile("" ::"v"(sa[v]));
#pragma unroll
            for (int j = 0; j < NB; ++j)
                if constexpr (HAS_RES) asm volatile("" ::"v"(rv[v][j]));
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            asm volatile("" ::"v"(sb[j]));
            if constexpr (HAS_BIAS) asm volatile("" ::"v"(bv[j]));
        }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int n = cbase + 32 * j;
        if (n >= N) continue;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = rbase + 8 * (v >> 2) + (v & 3);
            if (m < M) store_epilogue_v<EPI>(C, (size_t)m * N + n, acc[j][v], sa[v], sb[j], bv[j], rv[v][j]);
        }
    }
}

template <int EPI>
struct StreamLaunch {
    template <int NB, int KS>
    static void go(const GemmArgs& a, hipStream_t s) {
        const dim3 grid((a.N + 32 * NB - 1) / (32 * NB), (a.M + 31) / 32);
        gemm_i8_stream_kernel<EPI, NB, KS><<<grid, 64 * KS, 0, s>>>(
            a.M, a.N, a.K, reinterpret_cast<const int8_t*>(a.A), reinterpret_cast<const int8_t*>(a.BT),
            a.sA, a.sB, a.bias, a.residual, a.C);
    }
    static void run(const GemmArgs& a, hipStream_t s) {
        // Two 32-column blocks per wave once there are enough of them to fill
        // the GPU several times over; one otherwise.  With fewer than 1024
        // blocks, the K-groups are split over 4 waves per block from 16
        // groups up and over 2 from 4 (M=128: 12.9 -> 9.7 us at K=3072,
        // N=768; 6.2 -> 5.6 us at K=768; no change at M >= 512).
        const long long blocks1 = (long long)((a.M + 31) / 32) * ((a.N + 31) / 32);
        const long long waves2 = (long long)((a.M + 31) / 32) * ((a.N + 63) / 64);
        const int ng = a.K / KG;
        if (waves2 >= 1024) {
            go<2, 1>(a, s);
        } else if (blocks1 < 1024 && ng >= 16) {
            go<1, 4>(a, s);
        } else if (blocks1 < 1024 && ng >= 4) {
            go<1, 2>(a, s);
        } else {
            go<1, 1>(a, s);
        }
    }
};

}  // namespace

bool gemm_i8_stream_applies(const GemmArgs& a) {
    if (a.K % KG != 0 || a.K == 0) return false;
    if (((uintptr_t)a.A % 16) || ((uintptr_t)a.BT % 16)) return false;
    return (a.M + 31) / 32 <= 65535;
}

void launch_gemm_i8_stream(const GemmArgs& a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    dispatch_epilogue<StreamLaunch>(a.epi, a, s);
}

}  // namespace ie
