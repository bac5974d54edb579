// gemm_i8_stream.hip — INT8 GEMM for small grids (at most two 32 x 32 blocks
// of C per CU: prefill-sized M of a few dozen to a few hundred rows against
// GPT-2-sized outputs) on gfx950.
//
// Same result as the reference's K14 kernel (kernels/quantization/
// 14_int8_gemm.cu:65-170): exact int32 K-sum, then the dequant epilogue.
//
// With so few 64 x 64 tiles a workgroup per tile leaves most CUs idle, and
// each busy CU streams long A and B panels; what bounds the launch is how
// fast one CU takes in its bytes.  So here a workgroup owns a single 32 x 32
// block of C (v_mfma_i32_32x32x32_i8, 16 int32 accumulators per lane) and
// its KS waves split the block's 128-byte K-groups into contiguous ranges:
//   * each wave streams its range through its own ring of LR LDS slots (a
//     slot: 32 A rows + 32 B rows x 128 bytes = 8 KiB), LR - 1 groups ahead,
//     with global_load_lds_dwordx4 (16 bytes per lane straight into LDS): a
//     wave-load covers 8 rows x 128 contiguous bytes, 8 cache lines per KiB.
//     Loading the MFMA operand layout directly into registers (32 rows x 32
//     bytes per wave instruction, 32 lines per KiB) took in about half the
//     bytes per CU: M = 128, K = 3072, N = 768 10.5 -> 6.9 us, K = 768 5.7 ->
//     4.6 us, M = 32 / 64 / 256 at K = 3072 11.5 / 11.0 / 10.1 -> 7.2 / 7.0 /
//     6.6 us (weights rotated through 1 GiB, same bits);
//   * LDS rows are 128 bytes with chunk c of row r at slot c ^ ((r >> 1) & 7),
//     which spreads the 32 rows an operand read touches over all banks;
//   * a wave reads only slots it filled, so a wait on its own vmcnt is the
//     whole synchronisation of the K loop (no barrier).  The ring is the
//     kernel's only LDS object: with a second one (the partial tiles of the
//     K split) the compiler can no longer tell the LDS reads from the copies
//     in flight and drains every copy before each read, so the partial tiles
//     reuse the ring once it is empty;
//   * KS = 2 (K split over two waves, their int32 tiles added in LDS, exact)
//     measured best at K = 640-3072; one, three or four waves were slower
//     (M = 128, K = 3072: 8.8 / 6.9 / 6.9 / 7.3 us for KS = 1 / 2 / 3 / 4).
// Requirements (checked by gemm_i8_stream_applies): K % 128 == 0, 16-byte
// aligned A and BT.  Rows past M or N read the last valid row (results
// discarded).
#include "device_util.h"
#include "epilogue.h"
#include "ie_internal.h"

namespace ie {
namespace {

constexpr int KG = 128;              // K bytes per group
constexpr int LR = 4;                // ring slots per wave, LR - 1 groups in flight
constexpr int LSLOT = 2 * 32 * KG;   // one K-group of the block's A and B rows: 8 KiB
constexpr int COPIES = 8;            // wave-loads per K-group (4 for A, 4 for B)

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gbl_ptr_t;

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

// Rows [r0, r0 + 8) x 128 bytes at K offset k0 of a K-contiguous operand
// into LDS with one wave-wide 16-byte-per-lane direct load: lane l fetches
// chunk (l % 8) ^ swz(r) of row r = r0 + l / 8 into slot l % 8, so chunk c of
// row r lands at slot c ^ swz(r).
__device__ __forceinline__ void copy_rows(const int8_t* __restrict__ src, int ld, int rows_valid, int row0, int k0,
                                          int r0, int8_t* dst) {
    const int lane = threadIdx.x & 63;
    const int r = r0 + (lane >> 3);
    const int c = (lane & 7) ^ swz(r);
    const int gr = min(row0 + r, rows_valid - 1);
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)(src + (size_t)gr * ld + k0 + c * 16),
                                     (lds_ptr_t)(dst + r0 * KG), 16, 0, 0);
}

__device__ __forceinline__ i32x4 read_frag(const int8_t* oper, int row, int chunk) {
    return *reinterpret_cast<const i32x4*>(oper + row * KG + ((chunk ^ swz(row)) << 4));
}

template <int EPI, int KS>
__global__ __launch_bounds__(64 * KS) void gemm_i8_stream_kernel(
    int M, int N, int K, const int8_t* __restrict__ A, const int8_t* __restrict__ BT,
    const float* __restrict__ sA, const float* __restrict__ sB, const float* bias,
    const float* residual, void* C, const QkvRoute route) {
    static_assert((KS - 1) * 64 * (int)sizeof(i32x16) <= KS * LR * LSLOT, "partial tiles fit the rings");
    __shared__ __attribute__((aligned(1024))) int8_t lds[KS * LR * LSLOT];
    const int lane = threadIdx.x & 63;
    const int wave = KS == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
    int8_t* ring = lds + wave * (LR * LSLOT);
    const int ngt = K / KG;
    const int g0 = (int)((long long)ngt * wave / KS), g1 = (int)((long long)ngt * (wave + 1) / KS);
    const int nk = g1 - g0;

    i32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0;
    // Copies group g of the block's A and B rows into ring slot `slot`.
    auto issue = [&](int g, int slot) {
        int8_t* dst = ring + slot * LSLOT;
        const int k0 = g * KG;
#pragma unroll
        for (int j = 0; j < 4; ++j) copy_rows(A, K, M, m0, k0, 8 * j, dst);
#pragma unroll
        for (int j = 0; j < 4; ++j) copy_rows(BT, K, N, n0, k0, 8 * j, dst + 32 * KG);
    };
    if (nk > 0) {
        // Groups past the range re-read its last group (into slots that are
        // never read), so every step issues exactly COPIES loads and each wait
        // below leaves the LR - 2 younger groups in flight.
#pragma unroll
        for (int p = 0; p < LR - 1; ++p) issue(g0 + min(p, nk - 1), p);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((LR - 2) * COPIES) : "memory");
        const int fr = lane & 31, h = lane >> 5;
        for (int u = 0; u < nk; ++u) {
            // slot (u - 1) % LR: its reads fed the previous step's MFMAs
            issue(g0 + min(u + LR - 1, nk - 1), (u + LR - 1) % LR);
            const int8_t* src = ring + (u % LR) * LSLOT;
            // MFMA step q takes chunk 2q + h of each lane's row, for A and B alike
            i32x4 af[4], bf[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                af[q] = read_frag(src, fr, 2 * q + h);
                bf[q] = read_frag(src + 32 * KG, fr, 2 * q + h);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[q], bf[q], acc, 0, 0, 0);
            // group u + 1 has landed
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((LR - 2) * COPIES) : "memory");
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    if constexpr (KS > 1) {
        // the rings are drained: once every wave is past its K loop their
        // memory takes waves 1..KS-1's tiles, which wave 0 adds
        i32x16* red = reinterpret_cast<i32x16*>(lds);
        __syncthreads();
        if (wave > 0) red[(wave - 1) * 64 + lane] = acc;
        __syncthreads();
        if (wave > 0) return;
#pragma unroll
        for (int w = 0; w < KS - 1; ++w) acc += red[w * 64 + lane];
    }

    // Accumulator v of lane l is C[rbase + 8 (v / 4) + v % 4][n0 + l % 32].
    // Every operand the stores need (scales, bias, residual; clamped
    // indices) is gathered first and consumed once in straight-line code:
    // loaded inside the branchy store loop, each would wait for all earlier
    // stores (vmcnt counts stores, and C may alias them).
    const int cbase = n0 + (lane & 31);
    const int rbase = m0 + 4 * (lane >> 5);
    constexpr bool ROUTE = EPI == kEpiQKVRoute;
    constexpr bool HAS_BIAS =
        EPI == IE_EPI_BIAS || EPI == IE_EPI_BIAS_GELU || EPI == IE_EPI_BIAS_RESIDUAL || ROUTE;
    constexpr bool HAS_RES = EPI == IE_EPI_BIAS_RESIDUAL;
    float sa[16] = {}, sb = 0.0f, bv = 0.0f, rv[16] = {};
    int slot[ROUTE ? 16 : 1] = {};
    if constexpr (EPI != IE_EPI_I32) {
        const int n = min(cbase, N - 1);
        sb = sB[n];
        if constexpr (HAS_BIAS) bv = bias[n];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = min(rbase + 8 * (v >> 2) + (v & 3), M - 1);
            sa[v] = sA[m];
            if constexpr (HAS_RES) rv[v] = residual[(size_t)m * N + n];
            if constexpr (ROUTE) slot[v] = route.row_slot[m];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            asm volatile("" ::"v"(sa[v]));
            if constexpr (HAS_RES) asm volatile("" ::"v"(rv[v]));
        }
        asm volatile("" ::"v"(sb));
        if constexpr (HAS_BIAS) asm volatile("" ::"v"(bv));
    }
    if (cbase < N) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = rbase + 8 * (v >> 2) + (v & 3);
            if (m >= M) continue;
            if constexpr (ROUTE)
                route_store(route, m, cbase, slot[v], acc[v], sa[v], sb, bv);
            else
                store_epilogue_v<EPI>(C, (size_t)m * N + cbase, acc[v], sa[v], sb, bv, rv[v]);
        }
    }
}

template <int EPI>
struct StreamLaunch {
    template <int KS>
    static void go(const GemmArgs& a, hipStream_t s) {
        const dim3 grid((a.N + 31) / 32, (a.M + 31) / 32);
        gemm_i8_stream_kernel<EPI, KS><<<grid, 64 * KS, 0, s>>>(
            a.M, a.N, a.K, reinterpret_cast<const int8_t*>(a.A), reinterpret_cast<const int8_t*>(a.BT),
            a.sA, a.sB, a.bias, a.residual, a.C, a.route);
    }
    static void run(const GemmArgs& a, hipStream_t s) {
        if (a.K / KG >= 2)
            go<2>(a, s);
        else
            go<1>(a, s);
    }
};

}  // namespace

// While its 32 x 32 blocks fit one round of workgroups (two per CU: 64 KiB
// of LDS each).  Against the 64 x 64 LDS tile kernel (weights rotated
// through 1 GiB, same bits): ahead up to 512 blocks (M = 128, N = 2304, K =
// 768: 4.75 against 5.41 us; M = 512, N = 768, K = 3072: 7.2 against 10.4;
// 512 blocks: 5.26-8.8 against 5.47-10.5), behind from the second round on
// (576 blocks, M = 256, N = 2304: 7.97 against 5.63 us).
bool gemm_i8_stream_applies(const GemmArgs& a) {
    if (a.K % KG != 0 || a.K == 0) return false;
    if (((uintptr_t)a.A % 16) || ((uintptr_t)a.BT % 16)) return false;
    const long long blocks = (long long)((a.M + 31) / 32) * ((a.N + 31) / 32);
    return (a.M + 31) / 32 <= 65535 && blocks <= 2LL * num_cus();
}

void launch_gemm_i8_stream(const GemmArgs& a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    if (a.epi == kEpiQKVRoute)
        StreamLaunch<kEpiQKVRoute>::run(a, s);
    else
        dispatch_epilogue<StreamLaunch>(a.epi, a, s);
}

}  // namespace ie
