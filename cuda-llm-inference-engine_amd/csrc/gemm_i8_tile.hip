// gemm_i8_tile.hip — INT8 GEMM for prefill-sized problems on gfx950 (M of a
// few hundred to a few thousand rows, GPT-2-sized N and K, more 32 x 32
// blocks than two per CU).
//
// Result identical to the reference's K14 kernel (kernels/quantization/
// 14_int8_gemm.cu:65-170): exact int32 K-sum, then the dequant epilogue.
//
// At these sizes a workgroup owns only 6-24 K-stages, so what bounds it is
// the memory latency each stage waits for, not the matrix cores; several
// small workgroups per CU cover it better than one large one.  The tile is
// BM x BN (64 x 64 or 128 x 64) on four waves (2 x 2, each (BM/2) x (BN/2)
// as 32x32 blocks of v_mfma_i32_32x32x32_i8), and K advances through a ring
// of NSTAGE 128-byte stages in LDS (2-3; 4 for long K or a one-round grid),
// NSTAGE - 1 of them in flight while one is read:
//   * global -> LDS copies are global_load_lds_dwordx4 (16 B per lane straight
//     into LDS); a wave-load fills 8 rows x 128 B; the lane -> global address
//     map applies the LDS swizzle, so the lane-ordered destination lands each
//     16-byte chunk c of row r at slot c ^ ((r >> 1) & 7), which spreads the
//     rows one MFMA operand read touches over all banks;
//   * a stage is read as four k-substeps of 32 bytes (one MFMA K each);
//   * workgroup ids are remapped so each XCD (ids = xcd mod 8) receives a
//     contiguous run of tiles, walked in groups of GROUP_M tile rows, so the
//     workgroups resident on one XCD share A and B panels in its L2.
// Requirements (checked by the launcher): K % 128 == 0, 16-byte aligned A/BT.
// Rows past M or N read the last valid row (no fault, results discarded).

#include "device_util.h"
#include "epilogue.h"
#include "ie_internal.h"

namespace ie {
namespace {

constexpr int BK = 128;
constexpr int CHUNKS = BK / 16;  // 16-byte chunks per LDS row
constexpr int GROUP_M = 4;

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gbl_ptr_t;

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

// Rows [r0, r0 + 8) x BK bytes of a K-contiguous operand into LDS with one
// wave-wide 16-byte-per-lane direct load.
__device__ __forceinline__ void load_rows(const int8_t* __restrict__ src, int ld, int rows_valid, int row0, int k0,
                                          int r0, int8_t* lds_oper) {
    const int lane = threadIdx.x & 63;
    const int r = r0 + lane / CHUNKS;
    const int c = (lane % CHUNKS) ^ swz(r);
    const int gr = min(row0 + r, rows_valid - 1);
    const int8_t* g = src + (size_t)gr * ld + k0 + c * 16;
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)g, (lds_ptr_t)(lds_oper + r0 * BK), 16, 0, 0);
}

__device__ __forceinline__ i32x4 read_frag(const int8_t* lds_oper, int row, int chunk) {
    return *reinterpret_cast<const i32x4*>(lds_oper + row * BK + ((chunk ^ swz(row)) << 4));
}

template <int EPI, int BM, int BN, int NSTAGE, bool NT>
__global__ __launch_bounds__(256) void gemm_i8_tile_kernel(int M, int N, int K, const int8_t* __restrict__ A,
                                                           const int8_t* __restrict__ BT,
                                                           const float* __restrict__ sA,
                                                           const float* __restrict__ sB, const float* bias,
                                                           const float* residual, void* C, int tiles_m,
                                                           int tiles_n, const QkvRoute route) {
    constexpr int OA = BM * BK, STAGE = (BM + BN) * BK;
    constexpr int MI = BM / 64, NJ = BN / 64;  // 32x32 blocks per wave
    constexpr int LA = BM / 32, LB = BN / 32;  // wave-loads per operand per stage (8 rows each, 4 waves)
    constexpr int LPS = LA + LB;
    static_assert(MI >= 1 && NJ >= 1 && (NSTAGE - 1) * LPS <= 63, "tile and ring fit");
    // (kEpiQKVRoute: BM row slots after the ring, in the same array: a
    // second LDS object would make the compiler drain the copies in flight
    // before every LDS read of the K loop)
    constexpr bool ROUTE = EPI == kEpiQKVRoute;
    __shared__ __attribute__((aligned(1024))) int8_t lds[NSTAGE * STAGE + (ROUTE ? BM * 4 : 0)];

    // XCD-aware, grouped tile order.
    const int nwg = gridDim.x;
    int id = blockIdx.x;
    if ((nwg & 7) == 0) id = (id & 7) * (nwg >> 3) + (id >> 3);
    const int per_group = GROUP_M * tiles_n;
    const int group = id / per_group;
    const int first_m = group * GROUP_M;
    const int gm = min(tiles_m - first_m, GROUP_M);
    const int in_group = id - group * per_group;
    const int m0 = (first_m + in_group % gm) * BM, n0 = (in_group / gm) * BN;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    i32x16 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

    const int nk = K / BK;
    // Copies stage kt_src into LDS slot `slot`.  Every iteration issues one
    // stage, so the loop body is branch-free: past the last stage the copy
    // re-reads stage nk-1 into the slot just freed, which is never read again.
    auto issue = [&](int kt_src, int slot) {
        int8_t* sa = lds + slot * STAGE;
        int8_t* sb = sa + OA;
        const int k0 = kt_src * BK;
#pragma unroll
        for (int j = 0; j < LA; ++j) load_rows(A, K, M, m0, k0, (wave * LA + j) * 8, sa);
#pragma unroll
        for (int j = 0; j < LB; ++j) load_rows(BT, K, N, n0, k0, (wave * LB + j) * 8, sb);
    };

    // Prologue: stages 0 .. NSTAGE-2 in flight, stage 0 landed.
#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p) issue(min(p, nk - 1), p);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTAGE - 2) * LPS) : "memory");
    __builtin_amdgcn_s_barrier();

    const int frow = lane & 31;
    const int fchunk = lane >> 5;
    // Operand fragments in two register slots (k-substeps alternate).
    i32x4 af[2][MI], bf[2][NJ];
    auto frags = [&](const int8_t* sa, const int8_t* sb, int ks, int slot) {
#pragma unroll
        for (int i = 0; i < MI; ++i) af[slot][i] = read_frag(sa, wm * (BM / 2) + i * 32 + frow, ks * 2 + fchunk);
#pragma unroll
        for (int j = 0; j < NJ; ++j) bf[slot][j] = read_frag(sb, wn * (BN / 2) + j * 32 + frow, ks * 2 + fchunk);
    };
    auto mfmas = [&](int slot) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[slot][i], bf[slot][j], acc[i][j], 0, 0, 0);
    };
    frags(lds, lds + OA, 0, 0);

    constexpr int SUB = BK / 32;  // MFMA k-substeps per stage
    for (int kt = 0; kt < nk; ++kt) {
        const int8_t* sa = lds + (kt % NSTAGE) * STAGE;
        const int8_t* sb = sa + OA;
#pragma unroll
        for (int ks = 0; ks < SUB; ++ks) {
            const int slot = ks & 1;
            __builtin_amdgcn_sched_barrier(0);
            if (ks + 1 < SUB) {
                // the copies of stage kt + NSTAGE - 1 go into the slot freed
                // by iteration kt - 1 (every wave passed its last barrier)
                if (ks == 0) issue(min(kt + NSTAGE - 1, nk - 1), (kt + NSTAGE - 1) % NSTAGE);
                frags(sa, sb, ks + 1, slot ^ 1);
                mfmas(slot);
            } else {
                // last substep: its MFMAs, then stage kt + 1 must have landed
                // (this wave's copies: vmcnt; everyone's: the barrier; a bare
                // s_barrier, since __syncthreads()' fence drains vmcnt to 0),
                // then the next stage's first fragments
                mfmas(slot);
                __builtin_amdgcn_sched_barrier(0);
                asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((NSTAGE - 2) * LPS) : "memory");
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                const int8_t* na = lds + ((kt + 1) % NSTAGE) * STAGE;
                frags(na, na + OA, 0, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");

    // Epilogue.  Lane l of a 32x32 block holds rows 8q + 4(l/32) + r (q, r < 4)
    // of column l % 32.  Every operand the stores need (scales, bias,
    // residual; clamped indices) is gathered first and consumed once in
    // straight-line code: loaded inside the branchy store loop, each would
    // wait for all earlier stores (vmcnt counts stores, and C may alias them).
    const int h = lane >> 5;
    const int rbase = m0 + wm * (BM / 2) + 4 * h;
    const int cbase = n0 + wn * (BN / 2) + (lane & 31);
    constexpr bool HAS_BIAS =
        EPI == IE_EPI_BIAS || EPI == IE_EPI_BIAS_GELU || EPI == IE_EPI_BIAS_RESIDUAL || ROUTE;
    constexpr bool HAS_RES = EPI == IE_EPI_BIAS_RESIDUAL;
    auto row = [&](int i, int v) { return rbase + i * 32 + 8 * (v >> 2) + (v & 3); };
    float sa[MI][16] = {}, sb[NJ] = {}, bv[NJ] = {}, rv[MI][16][NJ] = {};
    // kEpiQKVRoute: the tile's row slots go to LDS (32 of them per lane in
    // registers cost a wave per SIMD), read back beside each store
    int* lslot = reinterpret_cast<int*>(lds + NSTAGE * STAGE);
    if constexpr (ROUTE) {
        if (threadIdx.x < BM) lslot[threadIdx.x] = route.row_slot[min(m0 + (int)threadIdx.x, M - 1)];
        __syncthreads();
    }
    if constexpr (EPI != IE_EPI_I32) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int n = min(cbase + j * 32, N - 1);
            sb[j] = sB[n];
            if constexpr (HAS_BIAS) bv[j] = bias[n];
        }
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = min(row(i, v), M - 1);
                sa[i][v] = sA[m];
                if constexpr (HAS_RES) {
#pragma unroll
                    for (int j = 0; j < NJ; ++j) rv[i][v][j] = residual[(size_t)m * N + min(cbase + j * 32, N - 1)];
                }
            }
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                asm volatile("" ::"v"(sa[i][v]));
                if constexpr (HAS_RES) {
#pragma unroll
                    for (int j = 0; j < NJ; ++j) asm volatile("" ::"v"(rv[i][v][j]));
                }
            }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            asm volatile("" ::"v"(sb[j]));
            if constexpr (HAS_BIAS) asm volatile("" ::"v"(bv[j]));
        }
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int m = row(i, v);
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int n = cbase + j * 32;
                if (n >= N) continue;
                if constexpr (ROUTE)
                    route_store(route, m, n, lslot[m - m0], acc[i][j][v], sa[i][v], sb[j], bv[j]);
                else
                    store_epilogue_v<EPI, NT>(C, (size_t)m * N + n, acc[i][j][v], sa[i][v], sb[j], bv[j], rv[i][v][j]);
            }
        }
    }
}

template <int EPI>
struct TileLaunch {
    template <int BM, int BN, int NSTAGE>
    static void go(const GemmArgs& a, hipStream_t s) {
        const int tm = (a.M + BM - 1) / BM, tn = (a.N + BN - 1) / BN;
        // C of 16 MiB or more goes out with non-temporal stores (M = 2048:
        // N = 2304 12.5 -> 10.9 us, N = 3072 13.5 -> 11.0 us; at N = 768,
        // 6.3 MB of C, they measured slower: 6.15 -> 6.7 us)
        // (routed stores are plain: Q and the caches are read next)
        auto* k = gemm_i8_tile_kernel<EPI, BM, BN, NSTAGE, false>;
        if constexpr (EPI != kEpiQKVRoute)
            if ((size_t)a.M * a.N * 4 >= ((size_t)16 << 20)) k = gemm_i8_tile_kernel<EPI, BM, BN, NSTAGE, true>;
        k<<<tm * tn, 256, 0, s>>>(a.M, a.N, a.K, reinterpret_cast<const int8_t*>(a.A),
                                 reinterpret_cast<const int8_t*>(a.BT), a.sA, a.sB, a.bias, a.residual, a.C, tm, tn,
                                 a.route);
    }
    // Measured on the GPT-2 prefill shapes (M = 128-2048, K = 768 / 3072,
    // N = 768-3072, bias epilogue; same box, bit-identical C): 128 x 64 tiles
    // beat 64 x 64 once there are two per CU (M = 2048, N = 2304: 12.1
    // against 13.7 us) and keep two stages (three: 11.1 -> 13.7 us, fewer
    // workgroups per CU); 64 x 64 tiles take three stages at K = 768, two in
    // flight, which pays when the weights come from the MALL or HBM rather
    // than L2 (GPT-2 prefill TTFT at batch 1: 0.705 -> 0.684 ms; weights
    // rotated through 1 GiB, M = 512, N = 768: 7.55 -> 5.95 us; the same
    // weights every launch, L2-resident: 5.09 -> 5.20 us), and four over long
    // K (K = 3072) or when the grid is one round of workgroups, one per CU
    // (rotated weights, K = 768: M = 512, N = 768 5.88 -> 5.37 us; M = 128,
    // N = 2304 6.01 -> 5.41 us, N = 3072 6.05 -> 5.49 us; with 288-384 tiles
    // four stages measured 3% slower); six or eight stages measured slower
    // still, in one round too (K = 3072: 10.4 -> 10.9-11.1 us); 128 x 128
    // tiles lost everywhere.
    static void run(const GemmArgs& a, hipStream_t s) {
        const bool long_k = a.K >= 2048;
        if (gemm_i8_tile_shape(a) == 128064) {
            if (long_k) go<128, 64, 4>(a, s);
            else go<128, 64, 2>(a, s);
        } else {
            const long long tiles = (long long)((a.M + 63) / 64) * ((a.N + 63) / 64);
            if (long_k || tiles <= num_cus()) go<64, 64, 4>(a, s);
            else go<64, 64, 3>(a, s);
        }
    }
};

}  // namespace

// Tile shape BM * 1000 + BN for a problem: 128 x 64 once that gives two
// tiles per CU, else 64 x 64.
int gemm_i8_tile_shape(const GemmArgs& a) {
    const long long t = (long long)((a.M + 127) / 128) * ((a.N + 63) / 64);
    return t >= 2LL * num_cus() ? 128064 : 64064;
}

// Grids small enough for one round of 32 x 32 blocks take the K-split
// stream kernel first (gemm_i8_stream_applies).
bool gemm_i8_tile_applies(const GemmArgs& a) {
    if (a.K % BK != 0 || a.K == 0) return false;
    if (((uintptr_t)a.A % 16) || ((uintptr_t)a.BT % 16)) return false;
    const long long t = (long long)((a.M + 63) / 64) * ((a.N + 63) / 64);
    return t < (1LL << 31);
}

void launch_gemm_i8_tile(const GemmArgs& a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    if (a.epi == kEpiQKVRoute)
        TileLaunch<kEpiQKVRoute>::run(a, s);
    else
        dispatch_epilogue<TileLaunch>(a.epi, a, s);
}

}  // namespace ie
