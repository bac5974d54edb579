// gemm_i8_mfma256.hip — large-tile INT8 GEMM for gfx950 (M, N >= a few
// thousand; the 8192^3 configuration).
//
// Result identical to the reference's K14 kernel (kernels/quantization/
// 14_int8_gemm.cu:65-170): exact int32 K-sum, then the dequant epilogue.
//
// MI355X mapping:
//   * 256x256 C tile per 512-thread workgroup; each of the 2 x 4 waves owns
//     128x64 as 4x2 blocks of v_mfma_i32_32x32x32_i8 (128 int32 accumulators
//     per lane), two waves per SIMD so one's MFMAs run while the other waits
//     at the stage barrier; each 16-byte A fragment read from LDS feeds two
//     MFMAs, each B fragment four (a 4-wave 128x128 layout is kept as NW = 4);
//   * K advances 128 bytes per stage; a stage is 2 x 256 rows x 128 B = 64 KiB
//     and two stages (128 KiB of the 160 KiB LDS) alternate: one stage's
//     copies in flight while the other is read (four k-substeps of 32 B);
//   * global -> LDS copies go straight into LDS (16 B per lane, no VGPR round
//     trip); a wave-load fills 1 KiB = 8 rows, the lane -> global address map
//     applies the LDS swizzle, so the fixed lane-ordered LDS destination lands
//     each 16-byte chunk at its swizzled slot.  Operands under 2 GiB use the
//     buffer form (buffer_load_dwordx4 ... lds): a lane's 32-bit row offset is
//     fixed for the whole K loop and the stage's K offset is one scalar, so a
//     copy needs no per-stage address arithmetic (8192^3: 441.6 against 457.8
//     us, same box, same bits); larger ones use global_load_lds_dwordx4 with
//     64-bit addresses;
//   * LDS rows are 128 B with 16-byte chunk c of row r stored at slot
//     c ^ ((r >> 1) & 7) (swz), which spreads the rows an MFMA operand read
//     touches over all banks;
//   * workgroup ids are remapped so each XCD (ids = xcd mod 8) receives a
//     contiguous run of tiles, walked in groups of GROUP_M tile rows, so the
//     workgroups resident on one XCD share A and B panels in its L2;
//   * one persistent workgroup per CU walks tiles b, b + gridDim.x, ...; a
//     tile's last K stage issues the next tile's first stage into the LDS
//     slot it frees, so the next tile starts on landed data (8192^3 +0.5-0.6%
//     over 3 same-box passes, same bits), and, once its own reads are done,
//     the next tile's second stage into its own slot, ahead of the tile's C
//     stores: vmcnt counts stores too, so a wait for copies issued after the
//     stores would drain them (8192^3: 437.8 -> 431.8 us, medians of 6
//     alternated same-box runs, same bits).
// Requirements (checked by the launcher): K % 128 == 0, 16-byte aligned A/BT.
// Rows past M or N read the last valid row (no fault, results discarded).
#include <algorithm>
#include <type_traits>

#include "device_util.h"
#include "epilogue.h"
#include "ie_internal.h"

namespace ie {
namespace {

// 128-byte stages, two of them (128 KiB of LDS): one stage's copies in flight
// while the other is computed, with half the barriers of 64-byte stages in a
// four-deep ring (2396 against 2266 TOP/s at 8192^3, same box, same bits).
constexpr int BM = 256, BN = 256, BK = 128;
constexpr int NSTAGE = 256 / BK;
constexpr int OPER = BM * BK;          // bytes of one operand tile per stage
constexpr int STAGE = 2 * OPER;        // A + B
constexpr int GROUP_M = 4;             // measured ahead of 2, 8 and 16
constexpr int CHUNKS = BK / 16;        // 16-byte chunks per LDS row
constexpr int ROWS_PER_LOAD = 64 / CHUNKS;          // rows one wave-load fills

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gbl_ptr_t;

// The 16 rows one quarter-wave of an MFMA operand read touches cover all 64
// banks when chunk c of row r sits at slot c ^ swz(r): (r >> 2) & 3 for
// 64-byte rows, (r >> 1) & 7 for 128-byte rows.
__device__ __forceinline__ int swz(int r) { return CHUNKS == 4 ? (r >> 2) & 3 : (r >> 1) & 7; }

// Copies rows [r0, r0 + ROWS_PER_LOAD) x BK bytes of a K-contiguous operand
// into LDS with one wave-wide 16-byte-per-lane direct load.
__device__ __forceinline__ void load_rows(const int8_t* __restrict__ src, int ld, int rows_valid,
                                          int row0, int k0, int r0, int8_t* lds_oper) {
    const int lane = threadIdx.x & 63;
    const int r = r0 + lane / CHUNKS;
    const int c = (lane % CHUNKS) ^ swz(r);
    const int gr = min(row0 + r, rows_valid - 1);
    const int8_t* g = src + (size_t)gr * ld + k0 + c * 16;
    __builtin_amdgcn_global_load_lds((gbl_ptr_t)g, (lds_ptr_t)(lds_oper + r0 * BK), 16, 0, 0);
}

// The buffer form of load_rows: `voff` = the lane's byte offset of its row
// and chunk (row clamped to the valid rows), `k0` the stage's K offset; the
// descriptor covers the operand's `nbytes` (loads past it would read 0).
__device__ __forceinline__ void load_rows_buf(const int8_t* src, uint32_t nbytes, uint32_t voff, int k0,
                                              int8_t* lds_dst) {
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(src), 0, nbytes, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds_dst, 16, voff, k0, 0, 0);
}

__device__ __forceinline__ i32x4 read_frag(const int8_t* lds_oper, int row, int chunk) {
    return *reinterpret_cast<const i32x4*>(lds_oper + row * BK + ((chunk ^ swz(row)) << 4));
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// 4 x 4 transpose inside each lane quad: on entry lane j of the quad holds
// element (r, j) in x[r], on return element (j, c) in x[c].  Two butterfly
// rounds, each trading one bit of the lane index for one bit of the register
// index through a DPP quad permutation (quad_perm [1, 0, 3, 2], then
// [2, 3, 0, 1]).
__device__ __forceinline__ void quad_transpose(int32_t (&x)[4], int j) {
    const bool b0 = j & 1, b1 = j & 2;
#pragma unroll
    for (int s = 0; s < 2; ++s) {  // lane bit 0 <-> register bit 0: registers 2s, 2s + 1
        const int32_t send = b0 ? x[2 * s] : x[2 * s + 1];
        const int32_t recv = __builtin_amdgcn_update_dpp(0, send, 0xB1, 0xf, 0xf, false);
        x[2 * s] = b0 ? recv : x[2 * s];
        x[2 * s + 1] = b0 ? x[2 * s + 1] : recv;
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {  // lane bit 1 <-> register bit 1: registers s, s + 2
        const int32_t send = b1 ? x[s] : x[s + 2];
        const int32_t recv = __builtin_amdgcn_update_dpp(0, send, 0x4E, 0xf, 0xf, false);
        x[s] = b1 ? recv : x[s];
        x[s + 2] = b1 ? x[s + 2] : recv;
    }
}

// NW = 4: 2 x 2 waves of 128 x 128 (one wave per SIMD); NW = 8: 2 x 4 waves
// of 128 x 64 (two per SIMD, so one wave's MFMAs can run while the other
// waits at the stage barrier or for its copies).
// BUF: M*K and N*K below 2^31, so operands take the buffer-form copies.
template <int EPI, int NW, bool BUF>
__global__ __launch_bounds__(64 * NW, 1) void gemm_i8_256_kernel(
    int M, int N, int K, const int8_t* __restrict__ A, const int8_t* __restrict__ BT,
    const float* __restrict__ sA, const float* __restrict__ sB, const float* bias,
    const float* residual, void* C, int tiles_m, int tiles_n) {
    __shared__ __attribute__((aligned(1024))) int8_t lds[NSTAGE * STAGE];

    // Persistent: workgroup b takes tiles b, b + gridDim.x, ... (one
    // workgroup per CU), and the last K stage of a tile issues the next
    // tile's first stage, so that tile starts on landed data instead of a
    // workgroup launch and a cold first copy.
    // XCD-aware, grouped tile order over the whole grid of tiles.
    const int ntiles = tiles_m * tiles_n;
    auto origin = [&](int T, int& m0_, int& n0_) {
        int id = T;
        if ((ntiles & 7) == 0) id = (id & 7) * (ntiles >> 3) + (id >> 3);
        const int per_group = GROUP_M * tiles_n;
        const int group = id / per_group;
        const int first_m = group * GROUP_M;
        const int gm = min(tiles_m - first_m, GROUP_M);
        const int in_group = id - group * per_group;
        m0_ = (first_m + in_group % gm) * BM;
        n0_ = (in_group / gm) * BN;
    };
    int T = blockIdx.x;
    int m0, n0;
    origin(T, m0, n0);

    constexpr int WN = NW / 2;              // waves across N
    constexpr int NJ = 4 / (NW / 4);        // 32-column blocks per wave: 4 or 2
    constexpr int LOADS_PER_WAVE = BM / ROWS_PER_LOAD / NW;  // per operand per stage
    const int lane = threadIdx.x & 63;
    // wave-uniform, so the copies' LDS destinations (M0) are scalar arithmetic
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;

    i32x16 acc[4][NJ];

    const int nk = K / BK;
    constexpr bool HAS_BIAS = EPI == IE_EPI_BIAS || EPI == IE_EPI_BIAS_GELU || EPI == IE_EPI_BIAS_RESIDUAL;
    constexpr bool HAS_RES = EPI == IE_EPI_BIAS_RESIDUAL;
    // Full tiles of a C with 16-byte rows (N % 4 == 0) leave through the
    // quad-transposed epilogue below, except with a residual (its 128 loads
    // per lane would not stay in registers).
    const bool quad_c = !HAS_RES && (N & 3) == 0 && ((uintptr_t)C & 15) == 0;
    // Copies stage kt_src of the tile at (m0_, n0_) into LDS slot `slot`.
    // Every iteration issues one stage, so the loop body is branch-free: the
    // last stage's iteration issues the next tile's stage 0, or, after the
    // last tile, re-reads stage nk-1 into the slot just freed, which is never
    // read again.
    uint32_t voA[LOADS_PER_WAVE], voB[LOADS_PER_WAVE], vnA[LOADS_PER_WAVE], vnB[LOADS_PER_WAVE];
    auto offsets = [&](int m0_, int n0_, uint32_t (&oa)[LOADS_PER_WAVE], uint32_t (&ob)[LOADS_PER_WAVE]) {
        if constexpr (BUF) {
#pragma unroll
            for (int j = 0; j < LOADS_PER_WAVE; ++j) {
                const int r = (wave * LOADS_PER_WAVE + j) * ROWS_PER_LOAD + lane / CHUNKS;
                const int c = (lane % CHUNKS) ^ swz(r);
                oa[j] = (uint32_t)(min(m0_ + r, M - 1) * K + c * 16);
                ob[j] = (uint32_t)(min(n0_ + r, N - 1) * K + c * 16);
            }
        }
    };
    auto issue = [&](int kt_src, int slot, int m0_, int n0_, const uint32_t (&oa)[LOADS_PER_WAVE],
                     const uint32_t (&ob)[LOADS_PER_WAVE]) {
        int8_t* sa = lds + slot * STAGE;
        int8_t* sb = sa + OPER;
        const int k0 = kt_src * BK;
#pragma unroll
        for (int j = 0; j < LOADS_PER_WAVE; ++j) {
            const int r0 = (wave * LOADS_PER_WAVE + j) * ROWS_PER_LOAD;
            if constexpr (BUF) {
                load_rows_buf(A, (uint32_t)M * K, oa[j], k0, sa + r0 * BK);
                load_rows_buf(BT, (uint32_t)N * K, ob[j], k0, sb + r0 * BK);
            } else {
                load_rows(A, K, M, m0_, k0, r0, sa);
                load_rows(BT, K, N, n0_, k0, r0, sb);
            }
        }
    };
    constexpr int LOADS_PER_STAGE = 2 * LOADS_PER_WAVE;  // per wave
    static_assert(NSTAGE == 2, "the next tile's stage 0 goes into the slot the last stage frees");

    // Prologue of the first tile: stage 0 landed.
    offsets(m0, n0, voA, voB);
    issue(0, 0, m0, n0, voA, voB);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();

    const int frow = lane & 31;
    const int fchunk = lane >> 5;
    // Operand fragments live in two register slots: slot 0 = k-substep 0 of a
    // stage, slot 1 = k-substep 1.  An MFMA blocks instruction issue until the
    // matrix pipe takes it, so LDS reads and global copies are interleaved one
    // per MFMA (sched_group_barrier) to run in the shadow of the matrix work.
    i32x4 af[2][4], bf[2][NJ];
    auto frags = [&](const int8_t* sa, const int8_t* sb, int ks, int slot) {
#pragma unroll
        for (int i = 0; i < 4; ++i) af[slot][i] = read_frag(sa, wm * 128 + i * 32 + frow, ks * 2 + fchunk);
#pragma unroll
        for (int j = 0; j < NJ; ++j) bf[slot][j] = read_frag(sb, wn * 32 * NJ + j * 32 + frow, ks * 2 + fchunk);
    };
    auto mfma_rows = [&](int slot, int i0, int i1) {
#pragma unroll
        for (int i = i0; i < i1; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[slot][i], bf[slot][j], acc[i][j], 0, 0, 0);
    };
    frags(lds, lds + OPER, 0, 0);

    constexpr int SUB = BK / 32;  // MFMA k-substeps per stage (even)
    static_assert(SUB % 2 == 0, "fragment slots alternate within a stage");
    int base = 0;  // LDS slot of the tile's stage 0 (stage kt sits in slot (kt + base) % 2)
    bool first_tile = true;
    for (;;) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
    // the tile whose stage 0 the last K stage issues (this one again after the last tile)
    const int Tn = T + (int)gridDim.x;
    const bool more = Tn < ntiles;
    int mn0 = m0, nn0 = n0;
    if (more) origin(Tn, mn0, nn0);
    offsets(mn0, nn0, vnA, vnB);
    // One K stage; NEXT: its copies are the next tile's stage 0 (the last
    // stage), otherwise this tile's stage kt + 1; EARLY (stage 0 of every
    // tile after the first): stage 1 was issued by the previous tile's last
    // stage, ahead of that tile's C stores, and this wave's copies of it
    // landed at the wait that ends that tile's K loop, so this stage issues
    // nothing and its wait is for LDS reads only (the barrier covers the
    // other waves' copies): the previous tile's stores stay in flight instead
    // of being drained.  The last stage is peeled so every stage's body stays
    // one basic block, with the copies interleaved among its MFMAs.
    auto stage = [&](int kt, auto next_c, auto early_c) {
        constexpr bool NEXT = decltype(next_c)::value;
        constexpr bool EARLY = decltype(early_c)::value;
        const int8_t* sa = lds + ((kt + base) % NSTAGE) * STAGE;
        const int8_t* sb = sa + OPER;
#pragma unroll
        for (int ks = 0; ks < SUB; ++ks) {
            const int slot = ks & 1;
            __builtin_amdgcn_sched_barrier(0);
            if (ks + 1 < SUB) {
                // MFMAs on this substep's slot; in their shadow the next
                // substep's reads and, in the first, the copies of stage
                // kt + NSTAGE - 1 into the slot freed by iteration kt - 1
                if (ks == 0) {
                    if constexpr (NEXT)
                        issue(more ? 0 : nk - 1, (kt + 1 + base) % NSTAGE, mn0, nn0, vnA, vnB);
                    else if constexpr (!EARLY)
                        issue(kt + 1, (kt + 1 + base) % NSTAGE, m0, n0, voA, voB);
                }
                frags(sa, sb, ks + 1, slot ^ 1);
                mfma_rows(slot, 0, 4);
#pragma unroll
                for (int g = 0; g < 4 * NJ; ++g) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    if (ks == 0 && !EARLY) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
            } else {
                // the last substep: half its MFMAs, then stage kt+1 must have
                // landed (this wave's copies: vmcnt; everyone's: the barrier;
                // a bare s_barrier, since __syncthreads()' workgroup fence
                // drains vmcnt to 0), then its first reads beside the other half
                // (after the last stage of the last tile these read a stale
                // slot, unused; otherwise the next tile's stage 0)
                mfma_rows(slot, 0, 2);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (EARLY)
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                else
                    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"((NSTAGE - 2) * LOADS_PER_STAGE) : "memory");
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                {
                    const int8_t* na = lds + ((kt + 1 + base) % NSTAGE) * STAGE;
                    frags(na, na + OPER, 0, 0);
                }
                // the last stage: every wave is done with this slot (the
                // barrier above), so the next tile's stage 1 goes into it
                // now, ahead of this tile's stores
                if constexpr (NEXT)
                    if (more && nk >= 2) issue(1, (kt + base) % NSTAGE, mn0, nn0, vnA, vnB);
                mfma_rows(slot, 2, 4);
#pragma unroll
                for (int g = 0; g < 2 * NJ; ++g) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    int kt0 = 0;
    if (!first_tile && nk >= 2) {
        stage(0, std::false_type{}, std::true_type{});
        kt0 = 1;
    }
    for (int kt = kt0; kt + 1 < nk; ++kt) stage(kt, std::false_type{}, std::false_type{});
    stage(nk - 1, std::true_type{}, std::false_type{});
    // every copy this wave issued has landed, the next tile's stage 1 (issued
    // by the last stage) included: the next tile's first stage relies on it
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");

    // Full tiles with 16-byte C rows: the accumulators are transposed inside
    // each lane quad (quad_transpose), so lane j of a quad holds row 8q +
    // 4(l/32) + j of the quad's four consecutive columns and C leaves in
    // 16-byte non-temporal stores, 32 per lane instead of 128; a row then
    // needs one row scale per four values, so all of the tile's 16 row
    // scales, its column scales and biases are requested before the first
    // store, and no load waits behind the stores.  The per-element arithmetic
    // is epilogue_value's, as in the path below, so C has the same bits.
    const int h = lane >> 5;
    const int rbase = m0 + wm * 128 + 4 * h;
    if (quad_c && m0 + BM <= M && n0 + BN <= N) {
        const int jq = lane & 3;
        const int qcol = n0 + wn * 32 * NJ + (lane & 28);  // the quad's first column (block j = 0)
        float sb4[NJ][4] = {}, bv4[NJ][4] = {}, sa1[4][4] = {};
        if constexpr (EPI != IE_EPI_I32) {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    sb4[j][c] = sB[qcol + 32 * j + c];
                    if constexpr (HAS_BIAS) bv4[j][c] = bias[qcol + 32 * j + c];
                }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q) sa1[i][q] = sA[rbase + i * 32 + 8 * q + jq];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    int32_t x[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                    acc[i][j][4 * q + 3]};
                    quad_transpose(x, jq);
                    const size_t idx = (size_t)(rbase + i * 32 + 8 * q + jq) * N + qcol + 32 * j;
                    if constexpr (EPI == IE_EPI_I32) {
                        const i32x4 o = {x[0], x[1], x[2], x[3]};
                        __builtin_nontemporal_store(o, reinterpret_cast<i32x4*>(static_cast<int32_t*>(C) + idx));
                    } else {
                        f32x4 o;
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            o[c] = epilogue_value<EPI>(x[c], sa1[i][q], sb4[j][c], bv4[j][c], 0.0f);
                        __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(static_cast<float*>(C) + idx));
                    }
                }
    } else {
        // Partial tiles, other C widths and the residual epilogue: one store per
        // value.  Lane l of a 32x32 block holds rows 8q + 4(l/32) + r (q, r < 4)
        // of column l % 32.  Every operand the stores of a 32-row block need
        // (scales, bias, residual; clamped indices) is gathered before its
        // first store and consumed once in straight-line code: loaded inside
        // the branchy store loop, each would wait for all earlier stores
        // (vmcnt counts stores, and C may alias them).  Two waves per SIMD
        // leave no room for all 64 row scales beside the accumulators, so they
        // are gathered one block at a time.  C goes out as non-temporal stores
        // (2316 against 2187 TOP/s at 8192^3 with the stores cached in L2).
        const int cbase = n0 + wn * 32 * NJ + (lane & 31);
        float sb[NJ] = {}, bv[NJ] = {};
        if constexpr (EPI != IE_EPI_I32) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int n = min(cbase + j * 32, N - 1);
                sb[j] = sB[n];
                if constexpr (HAS_BIAS) bv[j] = bias[n];
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float sa[16] = {}, rv[16][NJ] = {};
            if constexpr (EPI != IE_EPI_I32) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int m = min(rbase + i * 32 + 8 * (v >> 2) + (v & 3), M - 1);
                    sa[v] = sA[m];
                    if constexpr (HAS_RES) {
#pragma unroll
                        for (int j = 0; j < NJ; ++j) rv[v][j] = residual[(size_t)m * N + min(cbase + j * 32, N - 1)];
                    }
                }
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    asm volatile("" ::"v"(sa[v]));
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        if constexpr (HAS_RES) asm volatile("" ::"v"(rv[v][j]));
                }
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    asm volatile("" ::"v"(sb[j]));
                    if constexpr (HAS_BIAS) asm volatile("" ::"v"(bv[j]));
                }
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int m = rbase + i * 32 + 8 * (v >> 2) + (v & 3);
                if (m >= M) continue;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int n = cbase + j * 32;
                    if (n < N)
                        store_epilogue_v<EPI, true>(C, (size_t)m * N + n, acc[i][j][v], sa[v], sb[j], bv[j], rv[v][j]);
                }
            }
        }
    }
    if (!more) break;
    first_tile = false;
    // the next tile: its stage 0 has landed and its first fragments are loaded
    T = Tn;
    m0 = mn0;
    n0 = nn0;
    base = (base + nk) % NSTAGE;
#pragma unroll
    for (int j = 0; j < LOADS_PER_WAVE; ++j) {
        voA[j] = vnA[j];
        voB[j] = vnB[j];
    }
    }
}

template <int EPI>
struct BigLaunch {
    static void run(const GemmArgs& a, hipStream_t s) {
        const int tm = (a.M + BM - 1) / BM, tn = (a.N + BN - 1) / BN;
        // 8 waves: 2231-2240 TOP/s steady state against 2153 with 4 (same box,
        // bit-identical C); with buffer-form copies 453.8 against 484.2 us.
        constexpr int NW = 8;
        const bool buf = (long long)a.M * a.K < (1LL << 31) && (long long)a.N * a.K < (1LL << 31);
        // one persistent workgroup per CU (128 KiB of LDS each)
        const unsigned grid = (unsigned)std::min<long long>((long long)tm * tn, num_cus());
        if (buf)
            gemm_i8_256_kernel<EPI, NW, true><<<grid, 64 * NW, 0, s>>>(
                a.M, a.N, a.K, reinterpret_cast<const int8_t*>(a.A), reinterpret_cast<const int8_t*>(a.BT),
                a.sA, a.sB, a.bias, a.residual, a.C, tm, tn);
        else
            gemm_i8_256_kernel<EPI, NW, false><<<grid, 64 * NW, 0, s>>>(
                a.M, a.N, a.K, reinterpret_cast<const int8_t*>(a.A), reinterpret_cast<const int8_t*>(a.BT),
                a.sA, a.sB, a.bias, a.residual, a.C, tm, tn);
    }
};

}  // namespace

bool gemm_i8_big_applies(const GemmArgs& a) {
    if (a.K % BK != 0 || a.K == 0) return false;
    if (((uintptr_t)a.A % 16) || ((uintptr_t)a.BT % 16)) return false;
    const long long tiles = (long long)((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    return tiles >= 128 && tiles < (1LL << 31);
}

void launch_gemm_i8_big(const GemmArgs& a, hipStream_t s) { dispatch_epilogue<BigLaunch>(a.epi, a, s); }

}  // namespace ie
