// gemm_i8_wide.hip — INT8 GEMM for write-dominated shapes on gfx950: a few
// hundred activation rows (M <= 1024), K = 768 and a wide N, such as BASELINE's
// M = 512 rows against the 768 x 50257 LM-head weights (39.5 GOP, but 103 MB of
// fp32 C against 38.6 MB of weights and 0.4 MB of activations).
//
// Result identical to the reference's K14 kernel (kernels/quantization/
// 14_int8_gemm.cu:65-170): exact int32 K-sum, then the dequant epilogue.
//
// Tile kernels re-read both operand panels for every tile: at this shape the
// 128 x 64 LDS tile kernel moves 453 MB of panels from L2 into the CUs for a
// 142 MB problem, and its K loop alone took 35.5 us of its 47.6 (a lab copy
// with the stores taken out).  Here the small operand stays put and only the
// weights stream:
//   * one persistent workgroup per CU owns a panel of 256 A rows for its whole
//     life, held in registers: each of its NW waves keeps 256 / NW rows x 768
//     bytes as the A operands of v_mfma_i32_32x32x32_i8 (96 VGPRs for 32 rows;
//     with 8 waves, two per SIMD, one wave's MFMAs run while the other waits
//     for its LDS fragment);
//   * B streams through LDS in chunks of 32 weight rows (= 32 C columns) x 768
//     bytes (24 KiB), in a ring of RING chunks filled by global_load_lds_dwordx4
//     (16 bytes per lane straight into LDS) RING - 1 chunks ahead; every wave
//     reads the whole chunk (a 16-byte B fragment feeds one MFMA per 32 rows
//     the wave holds), so a weight byte is fetched into a CU once per panel;
//   * each finished chunk (256 x 32 of C) is stored while the next chunks'
//     copies are in flight, so C leaves in a steady stream instead of bursts
//     at tile ends; the chunk's column scales and bias come with its copies
//     (4-byte LDS-direct loads), so the loop holds no register load, which
//     would make the compiler drain every copy in flight before its use;
//   * panels and chunks map to workgroups XCD-aware: the P panel workgroups of
//     one chunk stream sit on the same XCD (workgroup id mod 8) and walk the
//     same chunks at the same pace, so the second panel's copy of a chunk is
//     an L2 hit; with P panels a weight byte leaves HBM once and enters P CUs.
//   * the A panel (8 blocks of 32 rows x 768 bytes, one per wave) arrives
//     mostly through LDS: a block has a B chunk's shape and layout, so blocks
//     0-5 are copied with the same coalesced 1 KiB LDS-direct wave-loads and
//     their waves read their operands from there, while waves 6 and 7 load
//     theirs straight into registers at the same time (each wave instruction
//     32 rows x 32 bytes: the whole panel that way cost 4.5-6 us of a 34 us
//     launch; a second LDS round for blocks 6-7 was one more round trip);
//   * the int32 K-sum is exact in any order, so each workgroup walks K in its
//     own rotated order (k-step s covers K bytes 32 ((s + rot) mod 24) ..),
//     which spreads the workgroups' simultaneous requests for one panel;
// LDS layout of a chunk: row r (weight row, C column) holds its 48 16-byte
// pieces with piece t at slot t ^ (r & 7), so the 8 lanes of a fragment read
// group hit 8 different bank groups.
// Requirements (checked by gemm_i8_wide_applies): K == 768, 16-byte aligned
// A / BT, M <= 1024.  Rows past M or N read the last valid row (results
// discarded).
#include <algorithm>

#include "device_util.h"
#include "epilogue.h"
#include "ie_internal.h"

namespace ie {
namespace {

constexpr int KW = 768;              // the K this kernel takes
constexpr int KS = KW / 32;          // MFMA k-steps per chunk (24)
constexpr int PIECES = KW / 16;      // 16-byte pieces per weight row (48)
constexpr int PANEL = 256;           // A rows per workgroup
constexpr int CN = 32;               // C columns per chunk
constexpr int CHUNK = CN * KW;       // bytes of one B chunk (24 KiB)
constexpr int RING = 4;              // B chunks in the ring, RING - 1 in flight
constexpr int SLOTS = 6;             // 24 KiB LDS slots: the B ring, and the A panel's first 6 blocks at start

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* gbl_ptr_t;

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N < 63 ? N : 63) : "memory");
}

// The wait for chunk j < RING - 1, issued in the prologue back to back: after
// its copies come those of chunks j + 1 .. RING - 2 and j whole iterations
// (ITER operations each) of the loop.
template <int J, int COPIES, int ITER>
__device__ __forceinline__ void wait_prologue_chunk(int j) {
    if constexpr (J < RING - 1) {
        if (j == J) {
            wait_vm<(RING - 2 - J) * COPIES + J * ITER>();
            return;
        }
        wait_prologue_chunk<J + 1, COPIES, ITER>(j);
    }
}

template <int EPI, bool NT, int NW>
__global__ __launch_bounds__(64 * NW, 1) void gemm_i8_wide_kernel(int M, int N, const int8_t* __restrict__ A,
                                                              const int8_t* __restrict__ BT,
                                                              const float* __restrict__ sA,
                                                              const float* __restrict__ sB, const float* bias,
                                                              const float* residual, void* C, int panels) {
    // SLOTS chunk slots (the B ring uses RING of them), then per ring slot
    // the chunk's 32 column scales and 32 biases
    __shared__ __attribute__((aligned(1024))) int8_t lds[SLOTS * CHUNK + RING * 256];
    float (*cols)[64] = reinterpret_cast<float (*)[64]>(lds + SLOTS * CHUNK);
    constexpr bool HAS_SCALE = EPI != IE_EPI_I32;
    constexpr bool HAS_BIAS = EPI == IE_EPI_BIAS || EPI == IE_EPI_BIAS_GELU || EPI == IE_EPI_BIAS_RESIDUAL;
    constexpr bool HAS_RES = EPI == IE_EPI_BIAS_RESIDUAL;
    constexpr int RB = PANEL / 32 / NW;           // 32-row blocks per wave
    constexpr int WLOADS = CHUNK / 1024 / NW;     // wave-loads of 1 KiB per wave per chunk
    static_assert(RB * NW * 32 == PANEL && WLOADS * NW * 1024 == CHUNK, "panel and chunk split over waves");
    static_assert(RB == 1 && SLOTS >= RING && SLOTS < NW, "A blocks 0..SLOTS-1 through LDS, the rest direct");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int fr = lane & 31, h = lane >> 5;

    // Workgroup w sits on XCD w % 8; the workgroups of one XCD are split into
    // `panels` groups that walk the same chunk stream.
    const int G = gridDim.x;                 // a multiple of 8 * panels
    const int w = blockIdx.x;
    const int x = w & 7, l = w >> 3;
    const int per_xcd = G >> 3;
    const int panel = l % panels;
    const int streams = G / panels;
    const int stream = x * (per_xcd / panels) + l / panels;
    const int nchunks = (N + CN - 1) / CN;
    const int mine = stream < nchunks ? (nchunks - 1 - stream) / streams + 1 : 0;
    if (mine == 0) return;
    const int last_c = stream + (mine - 1) * streams;

    // B chunk c into ring slot `slot`: this wave's WLOADS wave-loads, and
    // (every wave, the same values) the chunk's 32 column scales and biases
    // into cols[slot]; past the workgroup's last chunk it re-reads that chunk
    // (the loop stays branch-free; the slot is not read again).
    auto issue = [&](int j, int slot) {
        const int c = min(stream + j * streams, last_c);
        int8_t* dst = lds + slot * CHUNK;
#pragma unroll
        for (int u = 0; u < WLOADS; ++u) {
            const int jl = wave * WLOADS + u;
            const int q = jl * 64 + lane;
            const int r = q / PIECES, t = q % PIECES;
            const int row = min(c * CN + r, N - 1);
            const int8_t* src = BT + (size_t)row * KW + ((t ^ (r & 7)) << 4);
            __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(dst + jl * 1024), 16, 0, 0);
        }
        if constexpr (HAS_SCALE) {
            const int nc = min(c * CN + fr, N - 1);
            const float* src = (HAS_BIAS && h) ? bias + nc : sB + nc;
            __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)&cols[slot][0], 4, 0, 0);
        }
    };

    // The wave's A rows (RB blocks of 32) as MFMA operands: lane (fr, h) of
    // k-step s holds bytes 32 kk(s) + 16 h .. + 16 of its row, kk(s) = (s +
    // rot) mod KS; and their scales.
    const int rot = (stream * 7 + panel * 13) % KS;
    auto kk = [&](int s) { const int t = s + rot; return t < KS ? t : t - KS; };
    const int mrow0 = panel * PANEL + wave * 32 * RB;
    // A block b (rows panel * PANEL + 32 b ..) into LDS slot `slot`, in the
    // B chunk layout; `nb` blocks copied by all waves together, wave-load
    // jl of the set covering 1 KiB of block jl / 24
    auto issue_a = [&](int b0, int slot0, int nb) {
        const int per = nb * (CHUNK / 1024) / NW;
#pragma unroll
        for (int u = 0; u < per; ++u) {
            const int jl = wave * per + u;
            const int blk = jl / (CHUNK / 1024), jb = jl % (CHUNK / 1024);
            const int q = jb * 64 + lane;
            const int r = q / PIECES, t = q % PIECES;
            const int row = min(panel * PANEL + (b0 + blk) * 32 + r, M - 1);
            const int8_t* src = A + (size_t)row * KW + ((t ^ (r & 7)) << 4);
            __builtin_amdgcn_global_load_lds((gbl_ptr_t)src, (lds_ptr_t)(lds + (slot0 + blk) * CHUNK + jb * 1024), 16, 0,
                                             0);
        }
    };
    // the wave's operands from its block in LDS (same reads as a B fragment)
    i32x4 a[RB][KS];
    auto read_a = [&](int slot) {
        const int8_t* al = lds + slot * CHUNK + fr * KW;
#pragma unroll
        for (int s = 0; s < KS; ++s) a[0][s] = *reinterpret_cast<const i32x4*>(al + (((2 * kk(s) + h) ^ (fr & 7)) << 4));
    };
    // Lane (fr, h) of a 32 x 32 accumulator block holds rows 8 q + 4 h + r
    // (v = 4 q + r) of column fr.
    auto mrow = [&](int i, int v) { return mrow0 + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3); };
    float sa[RB][16] = {};
    if constexpr (HAS_SCALE) {
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) sa[i][v] = sA[min(mrow(i, v), M - 1)];
    }

    // Prologue: waves SLOTS.. load their A block into registers while all
    // waves copy blocks 0 .. SLOTS - 1 into slots 0 .. SLOTS - 1 (and the row
    // scales were requested before both); once everything has landed the
    // first waves read their blocks, and after that B chunks 0 .. RING - 2 go
    // into the ring slots.
    if (wave >= SLOTS) {
        const int8_t* ar = A + (size_t)min(mrow0 + fr, M - 1) * KW + 16 * h;
#pragma unroll
        for (int s = 0; s < KS; ++s) a[0][s] = *reinterpret_cast<const i32x4*>(ar + 32 * kk(s));
    }
    issue_a(0, 0, SLOTS);
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) asm volatile("" ::"v"(sa[i][v]));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (wave < SLOTS) read_a(wave);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // every operand register is final here (the compiler's own waits, if
    // any, stay out of the loop)
#pragma unroll
    for (int s = 0; s < KS; ++s) asm volatile("" ::"v"(a[0][s]));
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int p = 0; p < RING - 1; ++p) issue(p, p);
    constexpr int COPIES = WLOADS + (HAS_SCALE ? 1 : 0);

    // Vector-memory operations a wave issues per chunk: its copies, the
    // residual gathers and the C stores (vmcnt counts stores).  Waiting at
    // chunk j (j >= RING - 1) finds the stores and gathers of chunk
    // j - RING + 1 and RING - 2 whole chunks issued after chunk j's copies;
    // the first RING - 1 chunks were issued in the prologue, so fewer
    // operations follow them.
    constexpr int GATHER = HAS_RES ? 16 * RB : 0;
    constexpr int STORES = 16 * RB;
    constexpr int AFTER = GATHER + STORES + (RING - 2) * (COPIES + GATHER + STORES);
    // vmcnt holds 6 bits: past 63 the wait also covers a few older stores
    // (and at most the next chunk's copies), which have had a chunk's time
    constexpr int WAITN = AFTER < 63 ? AFTER : 63;
    static_assert(AFTER >= WAITN, "the wait covers chunk j's copies");
    constexpr int ITER = COPIES + GATHER + STORES;
    // A store whose lanes all hold rows past M is branched around (no lane
    // active), so only a wave whose 32 rows are all below M is sure to issue
    // its STORES per chunk; the others count only their copies and gathers,
    // which are unconditional.  (A chunk's first column is always below N,
    // so a full-row wave issues every store.)
    const bool rows_full = mrow0 + 32 * RB <= M;
    constexpr int ITER_C = COPIES + GATHER;
    constexpr int AFTER_C = GATHER + (RING - 2) * ITER_C;
    constexpr int WAITN_C = AFTER_C < 63 ? AFTER_C : 63;

    for (int j = 0; j < mine; ++j) {
        const int c = stream + j * streams;
        const int slot = j % RING;
        // chunk j landed: this wave's copies (vmcnt), every wave's (barrier);
        // the barrier also means every wave is done reading chunk j - 1, whose
        // slot the copies issued next refill
        __builtin_amdgcn_sched_barrier(0);
        if (j >= RING - 1) {
            if (rows_full)
                wait_vm<WAITN>();
            else
                wait_vm<WAITN_C>();
        } else if (rows_full) {
            wait_prologue_chunk<0, COPIES, ITER>(j);
        } else {
            wait_prologue_chunk<0, COPIES, ITER_C>(j);
        }
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue(j + RING - 1, (j + RING - 1) % RING);

        // epilogue operands of this chunk (the residual requested before the MFMAs)
        const int n = c * CN + fr;
        const int nc = min(n, N - 1);
        float sb = 0.0f, bv = 0.0f, rv[RB][16] = {};
        if constexpr (HAS_SCALE) sb = cols[slot][fr];
        if constexpr (HAS_BIAS) bv = cols[slot][32 + fr];
        if constexpr (HAS_RES) {
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) rv[i][v] = residual[(size_t)min(mrow(i, v), M - 1) * N + nc];
        }

        const int8_t* bl = lds + slot * CHUNK + fr * KW;
        const int sw = fr & 7;
        i32x16 acc[RB];
#pragma unroll
        for (int i = 0; i < RB; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][v] = 0;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const i32x4 b = *reinterpret_cast<const i32x4*>(bl + (((2 * kk(s) + h) ^ sw) << 4));
#pragma unroll
            for (int i = 0; i < RB; ++i) acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i][s], b, acc[i], 0, 0, 0);
        }

        if (n < N) {
#pragma unroll
            for (int i = 0; i < RB; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int m = mrow(i, v);
                    if (m < M)
                        store_epilogue_v<EPI, NT>(C, (size_t)m * N + n, acc[i][v], sa[i][v], sb, bv, rv[i][v]);
                }
        }
    }
    // no copy may still be writing LDS when the workgroup ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int EPI>
struct WideLaunch {
    static void run(const GemmArgs& a, hipStream_t s) {
        const int panels = (a.M + PANEL - 1) / PANEL;
        const int G = std::max(8 * panels, num_cus() / (8 * panels) * (8 * panels));
        // 8 waves of 32 rows (two per SIMD): 4 of 64 rows (192 A registers,
        // one wave per SIMD) waited on every LDS fragment read
        constexpr int NW = 8;
        gemm_i8_wide_kernel<EPI, false, NW><<<G, 64 * NW, 0, s>>>(
            a.M, a.N, reinterpret_cast<const int8_t*>(a.A), reinterpret_cast<const int8_t*>(a.BT), a.sA, a.sB,
            a.bias, a.residual, a.C, panels);
    }
};

}  // namespace

bool gemm_i8_wide_applies(const GemmArgs& a) {
    if (a.K != KW || a.M > 4 * PANEL) return false;
    if (((uintptr_t)a.A % 16) || ((uintptr_t)a.BT % 16)) return false;
    // enough chunks that every workgroup streams several
    const long long panels = (a.M + PANEL - 1) / PANEL;
    return (long long)((a.N + CN - 1) / CN) * panels >= 6LL * num_cus();
}

void launch_gemm_i8_wide(const GemmArgs& a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    dispatch_epilogue<WideLaunch>(a.epi, a, s);
}

}  // namespace ie
