// decode_attn.hip — split-K paged decode attention for gfx950.
//
// Computes what the reference's K13 computes (kernels/decode/13_decode_attn.cuh
// :30-189 and 13_decode_attn.cu:10-109): for every sequence b and query head h,
// softmax(q . K^T / sqrt(d)) V over the sequence's first context_lens[b] cached
// tokens, gathered through the block table, with the work split over KV blocks
// (pass 1 writes per-split partials (o, m, l); pass 2 merges them).  The split
// plan is the caller's (the reference rule by default, see capi.cpp).
//
// MI355X layout of pass 1 (grid = splits x H_kv x B):
//   * one workgroup per (b, kv head, split) serves all G = H_q/H_kv query heads
//     of that KV head, so each K/V byte is read from HBM once (the reference
//     launches one block per query head and re-reads KV G times);
//   * the split's tokens are walked in 16-token chunks; inside a chunk
//     each 16-lane DPP row owns one token per step and each lane one
//     d/16-element slice of it, so a row reads the token's whole K (or V)
//     vector as one contiguous 256/512-byte run with 16-byte loads;
//   * q . k is reduced over the row with four DPP rotations; the chunk max
//     is shared across the wave with two cross-row shuffles, so a wave keeps
//     one running max per head and rescales once per 16 tokens, not per token;
//   * scores are pre-multiplied by log2(e)/sqrt(d), so the softmax uses the
//     hardware exp2; partials store m in that base-2 domain;
//   * a long split (>= 256 tokens) is one wave: no LDS merge and no barrier
//     at the end, so a finishing wave never holds up the memory pipeline of
//     the others (measured ~9% faster than four waves per split at ctx 8192);
//     the waves of several KV heads share a workgroup so the heads' slices of
//     a block are fetched together; each wave keeps a ring of chunks in
//     flight (three for fp32 d = 128), and such launches cut the batch's
//     chunks into equal workgroup ranges across sequences (balanced kernel
//     below) instead of one workgroup per (b, split);
//     a short one is shared by four waves that take its chunks round-robin
//     and merge in LDS, so its few chunks load in parallel;
//   * every split writes its slot, empty ones as (o=0, m=-inf, l=0), so the
//     merge never reads stale workspace (the reference skips the write).
// Pass 2 (one wave per (b, query head)) merges the splits with l > 0; with a
// single split pass 1 writes O itself and pass 2 is skipped.  (A
// "last split to arrive merges" variant needs a device-scope release per
// workgroup, which on gfx950 writes back the XCD's L2 and cost more than the
// second launch.  Without the release, partials written by agent-scope
// atomic stores, a counter per (b, kv head) and the last workgroup merging
// with agent-scope loads gave the same bits but took longer still: cfg3
// 13.65 -> 16.5 us, since that workgroup's store, counter and load round
// trips run one after another at the end of the launch.)
#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>

#include "attn_split.h"
#include "device_util.h"
#include "ie_internal.h"

namespace ie {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
// Cache-policy bits of an LDS-direct load: non-temporal (the cache stream of
// a long-context launch is read once; non-temporal K and V loads measured
// +1-2.5% for fp32 cfg4 at ctx 4096-32768).
constexpr int kCpolNT = 2;

// One-wave splits: KV heads (waves) per workgroup at most, and KV chunks per
// wave in the register ring (R - 1 in flight while one is computed).  The
// stream is bound by bytes in flight per CU; with d = 128 fp32 a 16-token
// chunk is 64 VGPRs per lane, so the ring that keeps three chunks in flight
// only fits at one wave per SIMD (arch VGPRs plus AGPRs), i.e. 4 heads per
// workgroup: measured 0.676-0.687 of HBM peak at ctx 8192 against 0.634-0.653
// for 8 heads with a ping-pong pair.  bf16 and d = 64 keep 8 heads and the
// pair (deeper rings or 32-token bf16 chunks measured slower: the unpacked
// elements need the registers).  G = 8 at d = 128 holds 8 heads' q and o per
// wave, so it takes 4 waves per workgroup (one per SIMD, all registers) and
// the pair: at 8 waves, or with a four-chunk fp32 ring, it spilled and ran at
// 0.15-0.25 of HBM peak against 0.52-0.66 (fp32 then; 0.68-0.70 at ctx 8192
// with v_exp_f32 weights and scalar block ids), and a three-chunk fp32 ring
// spills too.  bf16 at G >= 4 takes the MFMA walk below.
template <int D, typename KV, int G>
constexpr int wave_heads() { return (D == 128 && sizeof(KV) == 4) || (D == 128 && G == 8) ? 4 : 8; }
template <int D, typename KV, int G>
constexpr int wave_ring() { return D == 128 && sizeof(KV) == 4 && G < 8 ? 4 : 2; }

// Merges the S split partials (o[D], m, l) of one (b, query head) with one
// wave: lanes read the (m, l) of 64 splits at a time in parallel, and the
// o rows are accumulated with loads that do not depend on each other, so the
// merge costs a few memory round trips rather than one per split.  Empty
// splits hold (0, -inf, 0) and get weight 0.
template <int D>
__device__ __forceinline__ void merge_head(const float* __restrict__ w, int S,
                                           float* __restrict__ out, int lane) {
    constexpr int PER = D / 64;
    float mx = -INFINITY;
    for (int s0 = 0; s0 < S; s0 += 64) {
        const int s = s0 + lane;
        if (s < S) {
            const float* p = w + (size_t)s * (D + 2);
            if (p[D + 1] > 0.0f) mx = fmaxf(mx, p[D]);
        }
    }
    mx = wave_max(mx);
    float o[PER], l = 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) o[i] = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 64) {
        const int s = s0 + lane;
        float f = 0.0f;
        bool on = false;
        if (s < S) {
            const float* p = w + (size_t)s * (D + 2);
            const float ls = p[D + 1];
            on = ls > 0.0f;
            f = on ? exp2_sm(p[D] - mx) : 0.0f;
            l = fmaf(ls, f, l);
        }
        // Splits with l > 0; an empty one (l = 0, whose o the balanced pass
        // does not write) reads split s0's row instead (a cache hit) and adds
        // 0, so its own o is never touched.
        const unsigned long long live = __ballot(on);
        const int cnt = min(64, S - s0);
        const float* p0 = w + (size_t)s0 * (D + 2) + lane;
        for (int jb = 0; jb < cnt; jb += 8) {
            // Eight splits' o rows in flight, branch-free; their addresses
            // depend only on the scalar mask, so the loads go out at once.
            float pv[8][PER];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int j = (live >> (jb + u)) & 1ull ? jb + u : 0;
#pragma unroll
                for (int i = 0; i < PER; ++i) pv[u][i] = p0[(size_t)j * (D + 2) + 64 * i];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const bool lv = (live >> (jb + u)) & 1ull;
                const float fj = __shfl(f, (jb + u) & 63, 64);
#pragma unroll
                for (int i = 0; i < PER; ++i) o[i] = fmaf(lv ? pv[u][i] : 0.0f, lv ? fj : 0.0f, o[i]);
            }
        }
    }
    l = wave_sum(l);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int i = 0; i < PER; ++i) out[lane + 64 * i] = o[i] * inv;
}

// fp32 d = 128 one-wave splits with the K half of each chunk landed in LDS
// (global_load_lds_dwordx4, 16 bytes per lane straight into a per-wave ring
// slot) and the V half in registers.  The ring stays at R = 4 chunks, R - 1
// in flight: a fifth keeps 80 vector-memory operations outstanding, past
// vmcnt's 63, and the compiler then drains the counter to zero.  What the LDS
// buys is register room: no K copies, and the V loads stay where they are
// issued (opaque_global), so the ring streams instead of issuing three chunks
// at once and draining; measured 0.67 / 0.69-0.72 / 0.78 of HBM peak at ctx
// 4096 / 8192 / 32768 against 0.64 / 0.67-0.69 / 0.77 for the register ring
// (same boxes, 32 x 32/8 heads, ragged).  Lane (grp, li) loads K of token
// c0 + 4j + grp, elements 8 li .. 8 li + 7, as two 16-byte pieces into piece
// 2j + h of the slot at lane * 16, and reads back exactly the bytes it loaded.
// Ordering (the compiler does not see the LDS reads, which are inline asm,
// so it neither drains the ring before them nor knows they wait on the DMA):
//   * a chunk's K copies are issued before its V loads (a scheduling barrier
//     keeps that order) and vector memory operations retire in order, so once
//     the chunk's last V load has landed its K is in LDS; the K read takes
//     that V register as an input operand, which makes the compiler wait for
//     it first;
//   * the read waits for its own LDS results before returning, and a slot is
//     refilled only by a later step, after the read.
// Block size 16 only (block ids by scalar loads, no vector table loads).
constexpr int kKldsRing = 4;
typedef __attribute__((address_space(3))) void* klds_ptr_t;
typedef __attribute__((address_space(1))) void* kgbl_ptr_t;

template <int G, int NW>
__device__ __forceinline__ void split_partial_klds(const float* __restrict__ Q, const float* __restrict__ kcache,
                                                   const float* __restrict__ vcache, const int* __restrict__ bt,
                                                   int b, int kvh, int H_q, int H_kv, int tok0, int tok1, int lane,
                                                   float qscale, float (&m)[G], float (&l)[G], float (&o)[G][8]) {
    constexpr int D = 128, EPL = 8, T = 4, R = kKldsRing, STEP = 16;
    // [wave][slot][piece][lane] 16-byte pieces: 8 KB per slot
    __shared__ __attribute__((aligned(16))) float4 kring[NW][R][2 * T][64];
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = lane >> 4, li = lane & 15;
    tok0 = __builtin_amdgcn_readfirstlane(tok0);
    tok1 = __builtin_amdgcn_readfirstlane(tok1);
    const size_t tok_stride = (size_t)H_kv * D;
    const float* kbase = kcache + (size_t)kvh * D + li * EPL;
    const float* vbase = opaque_global(vcache) + (size_t)kvh * D + li * EPL;

    float q[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
        load_q<EPL>(Q + ((size_t)b * H_q + (size_t)kvh * G + g) * D + li * EPL, q[g]);

    struct VChunk {
        float4 v[T][2];
        bool valid[T];
    };
    VChunk buf[R];
    int c0 = tok0;
    // the chunk's block id is wave-uniform: a scalar load, counted by lgkmcnt
    auto phys = [&](int cs) { return bt[__builtin_amdgcn_readfirstlane(min(cs, tok1 - 1) >> 4)]; };
    // an empty walk reads no table entry (tok1 == 0 would index bt[-1])
    int pn = c0 < tok1 ? phys(c0) : 0;
    // Issues chunk cs: K pieces into ring slot `slot`, then V into vb.
    auto issue = [&](VChunk& vb, int slot, int cs) {
        const int ph = pn;
        pn = phys(cs + STEP);
#pragma unroll
        for (int j = 0; j < T; ++j) {
            const int pos = cs + 4 * j + grp;
            const int pc = min(pos, tok1 - 1);
            const float* kp = kbase + ((size_t)ph * 16 + (pc & 15)) * tok_stride;
#pragma unroll
            for (int h = 0; h < 2; ++h)
                __builtin_amdgcn_global_load_lds((kgbl_ptr_t)(kp + 4 * h), (klds_ptr_t)&kring[wv][slot][2 * j + h][0],
                                                 16, 0, kCpolNT);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < T; ++j) {
            const int pos = cs + 4 * j + grp;
            vb.valid[j] = pos < tok1;
            const int pc = min(pos, tok1 - 1);
            const f32x4_t* vp = reinterpret_cast<const f32x4_t*>(vbase + ((size_t)ph * 16 + (pc & 15)) * tok_stride);
            const f32x4_t v0 = __builtin_nontemporal_load(vp), v1 = __builtin_nontemporal_load(vp + 1);
            vb.v[j][0] = make_float4(v0.x, v0.y, v0.z, v0.w);
            vb.v[j][1] = make_float4(v1.x, v1.y, v1.z, v1.w);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    const bool any = c0 < tok1;
    if (any) {
#pragma unroll
        for (int p = 0; p < R - 1; ++p) issue(buf[p], p, c0 + p * STEP);
    }

#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) q[g][e] *= qscale;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[g][e] = 0.0f;
    }

    auto consume = [&](const VChunk& vb, int slot) {
        // K of this chunk from LDS, after its last V load has landed
        float4 kv[T][2];
        const unsigned base = (unsigned)(uintptr_t)&kring[wv][slot][0][lane];
        asm volatile(
            "ds_read_b128 %0, %8\n\t"
            "ds_read_b128 %1, %8 offset:1024\n\t"
            "ds_read_b128 %2, %8 offset:2048\n\t"
            "ds_read_b128 %3, %8 offset:3072\n\t"
            "ds_read_b128 %4, %8 offset:4096\n\t"
            "ds_read_b128 %5, %8 offset:5120\n\t"
            "ds_read_b128 %6, %8 offset:6144\n\t"
            "ds_read_b128 %7, %8 offset:7168\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(kv[0][0]), "=&v"(kv[0][1]), "=&v"(kv[1][0]), "=&v"(kv[1][1]), "=&v"(kv[2][0]), "=&v"(kv[2][1]),
              "=&v"(kv[3][0]), "=&v"(kv[3][1])
            : "v"(base), "v"(vb.v[T - 1][1].w)
            : "memory");
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float sc[T];
#pragma unroll
            for (int j = 0; j < T; ++j) {
                const float kk[8] = {kv[j][0].x, kv[j][0].y, kv[j][0].z, kv[j][0].w,
                                     kv[j][1].x, kv[j][1].y, kv[j][1].z, kv[j][1].w};
                float dot = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) dot = fmaf(q[g][e], kk[e], dot);
                dot = row16_sum(dot);
                sc[j] = vb.valid[j] ? dot : -INFINITY;
            }
            float cm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            cm = max_xor32(max_xor16(cm));
            const float mn = fmaxf(m[g], cm);
            const float alpha = exp2_sm(m[g] - mn);
            float p[T], psum = 0.0f;
#pragma unroll
            for (int j = 0; j < T; ++j) {
                p[j] = exp2_sm(sc[j] - mn);
                psum += p[j];
            }
            l[g] = fmaf(l[g], alpha, psum);
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                float acc = o[g][e] * alpha;
#pragma unroll
                for (int j = 0; j < T; ++j) {
                    const float4 vv = vb.v[j][e >> 2];
                    const float ve = (e & 3) == 0 ? vv.x : (e & 3) == 1 ? vv.y : (e & 3) == 2 ? vv.z : vv.w;
                    acc = fmaf(p[j], ve, acc);
                }
                o[g][e] = acc;
            }
            m[g] = mn;
        }
    };
    if (any) {
        while (true) {
#pragma unroll
            for (int u = 0; u < R; ++u) {
                issue(buf[(u + R - 1) % R], (u + R - 1) % R, c0 + (R - 1) * STEP);
                consume(buf[u], u);
                c0 += STEP;
                if (c0 >= tok1) goto done;
            }
        }
    }
done:
#pragma unroll
    for (int g = 0; g < G; ++g) {
        l[g] = sum_xor32(sum_xor16(l[g]));
#pragma unroll
        for (int e = 0; e < EPL; ++e) o[g][e] = sum_xor32(sum_xor16(o[g][e]));
    }
}

// With WPS == 1 a workgroup holds blockDim.x / 64 waves, one per KV head
// (kv head = blockIdx.y * waves + wave), all on the same split.
template <int D, int G, typename KV, int WPS, bool BS16, int R, int NT, bool NTL = false>
__global__ __launch_bounds__(NT) void decode_attn_split_kernel(
    const float* __restrict__ Q, const KV* __restrict__ kcache, const KV* __restrict__ vcache,
    const int* __restrict__ block_table, const int* __restrict__ context_lens, int H_q,
    int H_kv, int block_size, int nbps, int num_splits, int blocks_per_split, float qscale,
    float* __restrict__ ws, float* __restrict__ O) {
    constexpr int EPL = D / 16;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int split = blockIdx.x, b = blockIdx.z;
    const int kvh = WPS == 1 ? blockIdx.y * (int)(blockDim.x >> 6) + wid : blockIdx.y;
    const int wave = WPS == 1 ? 0 : wid;
    const int grp = lane >> 4, li = lane & 15;

    const int* bt = block_table + (size_t)b * nbps;
    // Block size 16: the wave's first chunk is block split * blocks_per_split
    // + wave of the row whenever the split is not empty, so its id is loaded
    // together with the context length instead of after it (one scalar
    // round trip fewer before the first KV load; clamped into the row, and
    // unused, for an empty split).
    int pn0 = -1;
    if constexpr (BS16)
        if (nbps > 0) pn0 = bt[(int)min((long long)split * blocks_per_split + wave, (long long)nbps - 1)];
    const int ctx = context_lens[b];
    const long long span = (long long)blocks_per_split * block_size;
    const long long t0l = (long long)split * span;
    // Never walk past the table row, even if context_lens[b] breaks the
    // caller contract context_lens[b] <= max_context_len.
    const long long lim = min((long long)ctx, (long long)nbps * block_size);
    const int tok0 = (int)min(t0l, lim);
    const int tok1 = (int)min(t0l + span, lim);

    float m[G], l[G], o[G][EPL];
    split_partial<D, G, KV, WPS, BS16, R, NTL>(Q, kcache, vcache, bt, b, kvh, H_q, H_kv, block_size, tok0, tok1,
                                       wave, lane, qscale, m, l, o, pn0);
    // The partial of this split; an empty split writes o = 0, m = -inf, l = 0.
    // With a single split the partial is the result: O = o / l, written
    // directly with the merge's arithmetic (a merge of one split has weight
    // exp2(0) = 1), so no second launch is needed.
    if constexpr (WPS == 1) {
        if (grp == 0) {
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const size_t bh = (size_t)b * H_q + (size_t)kvh * G + g;
                if (num_splits == 1) {
                    const float inv = l[g] > 0.0f ? 1.0f / l[g] : 0.0f;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) O[bh * D + li * EPL + e] = o[g][e] * inv;
                    continue;
                }
                float* dst = ws + (bh * num_splits + split) * (D + 2);
#pragma unroll
                for (int e = 0; e < EPL; ++e) dst[li * EPL + e] = o[g][e];
                if (li == 0) {
                    dst[D] = m[g];
                    dst[D + 1] = l[g];
                }
            }
        }
        return;
    } else {
        split_finish_lds<D, G, WPS>(b, kvh, H_q, split, num_splits, wave, lane, m, l, o, ws, O);
    }
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ int wave_incl_scan_i(int v, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(v, o, 64);
        if (lane >= o) v += t;
    }
    return v;
}

template <int D, int G>
__device__ __forceinline__ void write_partial(float* __restrict__ dst, const float (&o)[D / 16], float m, float l,
                                              int li) {
    constexpr int EPL = D / 16;
#pragma unroll
    for (int e = 0; e < EPL; ++e) dst[li * EPL + e] = o[e];
    if (li == 0) {
        dst[D] = m;
        dst[D + 1] = l;
    }
}

// bf16 KV, d = 128: one wave's walk over chunks [tok0, tok1) of (sequence b,
// kv head kvh) for its G query heads on bf16 MFMAs (block size 16, so a
// 16-token chunk lies in one block).  The FMA form spends about 10 VALU
// operations per KV element (unpack, 2 G FMAs) and measured VALU-bound at
// bf16 (the chip issuing ~75% of its VALU rate); here:
//   * QK: S^T (16 tokens x 16 columns: query heads 0 .. G - 1, the rest
//     zero) = K_chunk (16 x 128) . Q^T on v_mfma_f32_16x16x32_bf16, K
//     straight from the cache as the A operand (lane (t, g): token t, d =
//     32 kb + 8 g .. + 8).  The scaled fp32 q is split exactly into three
//     bf16 parts (top, middle and low 8 significant bits: hi + mid + lo = q),
//     so every product is exact and only the fp32 sums round.  12 MFMAs.
//   * Softmax in that output layout: lane (j, g) holds head j's scores of
//     tokens 4 g .. 4 g + 3; a column's max and sum cross its four lanes
//     with two swaps.
//   * PV: O^T (128 x 16) += V^T . P^T on v_mfma_f32_16x16x16_bf16.  P^T is
//     the score layout itself (lane (j, g): head j, tokens 4 g .. 4 g + 3),
//     split into three bf16 parts as q; V^T comes from the chunk's V written
//     row-major into the wave's LDS tile and read with ds_read_tr16_b64: lane
//     16 g + 4 r + c supplies V[4 g + r][16 db + 4 c .. + 4], and the
//     transpose hands lane 16 g + i the d-row 16 db + i of tokens 4 g ..
//     4 g + 3 (the A operand).  24 MFMAs.
// Chunks past tok1 re-read the last token (masked to -inf, weight 0).
// Result: lane (j, g) holds m and l of head j and o[db][v] = O[head j][16 db
// + 4 g + v] (unnormalised, base-2 domain, as the partials the merge reads).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kMfTileRow = 144;  // LDS row of a V tile: 128 bf16 + 16 of padding (288 bytes)

// x = hi + mid + lo exactly, each a bf16 bit pattern (truncation keeps the
// top 8 significant bits; the remainders are exact in fp32).
__device__ __forceinline__ void split3(float x, uint32_t& h, uint32_t& m, uint32_t& l) {
    const uint32_t u = __float_as_uint(x);
    const float r = x - __uint_as_float(u & 0xFFFF0000u);
    const uint32_t ur = __float_as_uint(r);
    const float lo = r - __uint_as_float(ur & 0xFFFF0000u);
    h = u >> 16;
    m = ur >> 16;
    l = __float_as_uint(lo) >> 16;
}

template <int G>
__device__ __forceinline__ void mfma_walk_bf16(const float* __restrict__ Q, const uint16_t* kcache,
                                               const uint16_t* vcache, const int* __restrict__ bt, int b, int kvh,
                                               int H_q, int H_kv, int tok0, int tok1, int lane, float qscale,
                                               uint16_t* tile, float& m, float& l, f32x4_t (&o)[8]) {
    constexpr int D = 128;
    const int j = lane & 15, g = lane >> 4;
    // q^T parts (B operand): lane (j, g) holds q_j[32 kb + 8 g .. + 8]
    u32x4_t qp[3][4];
    {
        float qv[4][8];
        if (j < G) {
            const float4* q4 = reinterpret_cast<const float4*>(Q + ((size_t)b * H_q + (size_t)kvh * G + j) * D + 8 * g);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const float4 a = q4[8 * kb], c = q4[8 * kb + 1];
                qv[kb][0] = a.x; qv[kb][1] = a.y; qv[kb][2] = a.z; qv[kb][3] = a.w;
                qv[kb][4] = c.x; qv[kb][5] = c.y; qv[kb][6] = c.z; qv[kb][7] = c.w;
            }
        } else {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
#pragma unroll
                for (int e = 0; e < 8; ++e) qv[kb][e] = 0.0f;
        }
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t h0, m0, l0, h1, m1, l1;
                split3(qv[kb][2 * w] * qscale, h0, m0, l0);
                split3(qv[kb][2 * w + 1] * qscale, h1, m1, l1);
                qp[0][kb][w] = h0 | (h1 << 16);
                qp[1][kb][w] = m0 | (m1 << 16);
                qp[2][kb][w] = l0 | (l1 << 16);
            }
    }
    m = -INFINITY;
    l = 0.0f;
#pragma unroll
    for (int db = 0; db < 8; ++db) o[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (tok0 >= tok1) return;

    const size_t tstride = (size_t)H_kv * D;
    const uint16_t* kb0 = opaque_global(kcache) + (size_t)kvh * D + 8 * g;
    const uint16_t* vb0 = opaque_global(vcache) + (size_t)kvh * D + 8 * g;
    u32x4_t kf[2][4], vf[2][4];
    int pn = bt[tok0 >> 4];
    auto load = [&](u32x4_t (&kk)[4], u32x4_t (&vv)[4], int cs) {
        const size_t row = (size_t)pn * 16 + (min(cs + j, tok1 - 1) & 15);
        const u32x4_t* kp = reinterpret_cast<const u32x4_t*>(kb0 + row * tstride);
        const u32x4_t* vp = reinterpret_cast<const u32x4_t*>(vb0 + row * tstride);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            kk[kb] = kp[4 * kb];
            vv[kb] = vp[4 * kb];
        }
        pn = bt[min(cs + 16, tok1 - 1) >> 4];  // next chunk's block, one chunk ahead
    };
    typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
    auto consume = [&](const u32x4_t (&kk)[4], const u32x4_t (&vv)[4], int cs) {
        // four independent accumulators (one per 32-wide d block), added at the end
        f32x4_t ac[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            ac[kb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int pt = 0; pt < 3; ++pt)
                ac[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kk[kb]),
                                                                 __builtin_bit_cast(bf16x8_t, qp[pt][kb]), ac[kb], 0, 0,
                                                                 0);
        }
        const f32x4_t acc = (ac[0] + ac[1]) + (ac[2] + ac[3]);
        // V rows into the tile (row j = token cs + j), read back transposed below
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) *reinterpret_cast<u32x4_t*>(tile + j * kMfTileRow + 32 * kb + 8 * g) = vv[kb];
        float s[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) s[v] = cs + 4 * g + v < tok1 ? acc[v] : -INFINITY;
        float cm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        cm = max_xor32(max_xor16(cm));
        const float mn = fmaxf(m, cm);
        const float alpha = exp2_sm(m - mn);
        float p[4], ps = 0.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            p[v] = exp2_sm(s[v] - mn);
            ps += p[v];
        }
        ps = sum_xor32(sum_xor16(ps));
        l = fmaf(l, alpha, ps);
        m = mn;
        uint32_t ph[4], pm[4], pl[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) split3(p[v], ph[v], pm[v], pl[v]);
        i16x4_t pp[3];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            pp[0][v] = (short)ph[v];
            pp[1][v] = (short)pm[v];
            pp[2][v] = (short)pl[v];
        }
        const int r = (lane & 15) >> 2, c = lane & 3;
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            o[db] *= alpha;
            const i16x4_t vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_i16x4*)((__attribute__((address_space(3))) uint16_t*)tile + (4 * g + r) * kMfTileRow + 16 * db + 4 * c));
#pragma unroll
            for (int pt = 0; pt < 3; ++pt) o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vt, pp[pt], o[db], 0, 0, 0);
        }
    };
    int c0 = tok0;
    load(kf[0], vf[0], c0);
    bool more = true;
    while (more) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            if (more) {
                const bool nx = c0 + 16 < tok1;
                if (nx) load(kf[u ^ 1], vf[u ^ 1], c0 + 16);
                consume(kf[u], vf[u], c0);
                c0 += 16;
                more = nx;
            }
        }
    }
}

// One-wave splits with a work-balanced partition (used when a launch has
// many long splits).  With ragged context lengths a (b, split) grid leaves
// many splits short or empty, so some CUs finish early while others still
// stream full splits (measured: 67% of HBM peak for lengths U[ctx/2, ctx] at
// ctx 8192 against 71% for uniform lengths of the same total).  Here the
// batch's 16-token chunks, sequence after sequence, are cut into gridDim.x
// equal ranges of q chunks, one per workgroup; a workgroup walks the pieces of
// the sequences its range covers and writes each piece's partial into slot
// (its workgroup index - the first workgroup of that sequence).  q is at
// least ceil(nbmax / (S - 1)) chunks, so a sequence of at most nbmax chunks
// meets at most S workgroups and its pieces fit the S slots; the workgroup
// holding a sequence's last piece marks the remaining slots empty (m = -inf,
// l = 0), and an empty sequence's slots are marked by the
// workgroup its position falls in, so every slot is written exactly once and
// the merge pass is unchanged.  The partition depends only on the context
// lengths, so results do not depend on block placement.  Measured at ctx 8192
// fp32 (four-head workgroups, one per CU): 0.676 of HBM peak against 0.599
// for the (b, split) grid; bf16 at ctx 32768: 0.684 against 0.625.
template <int D, int G, typename KV, bool BS16, int R, int NT, bool KL = false, bool MF = false>
__global__ __launch_bounds__(NT) void decode_attn_balanced_kernel(
    const float* __restrict__ Q, const KV* __restrict__ kcache, const KV* __restrict__ vcache,
    const int* __restrict__ block_table, const int* __restrict__ context_lens, int B, int H_q,
    int H_kv, int block_size, int nbps, int num_splits, int nbmax, float qscale,
    float* __restrict__ ws) {
    constexpr int EPL = D / 16;
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kvh = blockIdx.y * (int)(blockDim.x >> 6) + wid;
    const int li = lane & 15, grp = lane >> 4;
    const int W = gridDim.x, w = blockIdx.x;
    // Tokens of sequence b the kernel may read: its length, clamped to the
    // table row and to the plan's nbmax chunks.
    const long long cap = min((long long)nbps * block_size, 16LL * nbmax);
    auto lim = [&](int b) { return (int)max(0LL, min((long long)context_lens[b], cap)); };

    int C = 0;
    for (int b0 = 0; b0 < B; b0 += 64) {
        const int b = b0 + lane;
        C += wave_sum_i(b < B ? (lim(b) + 15) >> 4 : 0);
    }
    const int minq = (nbmax + num_splits - 2) / (num_splits - 1);
    const int q = max(max((C + W - 1) / W, minq), 1);
    const int weff = (C + q - 1) / q;  // workgroups with chunks
    if (w >= max(weff, 1)) return;
    const int lo = w * q, hi = min(lo + q, C);

    // An empty slot needs only (m = -inf, l = 0): the merge gives it weight 0
    // and never reads its o.
    auto empty_slot = [&](int b, int slot) {
        if (lane != 0) return;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float* dst = ws + (((size_t)b * H_q + (size_t)kvh * G + g) * num_splits + slot) * (D + 2);
            dst[D] = -INFINITY;
            dst[D + 1] = 0.0f;
        }
    };

    // The range covers a contiguous run of sequences: find the first (the
    // first whose chunks end past lo, or an empty one at or past lo) with a
    // wave scan, then walk on with scalar state only.
    int bf = B, pf = C;
    int base = 0;  // chunks of the sequences before this group of 64
    for (int b0 = 0; b0 < B; b0 += 64) {
        const int b = b0 + lane;
        const int n = b < B ? (lim(b) + 15) >> 4 : 0;
        const int incl = wave_incl_scan_i(n, lane);
        const int pre = base + incl - n;
        const unsigned long long hit = __ballot(b < B && (base + incl > lo || pre >= lo));
        if (hit) {
            const int j = __builtin_ctzll(hit);
            bf = b0 + j;
            pf = __shfl(pre, j, 64);
            break;
        }
        base += __shfl(incl, 63, 64);
    }
    const bool last = w == max(weff, 1) - 1;
    int pre = __builtin_amdgcn_readfirstlane(pf);
    for (int bj = __builtin_amdgcn_readfirstlane(bf); bj < B; ++bj) {
        const int lb = lim(bj);
        const int post = pre + ((lb + 15) >> 4);
        // stop at the first sequence starting at or past hi, except the
        // empty ones at the very end, which belong to the last workgroup
        if (pre >= hi && !(last && post == pre)) break;
        if (post == pre) {  // empty sequence
            for (int slot = 0; slot < num_splits; ++slot) empty_slot(bj, slot);
        } else {
            const int seg = w - pre / q;
            const int tok0 = 16 * (max(lo, pre) - pre);
            const int tok1 = min(16 * (min(hi, post) - pre), lb);
            if constexpr (MF) {
                static_assert(D == 128 && sizeof(KV) == 2 && BS16, "bf16 MFMA walk: d = 128, block size 16");
                float mm, ll;
                f32x4_t oo[8];
                __shared__ __attribute__((aligned(16))) uint16_t vtile[NT / 64][16 * kMfTileRow];
                mfma_walk_bf16<G>(Q, reinterpret_cast<const uint16_t*>(kcache),
                                  reinterpret_cast<const uint16_t*>(vcache), block_table + (size_t)bj * nbps, bj, kvh,
                                  H_q, H_kv, tok0, tok1, lane, qscale, vtile[wid], mm, ll, oo);
                const int hj = lane & 15, gq = lane >> 4;
                if (hj < G && seg < num_splits) {
                    float* dst = ws + (((size_t)bj * H_q + (size_t)kvh * G + hj) * num_splits + seg) * (D + 2);
#pragma unroll
                    for (int db = 0; db < 8; ++db) {
                        *reinterpret_cast<float2*>(dst + 16 * db + 4 * gq) = make_float2(oo[db][0], oo[db][1]);
                        *reinterpret_cast<float2*>(dst + 16 * db + 4 * gq + 2) = make_float2(oo[db][2], oo[db][3]);
                    }
                    if (gq == 0) {
                        dst[D] = mm;
                        dst[D + 1] = ll;
                    }
                }
            } else {
                float m[G], l[G], o[G][EPL];
                if constexpr (KL)
                    split_partial_klds<G, NT / 64>(Q, kcache, vcache, block_table + (size_t)bj * nbps, bj, kvh, H_q,
                                                    H_kv, tok0, tok1, lane, qscale, m, l, o);
                else
                    split_partial<D, G, KV, 1, BS16, R>(Q, kcache, vcache, block_table + (size_t)bj * nbps, bj, kvh,
                                                     H_q, H_kv, block_size, tok0, tok1, 0, lane, qscale, m, l, o);
                if (grp == 0 && seg < num_splits) {
#pragma unroll
                    for (int g = 0; g < G; ++g)
                        write_partial<D, G>(
                            ws + (((size_t)bj * H_q + (size_t)kvh * G + g) * num_splits + seg) * (D + 2), o[g], m[g],
                            l[g], li);
                }
            }
            if (post <= hi)  // the sequence ends here: its later slots are empty
                for (int slot = seg + 1; slot < num_splits; ++slot) empty_slot(bj, slot);
        }
        pre = post;
    }
}

template <int D>
__global__ __launch_bounds__(256) void decode_attn_merge_kernel(int BH, int num_splits,
                                                                const float* __restrict__ ws,
                                                                float* __restrict__ O) {
    const int bh = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (bh >= BH) return;
    merge_head<D>(ws + (size_t)bh * num_splits * (D + 2), num_splits, O + (size_t)bh * D,
                  threadIdx.x & 63);
}

// Splits of at least kWaveSplitTokens tokens get one wave each (16+ chunks
// per wave keep its loads streaming) when there are at least kWaveSplitUnits
// (b, kv head, split) units to fill the GPU; otherwise four waves share a
// split, which would else be walked one chunk latency at a time (a handful of
// units, as in the GPT-2 decode step, needs that parallelism).
constexpr long long kWaveSplitTokens = 256;
constexpr long long kWaveSplitUnits = 1024;
// Batches up to this size use the balanced partition for one-wave splits
// (every workgroup scans the context lengths twice).
constexpr int kBalancedMaxB = 4096;
// At most this many (kv head, split) units per sequence count as few.
constexpr long long kFewUnits = 64;

// Workgroups of `threads` threads of kernel f resident per CU (at least 1),
// looked up once per kernel.
int resident_per_cu(const void* f, int threads) {
    static std::mutex mu;
    static std::map<std::pair<const void*, int>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find({f, threads});
    if (it != cache.end()) return it->second;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, threads, 0) != hipSuccess || n < 1) n = 1;
    cache[{f, threads}] = n;
    return n;
}

// Bytes of K and V a launch may read (every sequence at the plan's longest
// context), and the size past which the cache is streamed non-temporally.
long long kv_stream_bytes(const DecodeArgs& a) {
    const long long ctx = std::min<long long>((long long)a.num_splits * a.blocks_per_split * a.block_size,
                                              (long long)a.num_blocks_per_seq * a.block_size);
    return (long long)a.B * ctx * a.H_kv * a.d * 2 * (a.kv_dtype == IE_KV_BF16 ? 2 : 4);
}
constexpr long long kStreamKvBytes = 32ll << 20;

template <int D, int G, typename KV>
void launch_split(const DecodeArgs& a, hipStream_t s) {
    const float qscale = (1.0f / sqrtf((float)D)) * 1.4426950408889634f;
    const bool wave = (long long)a.blocks_per_split * a.block_size >= kWaveSplitTokens &&
                      (long long)a.num_splits * a.H_kv * a.B >= kWaveSplitUnits;
    // One-wave splits: the waves of up to 8 KV heads of the same (b, split)
    // share a workgroup, so the heads' slices of each block (contiguous in
    // the cache row) are read together; measured 5% faster than one wave per
    // workgroup at ctx 8192.
    constexpr int HWMAX = wave_heads<D, KV, G>();
    constexpr int RW = wave_ring<D, KV, G>();
    constexpr int NTW = 64 * HWMAX;
    int hw = 1;
    if (wave)
        for (int c = HWMAX; c >= 1; c >>= 1)
            if (a.H_kv % c == 0) {
                hw = c;
                break;
            }
    const dim3 grid(a.num_splits, a.H_kv / hw, a.B);
    // Scalar block ids measured 12% faster for bf16 KV at ctx 8192 and 1%
    // slower for fp32 one-wave splits (where the per-lane table loads already
    // sit behind the chunk's own KV loads); fp32 long splits keep those,
    // except at G = 8, whose walk is VALU-bound and gains 5% without the
    // per-lane table loads and block arithmetic.
    const bool bs16 = a.block_size == 16 && !(wave && sizeof(KV) == 4 && G < 8);
    if (wave && a.num_splits >= 2 && a.B <= kBalancedMaxB) {
        // As many workgroups as are resident at once (occupancy x CUs), so the
        // equal ranges all run in one round.
        // fp32 d = 128 with block size 16 lands K in LDS (G = 8 has no
        // register room for the ring beside its 8 heads' q and o).
        constexpr bool KL = D == 128 && sizeof(KV) == 4 && G <= 4;
        // bf16 d = 128, G >= 4, block size 16: the MFMA walk (an fp32 form on
        // v_mfma_f32_16x16x4_f32 measured 0.35 against 0.61 of HBM peak at
        // G = 8, so fp32 keeps the FMA walk)
        constexpr bool MF = D == 128 && sizeof(KV) == 2 && G >= 4;
        auto* kb = (KL && a.block_size == 16)   ? decode_attn_balanced_kernel<D, G, KV, true, RW, NTW, KL>
                   : (MF && a.block_size == 16) ? decode_attn_balanced_kernel<D, G, KV, true, RW, NTW, false, MF>
                   : bs16                       ? decode_attn_balanced_kernel<D, G, KV, true, RW, NTW>
                                                : decode_attn_balanced_kernel<D, G, KV, false, RW, NTW>;
        const int gy = a.H_kv / hw;
        const unsigned W = (unsigned)std::max(1, resident_per_cu((const void*)kb, 64 * hw) * num_cus() / gy);
        // chunks the plan covers (S x blocks per split, at least max_context_len)
        const int nbmax = (int)std::min<long long>(((long long)a.num_splits * a.blocks_per_split * a.block_size + 15) / 16,
                                                   ((long long)a.num_blocks_per_seq * a.block_size + 15) / 16);
        kb<<<dim3(W, gy), 64 * hw, 0, s>>>(a.Q, static_cast<const KV*>(a.k_cache), static_cast<const KV*>(a.v_cache),
                                           a.block_table, a.context_lens, a.B, a.H_q, a.H_kv, a.block_size,
                                           a.num_blocks_per_seq, a.num_splits, nbmax, qscale, a.workspace);
        return;
    }
    // Few units per sequence (GPT-2: 12 heads, one to three splits): 8 waves
    // share each split, so a wave walks half as many chunks one after
    // another; measured +2.4% decode tok/s at batch 1 (16 waves: +1%) and
    // +1.1% at batch 16, where it fits without spilling (G <= 4).  The count
    // is decided per sequence, not per batch, so a sequence's output has the
    // same bits at every batch size (the engine's batch invariance).
    constexpr int WF = 8;
    constexpr bool WF_FITS = G <= 4;
    const bool few = WF_FITS && !wave && (long long)a.num_splits * a.H_kv <= kFewUnits;
    // Multi-wave splits stream the cache with non-temporal loads when the
    // launch reads more of it than the caches would keep (kv_stream_bytes):
    // cfg3 (50 MB) 15.3 -> 13.9 us; one-wave splits measured slightly slower
    // with them and keep plain loads.
    const bool ntl = kv_stream_bytes(a) > kStreamKvBytes;
    using KernelT = decltype(&decode_attn_split_kernel<D, G, KV, 4, true, 2, 256>);
    KernelT k = wave ? (bs16 ? decode_attn_split_kernel<D, G, KV, 1, true, RW, NTW>
                             : decode_attn_split_kernel<D, G, KV, 1, false, RW, NTW>)
                : ntl ? (bs16 ? decode_attn_split_kernel<D, G, KV, 4, true, 2, 256, true>
                              : decode_attn_split_kernel<D, G, KV, 4, false, 2, 256, true>)
                      : (bs16 ? decode_attn_split_kernel<D, G, KV, 4, true, 2, 256>
                              : decode_attn_split_kernel<D, G, KV, 4, false, 2, 256>);
    if constexpr (WF_FITS)
        if (few)
            k = ntl ? (bs16 ? decode_attn_split_kernel<D, G, KV, WF, true, 2, 64 * WF, true>
                            : decode_attn_split_kernel<D, G, KV, WF, false, 2, 64 * WF, true>)
                    : (bs16 ? decode_attn_split_kernel<D, G, KV, WF, true, 2, 64 * WF>
                            : decode_attn_split_kernel<D, G, KV, WF, false, 2, 64 * WF>);
    k<<<grid, wave ? 64 * hw : few ? 64 * WF : 256, 0, s>>>(
        a.Q, static_cast<const KV*>(a.k_cache), static_cast<const KV*>(a.v_cache),
        a.block_table, a.context_lens, a.H_q, a.H_kv, a.block_size, a.num_blocks_per_seq,
        a.num_splits, a.blocks_per_split, qscale, a.workspace, a.O);
}

template <int D, typename KV>
void launch_g(const DecodeArgs& a, hipStream_t s) {
    switch (a.H_q / a.H_kv) {
        case 1: launch_split<D, 1, KV>(a, s); break;
        case 2: launch_split<D, 2, KV>(a, s); break;
        case 4: launch_split<D, 4, KV>(a, s); break;
        default: launch_split<D, 8, KV>(a, s); break;
    }
}

template <int D>
void launch_d(const DecodeArgs& a, hipStream_t s) {
    if (a.kv_dtype == IE_KV_BF16)
        launch_g<D, uint16_t>(a, s);
    else
        launch_g<D, float>(a, s);
    if (a.num_splits == 1) return;  // the split kernel wrote O
    const int BH = a.B * a.H_q;
    decode_attn_merge_kernel<D><<<(BH + 3) / 4, 256, 0, s>>>(BH, a.num_splits, a.workspace, a.O);
}

}  // namespace

void launch_decode_attn(const DecodeArgs& a, hipStream_t s) {
    if (a.B == 0) return;
    if (a.d == 64)
        launch_d<64>(a, s);
    else
        launch_d<128>(a, s);
}

}  // namespace ie
