// attn_split.h — the per-split body of the paged decode attention, shared
// by decode_attn.hip (the standalone split kernels) and qkv_attn.hip (the
// engine's fused QKV projection + attention), so both give the same bits for
// the same split plan.  See decode_attn.hip for the layout.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

#include "device_util.h"

namespace ie {
namespace {

// Raw K/V words of one lane's d/16-element slice of one token; bf16 stays
// packed until use so a prefetched chunk costs half the registers.
template <int EPL, typename KV>
struct Slice {
    static constexpr int WORDS = EPL * (int)sizeof(KV) / 4;
    uint32_t w[WORDS];
};

// NTL: non-temporal loads (for a cache stream larger than the caches keep).
template <int EPL, typename KV, bool NTL = false>
__device__ __forceinline__ void load_raw(const KV* __restrict__ p, Slice<EPL, KV>& s) {
    constexpr int W = Slice<EPL, KV>::WORDS;
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
    if constexpr (W % 4 == 0) {
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const u32x4v* a = reinterpret_cast<const u32x4v*>(p) + i;
            const u32x4v v = NTL ? __builtin_nontemporal_load(a) : *a;
            s.w[4 * i + 0] = v.x;
            s.w[4 * i + 1] = v.y;
            s.w[4 * i + 2] = v.z;
            s.w[4 * i + 3] = v.w;
        }
    } else {
        static_assert(W == 2, "slice width");
        const u32x2v* a = reinterpret_cast<const u32x2v*>(p);
        const u32x2v v = NTL ? __builtin_nontemporal_load(a) : *a;
        s.w[0] = v.x;
        s.w[1] = v.y;
    }
}

template <int EPL, typename KV>
__device__ __forceinline__ float elem(const Slice<EPL, KV>& s, int e) {
    if constexpr (sizeof(KV) == 4) {
        return __builtin_bit_cast(float, s.w[e]);
    } else {
        const uint32_t w = s.w[e >> 1];
        return __builtin_bit_cast(float, (e & 1) ? (w & 0xffff0000u) : (w << 16));
    }
}

template <int EPL>
__device__ __forceinline__ void load_q(const float* __restrict__ p, float (&out)[EPL]) {
#pragma unroll
    for (int i = 0; i < EPL / 4; ++i) {
        const float4 v = reinterpret_cast<const float4*>(p)[i];
        out[4 * i + 0] = v.x;
        out[4 * i + 1] = v.y;
        out[4 * i + 2] = v.z;
        out[4 * i + 3] = v.w;
    }
}

// A chunk of 4T tokens: lane row grp holds tokens c0 + 4j + grp, j < T.
template <int D, typename KV, int T>
struct Chunk {
    static constexpr int EPL = D / 16;
    Slice<EPL, KV> k[T], v[T];
    bool valid[T];
};

// Loads this lane's slices of tokens c0 + 4j + grp (j < T) of a chunk.
template <int D, typename KV, int T, bool NTL = false>
__device__ __forceinline__ void load_chunk(Chunk<D, KV, T>& c, int c0, int grp, int tok1,
                                           const int* __restrict__ bt, int block_size,
                                           size_t tok_stride, const KV* kbase, const KV* vbase) {
// Branch-free: positions past tok1 re-read token tok1-1 (a cache hit) and are
// masked by `valid`, so the loads never sit in divergent control flow and the
// compiler can keep the next chunk in flight across the current one.
#pragma unroll
    for (int j = 0; j < T; ++j) {
        const int pos = c0 + 4 * j + grp;
        c.valid[j] = pos < tok1;
        const int pc = min(pos, tok1 - 1);
        const int blk = pc / block_size;
        const size_t row = (size_t)bt[blk] * block_size + (pc - blk * block_size);
        load_raw<D / 16, KV, NTL>(kbase + row * tok_stride, c.k[j]);
        load_raw<D / 16, KV, NTL>(vbase + row * tok_stride, c.v[j]);
    }
}

// Block size 16: the chunk's tokens (c0 a multiple of 4T) lie in blocks
// phys[0], phys[1], ... (16 tokens each), the same for every lane.
template <int D, typename KV, int T, bool NTL = false>
__device__ __forceinline__ void load_chunk16(Chunk<D, KV, T>& c, int c0, int grp, int tok1,
                                             const int (&phys)[(T + 3) / 4], size_t tok_stride,
                                             const KV* kbase, const KV* vbase) {
#pragma unroll
    for (int j = 0; j < T; ++j) {
        const int pos = c0 + 4 * j + grp;
        c.valid[j] = pos < tok1;
        const int pc = min(pos, tok1 - 1);
        const size_t row = (size_t)phys[j / 4] * 16 + (pc & 15);
        load_raw<D / 16, KV, NTL>(kbase + row * tok_stride, c.k[j]);
        load_raw<D / 16, KV, NTL>(vbase + row * tok_stride, c.v[j]);
    }
}

template <int D, int G, typename KV, int T>
__device__ __forceinline__ void consume_chunk(const Chunk<D, KV, T>& c, const float (&q)[G][D / 16],
                                              float (&m)[G], float (&l)[G], float (&o)[G][D / 16]) {
    constexpr int EPL = D / 16;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float s[T];
#pragma unroll
        for (int j = 0; j < T; ++j) {
            float dot = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) dot = fmaf(q[g][e], elem(c.k[j], e), dot);
            dot = row16_sum(dot);
            s[j] = c.valid[j] ? dot : -INFINITY;
        }
        float cm = s[0];
#pragma unroll
        for (int j = 1; j < T; ++j) cm = fmaxf(cm, s[j]);
        cm = max_xor32(max_xor16(cm));
        const float mn = fmaxf(m[g], cm);
        const float alpha = exp2_sm(m[g] - mn);
        float p[T], psum = 0.0f;
#pragma unroll
        for (int j = 0; j < T; ++j) {
            p[j] = exp2_sm(s[j] - mn);
            psum += p[j];
        }
        l[g] = fmaf(l[g], alpha, psum);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            float acc = o[g][e] * alpha;
#pragma unroll
            for (int j = 0; j < T; ++j) acc = fmaf(p[j], elem(c.v[j], e), acc);
            o[g][e] = acc;
        }
        m[g] = mn;
    }
}

// WPS waves per split: 4 for short splits (the waves take the split's chunks
// round-robin and merge in LDS), 1 for long ones (no LDS merge, no barrier).
// BS16: block_size == 16 (the engine's and the reference's), see below.
// Partial softmax state (m, l, o) over tokens [tok0, tok1) of sequence b for
// the G query heads of KV head kvh; the split's WPS waves take its 16-token
// chunks round-robin (this one is `wave`).  bt is the sequence's block-table
// row.  On return every lane holds the wave's totals (o summed over the four
// lane rows).
//
// SplitWalk holds a wave's walk in two parts: begin() issues the block-table
// lookups and the first R - 1 chunks' loads, run() consumes the chunks with
// the query slice it is given.  split_partial calls them back to back; the
// engine's fused QKV + attention kernel issues begin() before its projection,
// so those loads are in flight while the projection runs, and hands run() a
// patch that substitutes the token it has just appended (held in LDS) for
// that token's cache row, which the early loads may have read before it was
// written.  The arithmetic and its order are the same either way.
template <int D, int G, typename KV, int WPS, bool BS16, int R, bool NTL = false>
struct SplitWalk {
    static constexpr int EPL = D / 16;
    // Chunk rows and ring depth: R chunks of 4T tokens cycle through the
    // registers, R - 1 of them in flight while one is computed.
    static constexpr int T = 4;            // lane rows hold T tokens each
    static constexpr int CT = 4 * T;       // tokens per chunk
    static constexpr int STEP = CT * WPS;  // tokens per round of the split's waves
    static constexpr int NPH = (T + 3) / 4;  // blocks per chunk
    // d = 128 bf16 rings keep their loads in place (measured 2-5% faster at
    // ctx 4096-32768); fp32 rings need the register room sinking gives them
    // and d = 64 bf16 measured 9% slower.
    static constexpr bool OPQ = sizeof(KV) == 2 && D == 128;

    Chunk<D, KV, T> buf[R];
    int pn[NPH];
    int c0, tok1, grp, block_size;
    size_t tok_stride;
    const KV* kbase;
    const KV* vbase;
    const int* bt;
    bool any;

    // With block size 16 a chunk lies in one block, so its physical block id
    // is wave-uniform: it comes from a scalar load issued one chunk ahead
    // (pn), which does not wait behind the in-flight KV loads as a vector
    // load would (they retire in issue order), so the next KV loads go out as
    // soon as a chunk is done.  Chunks past the end re-read the last token
    // (masked), so every step issues the same loads and the ring needs no
    // branches.
    __device__ __forceinline__ int phys(int cs) const { return bt[min(cs, tok1 - 1) >> 4]; }
    __device__ __forceinline__ void prefetch(int cs) {
#pragma unroll
        for (int k = 0; k < NPH; ++k) pn[k] = phys(cs + 16 * k);
    }
    __device__ __forceinline__ void next(Chunk<D, KV, T>& c, int cs) {
        if constexpr (BS16) {
            load_chunk16<D, KV, T, NTL>(c, cs, grp, tok1, pn, tok_stride, kbase, vbase);
            prefetch(cs + STEP);
        } else {
            load_chunk<D, KV, T, NTL>(c, cs, grp, tok1, bt, block_size, tok_stride, kbase, vbase);
        }
    }

    // pn0 >= 0: the physical block of the wave's first chunk, already loaded
    // by the caller (block size 16 only); otherwise begin() looks it up.
    __device__ __forceinline__ void begin(const KV* __restrict__ kcache, const KV* __restrict__ vcache,
                                          const int* __restrict__ bt_row, int kvh, int H_kv, int bs, int tok0,
                                          int tok1_, int wave, int lane, int pn0 = -1) {
        const int li = lane & 15;
        grp = lane >> 4;
        tok1 = tok1_;
        block_size = bs;
        bt = bt_row;
        tok_stride = (size_t)H_kv * D;
        kbase = (OPQ ? opaque_global(kcache) : kcache) + (size_t)kvh * D + li * EPL;
        vbase = (OPQ ? opaque_global(vcache) : vcache) + (size_t)kvh * D + li * EPL;
        c0 = tok0 + wave * CT;
        any = c0 < tok1;
        if constexpr (BS16) {
            static_assert(NPH == 1, "a chunk lies in one block");
            // An empty walk reads no table entry: with tok1 == 0 the clamp in
            // phys() would index bt[-1], and an empty row may have no entries.
            if (pn0 >= 0)
                pn[0] = pn0;
            else if (any)
                prefetch(c0);
            else
                pn[0] = 0;
        }
        if (any) {
#pragma unroll
            for (int p = 0; p < R - 1; ++p) next(buf[p], c0 + p * STEP);
        }
    }

    // q: this lane's slice of the G (scaled) query rows.  patch(chunk, cs)
    // may rewrite a chunk starting at token cs before it is consumed.
    template <class Patch>
    __device__ __forceinline__ void run(const float (&q)[G][EPL], float (&m)[G], float (&l)[G],
                                        float (&o)[G][EPL], Patch&& patch) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            m[g] = -INFINITY;
            l[g] = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) o[g][e] = 0.0f;
        }
        // Each step issues the chunk R - 1 rounds ahead into the buffer
        // consumed last, then consumes the current one.
        if (any) {
            bool more = true;
            while (more) {
#pragma unroll
                for (int u = 0; u < R; ++u) {
                    if (more) {
                        next(buf[(u + R - 1) % R], c0 + (R - 1) * STEP);
                        patch(buf[u], c0);
                        consume_chunk<D, G, KV, T>(buf[u], q, m, l, o);
                        c0 += STEP;
                        more = c0 < tok1;
                    }
                }
            }
        }
        // The four lane rows share the wave's running max: plain sums merge
        // them.
#pragma unroll
        for (int g = 0; g < G; ++g) {
            l[g] = sum_xor32(sum_xor16(l[g]));
#pragma unroll
            for (int e = 0; e < EPL; ++e) o[g][e] = sum_xor32(sum_xor16(o[g][e]));
        }
    }
};

template <int D, int G, typename KV, int WPS, bool BS16, int R, bool NTL = false>
__device__ __forceinline__ void split_partial(const float* __restrict__ Q, const KV* __restrict__ kcache,
                                              const KV* __restrict__ vcache, const int* __restrict__ bt,
                                              int b, int kvh, int H_q, int H_kv, int block_size, int tok0,
                                              int tok1, int wave, int lane, float qscale, float (&m)[G],
                                              float (&l)[G], float (&o)[G][D / 16], int pn0 = -1) {
    constexpr int EPL = D / 16;
    const int li = lane & 15;
    SplitWalk<D, G, KV, WPS, BS16, R, NTL> w;
    w.begin(kcache, vcache, bt, kvh, H_kv, block_size, tok0, tok1, wave, lane, pn0);
    float q[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        load_q<EPL>(Q + ((size_t)b * H_q + (size_t)kvh * G + g) * D + li * EPL, q[g]);
#pragma unroll
        for (int e = 0; e < EPL; ++e) q[g][e] *= qscale;
    }
    w.run(q, m, l, o, [](Chunk<D, KV, 4>&, int) {});
}

// End of a split shared by WPS > 1 waves: the waves' partials merged in
// LDS (weights exp2(m_w - max)), then O = o / l written directly when the
// split is the only one (num_splits == 1), or the split's (o, m, l) partial
// written to ws otherwise.  Every thread of the workgroup calls it.
template <int D, int G, int WPS>
__device__ __forceinline__ void split_finish_lds(int b, int kvh, int H_q, int split, int num_splits, int wave,
                                                 int lane, const float (&m)[G], const float (&l)[G],
                                                 const float (&o)[G][D / 16], float* __restrict__ ws,
                                                 float* __restrict__ O) {
    constexpr int EPL = D / 16;
    const int grp = lane >> 4, li = lane & 15;
    __shared__ float sm_m[WPS][G], sm_l[WPS][G];
    __shared__ float sm_o[WPS][G][D];
    if (grp == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < EPL; ++e) sm_o[wave][g][li * EPL + e] = o[g][e];
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            sm_m[wave][g] = m[g];
            sm_l[wave][g] = l[g];
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < G * D; idx += 64 * WPS) {
        const int g = idx / D, dd = idx - (idx / D) * D;
        float mx = sm_m[0][g];
#pragma unroll
        for (int w = 1; w < WPS; ++w) mx = fmaxf(mx, sm_m[w][g]);
        float ov = 0.0f, lv = 0.0f;
        if (mx != -INFINITY) {
#pragma unroll
            for (int w = 0; w < WPS; ++w) {
                const float f = exp2_sm(sm_m[w][g] - mx);
                ov = fmaf(sm_o[w][g][dd], f, ov);
                lv = fmaf(sm_l[w][g], f, lv);
            }
        }
        const size_t bh = (size_t)b * H_q + (size_t)kvh * G + g;
        if (num_splits == 1) {
            O[bh * D + dd] = ov * (lv > 0.0f ? 1.0f / lv : 0.0f);
            continue;
        }
        float* dst = ws + (bh * num_splits + split) * (D + 2);
        dst[dd] = ov;
        if (dd == 0) {
            dst[D] = mx;
            dst[D + 1] = lv;
        }
    }
}

}  // namespace
}  // namespace ie
