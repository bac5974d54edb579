// prefill_attn.hip — causal attention over a prompt chunk, for gfx950.
//
// Computes what the reference's K10 FlashAttention-2 forward computes
// (kernels/flash_attention/10_flash_attn_v2.cu:27-236; called for a fresh
// prompt at src/gpt2_engine.cu:484-493): for every sequence b, head h and query
// t, O = softmax(q . K^T / sqrt(d)) V over the keys at positions <= the
// query's position (all keys when not causal).  Two operand layouts:
//   * paged (the engine's prefill): Q and O token-major [B, P, H_q, d] (the
//     QKV projection's own layout, so no transposes), K/V read back from the
//     paged cache [phys][block_size][H_kv][d] (fp32 or bf16) through the block
//     table after the chunk's K/V were appended; query t of a sequence sits at
//     position start + t, so a chunk continuing an existing context sees the
//     earlier tokens too;
//   * contiguous [B, H, N, d] fp32 for Q, K, V, O (the reference's K10
//     signature, run_flash_attn_v2).
//
// MI355X layout (one workgroup of four waves per (query tile, h, b)):
//   * a workgroup owns 16 consecutive queries of one (b, h); its four waves
//     take the 16-token KV chunks up to the tile's causal limit round-robin,
//     each keeping its own running (m, l, o), and merge them in LDS at the end;
//   * the grid is one-dimensional, tile rank major: workgroup u takes pair
//     p = u % (H_q B) and tile rank r = u / (H_q B) (rank 0 = the last,
//     longest tile), so the longest tiles (causal triangles) are dispatched
//     first.  Workgroups go to the XCDs round-robin, so with H_q B a multiple
//     of 8 all tiles of one (b, h) run on one XCD (its K/V fetched into one
//     L2) and every XCD gets the same mix of tile lengths.  (With the tile
//     index fastest, XCD x took tile rank x of every pair: at 8 tiles XCD 0
//     held all the longest tiles, and each pair's K/V went to eight L2s);
//   * S^T = K Q^T and O^T += V^T P^T run on v_mfma_f32_16x16x4_f32.  Lane l
//     (i = l % 16, g = l / 16) holds, for query i of the tile:
//       - q: elements d/4*g .. d/4*g + d/4 - 1 (the B operand: MFMA step s
//         reads element d/4*g + s, and the K operand (A) of key i uses the
//         same element map, so the K-sum is exact in a permuted order);
//       - scores of keys 4g .. 4g+3 of the chunk (the MFMA result layout),
//         which are directly the B operand P^T of the P.V product (step s
//         takes key 4g + s);
//       - output elements d/16*(4g + v) + t (t = output tile, v = result row);
//   * the per-query max and sum run over the four lanes i, i+16, i+32, i+48
//     (two cross-row swaps), so a wave rescales once per 16 keys;
//   * scores are pre-multiplied by log2(e)/sqrt(d) (folded into q), so the
//     softmax uses the hardware exp2 (the decode kernel does the same);
//   * K/V of the next chunk are loaded while the current one is computed;
//     with block size 16 a chunk is one block and its physical id comes from a
//     wave-uniform scalar load.
#include <cmath>

#include "device_util.h"
#include "ie_internal.h"

namespace ie {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kQTile = 16;  // queries per workgroup
constexpr int kWaves = 4;

template <int W>
__device__ __forceinline__ void load_words(const void* p, uint32_t (&w)[W]) {
    if constexpr (W % 4 == 0) {
#pragma unroll
        for (int i = 0; i < W / 4; ++i) {
            const uint4 v = reinterpret_cast<const uint4*>(p)[i];
            w[4 * i] = v.x;
            w[4 * i + 1] = v.y;
            w[4 * i + 2] = v.z;
            w[4 * i + 3] = v.w;
        }
    } else if constexpr (W == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        w[0] = v.x;
        w[1] = v.y;
    } else {
        static_assert(W == 1, "slice width");
        w[0] = *reinterpret_cast<const uint32_t*>(p);
    }
}

// Element j of a lane's raw K or V slice.
template <typename KV, int W>
__device__ __forceinline__ float elem(const uint32_t (&w)[W], int j) {
    if constexpr (sizeof(KV) == 4) {
        return __builtin_bit_cast(float, w[j]);
    } else {
        const uint32_t x = w[j >> 1];
        return __builtin_bit_cast(float, (j & 1) ? (x & 0xffff0000u) : (x << 16));
    }
}

// A lane's share of one 16-token chunk: d/4 elements of key i's K, and
// d/16 elements (from d/16 * i) of each of the keys 4g .. 4g+3's V.
template <int D, typename KV>
struct Chunk {
    static constexpr int KW = D / 4 * (int)sizeof(KV) / 4;
    static constexpr int VW = D / 16 * (int)sizeof(KV) / 4;
    uint32_t k[KW];
    uint32_t v[4][VW];
};

// Where token `pos` of the current (b, kv head) lives, in elements from the
// head's base pointer.
//   LAYOUT 0, BS16: paged with block size 16; `phys` is the chunk's block.
//   LAYOUT 0:       paged, any block size (per-lane table lookup).
//   LAYOUT 1:       contiguous rows.
template <int LAYOUT, bool BS16>
struct TokenMap {
    const int* bt;
    int block_size;
    size_t stride;  // elements between consecutive token rows of one head
    __device__ __forceinline__ size_t off(int pos, int phys) const {
        if constexpr (LAYOUT == 1) {
            return (size_t)pos * stride;
        } else if constexpr (BS16) {
            return ((size_t)phys * 16 + (pos & 15)) * stride;
        } else {
            const int blk = pos / block_size;
            return ((size_t)bt[blk] * block_size + (pos - blk * block_size)) * stride;
        }
    }
};

template <int D, typename KV, int LAYOUT, bool BS16>
__device__ __forceinline__ void load_chunk(Chunk<D, KV>& c, int c0, int kend, int i, int g, int phys,
                                           const TokenMap<LAYOUT, BS16>& map, const KV* kbase,
                                           const KV* vbase) {
    const int kp = min(c0 + i, kend - 1);
    load_words(kbase + map.off(kp, phys) + (D / 4) * g, c.k);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int vp = min(c0 + 4 * g + s, kend - 1);
        load_words(vbase + map.off(vp, phys) + (D / 16) * i, c.v[s]);
    }
}

// One chunk: scores, masked online softmax, P.V.  qpos = this lane's query
// position (keys > qpos are masked when causal), kend = keys in range.
template <int D, typename KV>
__device__ __forceinline__ void consume(const Chunk<D, KV>& c, int c0, int g, const float (&q)[D / 4],
                                        int klim, float& m, float& l, f32x4 (&o)[D / 16]) {
    f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < D / 4; ++e)
        s = __builtin_amdgcn_mfma_f32_16x16x4f32(elem<KV>(c.k, e), q[e], s, 0, 0, 0);
    float cm = -INFINITY;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        if (c0 + 4 * g + v >= klim) s[v] = -INFINITY;
        cm = fmaxf(cm, s[v]);
    }
    cm = max_xor32(max_xor16(cm));
    const float mn = fmaxf(m, cm);
    const float mu = mn == -INFINITY ? 0.0f : mn;  // no key yet: keep o, l at 0
    const float alpha = exp2_sm(m - mu);
    float p[4], ls = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        p[v] = exp2_sm(s[v] - mu);
        ls += p[v];
    }
    ls = sum_xor32(sum_xor16(ls));
    l = fmaf(l, alpha, ls);
    m = mn;
#pragma unroll
    for (int t = 0; t < D / 16; ++t) {
        o[t] *= alpha;
#pragma unroll
        for (int sv = 0; sv < 4; ++sv)
            o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(elem<KV>(c.v[sv], t), p[sv], o[t], 0, 0, 0);
    }
}

// LAYOUT 0: Q/O [B, P, H_q, D], keys = start + P cached tokens.
// LAYOUT 1: Q/K/V/O [B, H, P, D], keys = P, start = 0.
template <int D, typename KV, int LAYOUT, bool BS16>
__global__ __launch_bounds__(256) void prefill_attn_kernel(
    const float* __restrict__ Q, const KV* __restrict__ kcache, const KV* __restrict__ vcache,
    const int* __restrict__ block_table, int nbps, int block_size, int P, int H_q, int H_kv,
    int start, int causal, float qscale, float* __restrict__ O) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = lane & 15, g = lane >> 4;
    const int ntiles = (P + kQTile - 1) / kQTile;
    const int pairs = (int)(gridDim.x / (unsigned)ntiles);  // H_q B
    const int r = (int)blockIdx.x / pairs, pr = (int)blockIdx.x - r * pairs;
    const int qt = ntiles - 1 - r;  // longest (last) tiles first
    const int h = pr % H_q, b = pr / H_q;
    const int kvh = h / (H_q / H_kv);
    const int q0 = qt * kQTile;
    const int qlast = min(q0 + kQTile - 1, P - 1);
    const int nkeys = start + P;
    // Keys this tile needs, and this lane's own limit.
    const int kend = causal ? min(start + qlast + 1, nkeys) : nkeys;
    const int klim = causal ? min(start + q0 + i + 1, kend) : kend;
    const int qi = min(q0 + i, P - 1);

    size_t qrow;
    TokenMap<LAYOUT, BS16> map{};
    const KV* kbase;
    const KV* vbase;
    if constexpr (LAYOUT == 0) {
        qrow = (((size_t)b * P + qi) * H_q + h) * D;
        map.bt = block_table + (size_t)b * nbps;
        map.block_size = block_size;
        map.stride = (size_t)H_kv * D;
        kbase = kcache + (size_t)kvh * D;
        vbase = vcache + (size_t)kvh * D;
    } else {
        qrow = (((size_t)b * H_q + h) * P + qi) * D;
        map.stride = D;
        kbase = kcache + ((size_t)b * H_kv + kvh) * P * D;
        vbase = vcache + ((size_t)b * H_kv + kvh) * P * D;
    }

    float q[D / 4];
#pragma unroll
    for (int e = 0; e < D / 4; e += 4) {
        const float4 v = *reinterpret_cast<const float4*>(Q + qrow + (D / 4) * g + e);
        q[e] = v.x * qscale;
        q[e + 1] = v.y * qscale;
        q[e + 2] = v.z * qscale;
        q[e + 3] = v.w * qscale;
    }

    float m = -INFINITY, l = 0.0f;
    f32x4 o[D / 16];
#pragma unroll
    for (int t = 0; t < D / 16; ++t) o[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    constexpr int STEP = 16 * kWaves;
    auto phys = [&](int cs) {
        if constexpr (LAYOUT == 0 && BS16) return map.bt[min(cs, kend - 1) >> 4];
        else return 0;
    };
    Chunk<D, KV> ca, cb;
    int c0 = 16 * wave;
    int pn = 0;
    if (c0 < kend) {
        load_chunk(ca, c0, kend, i, g, phys(c0), map, kbase, vbase);
        pn = phys(c0 + STEP);
    }
    auto next = [&](Chunk<D, KV>& c, int cs) {
        load_chunk(c, cs, kend, i, g, pn, map, kbase, vbase);
        pn = phys(cs + STEP);
    };
    // Ping-pong: chunk c0 + STEP (clamped past the end) is always in flight
    // while chunk c0 is computed.
    while (c0 < kend) {
        next(cb, c0 + STEP);
        consume(ca, c0, g, q, klim, m, l, o);
        c0 += STEP;
        if (c0 >= kend) break;
        next(ca, c0 + STEP);
        consume(cb, c0, g, q, klim, m, l, o);
        c0 += STEP;
    }

    // Merge the four waves' partial softmax states in LDS.
    __shared__ float sm_o[kWaves][kQTile][D + 4];
    __shared__ float sm_m[kWaves][kQTile], sm_l[kWaves][kQTile];
#pragma unroll
    for (int t = 0; t < D / 16; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v) sm_o[wave][i][(D / 16) * (4 * g + v) + t] = o[t][v];
    if (g == 0) {
        sm_m[wave][i] = m;
        sm_l[wave][i] = l;
    }
    __syncthreads();

    constexpr int PER = kQTile * D / 256;  // outputs per thread (4 or 8)
    const int qq = threadIdx.x / 16, col = (threadIdx.x % 16) * PER;
    if (q0 + qq >= P) return;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, sm_m[w][qq]);
    float f[kWaves], L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        f[w] = sm_m[w][qq] == -INFINITY ? 0.0f : exp2_sm(sm_m[w][qq] - mx);
        L = fmaf(f[w], sm_l[w][qq], L);
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    float out[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        float acc = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) acc = fmaf(f[w], sm_o[w][qq][col + e], acc);
        out[e] = acc * inv;
    }
    const int qo = q0 + qq;
    float* orow = LAYOUT == 0 ? O + (((size_t)b * P + qo) * H_q + h) * D
                              : O + (((size_t)b * H_q + h) * P + qo) * D;
#pragma unroll
    for (int e = 0; e < PER; e += 4)
        *reinterpret_cast<float4*>(orow + col + e) = make_float4(out[e], out[e + 1], out[e + 2], out[e + 3]);
}

template <int D, typename KV, int LAYOUT, bool BS16>
void launch_t(const PrefillArgs& a, hipStream_t s) {
    const dim3 grid((unsigned)((a.P + kQTile - 1) / kQTile * a.H_q * a.B));
    const float qscale = 1.4426950408889634f / sqrtf((float)D);
    prefill_attn_kernel<D, KV, LAYOUT, BS16><<<grid, 256, 0, s>>>(
        a.Q, static_cast<const KV*>(a.k), static_cast<const KV*>(a.v), a.block_table,
        a.num_blocks_per_seq, a.block_size, a.P, a.H_q, a.H_kv, a.start_pos, a.causal ? 1 : 0, qscale,
        a.O);
}

template <int D>
void launch_d(const PrefillArgs& a, hipStream_t s) {
    if (a.paged) {
        const bool bs16 = a.block_size == 16;
        if (a.kv_dtype == IE_KV_BF16)
            bs16 ? launch_t<D, uint16_t, 0, true>(a, s) : launch_t<D, uint16_t, 0, false>(a, s);
        else
            bs16 ? launch_t<D, float, 0, true>(a, s) : launch_t<D, float, 0, false>(a, s);
    } else {
        launch_t<D, float, 1, false>(a, s);
    }
}

}  // namespace

void launch_prefill_attn(const PrefillArgs& a, hipStream_t s) {
    if (a.B == 0 || a.P == 0) return;
    if (a.d == 64)
        launch_d<64>(a, s);
    else
        launch_d<128>(a, s);
}

}  // namespace ie
