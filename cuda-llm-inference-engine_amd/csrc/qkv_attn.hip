// qkv_attn.hip — the engine's QKV projection and decode attention in one
// launch, one workgroup per (sequence b, head h).
//
// In a decode step the attention of head h of sequence b needs only that
// head's q, k and v (and the cache), not the other heads' outputs, so the
// QKV projection and the attention need no grid-wide step between them when
// a workgroup owns the head's 3 x D projection rows.  The workgroup
//   1. requests the head's 3 x D weight rows and their epilogue operands,
//      and (SplitWalk::begin) the block-table lookups and first cache chunk
//      of each wave's share of the attention, which are in flight during
//      steps 2-3,
//   2. builds the int8 activation row of x[b] in LDS (LayerNorm + per-row
//      quantizer, as the fused GEMV prologue; its loads go out in step 1),
//   3. computes the rows with dot4 and the 16-lane DPP reduction and stores
//      them as the QKV epilogue does: q to Q, k and v appended to the cache at
//      the sequence's position (src/gpt2_engine.cu:464-481 of the reference);
//      the head's q, k and v also go to LDS, in the cache's representation,
//   4. walks the head's cached tokens on its 8 waves (SplitWalk::run) with q
//      from LDS, substituting the LDS k and v for every read of the appended
//      token's cache row (the early loads may have read it before it was
//      written), and merges the waves in LDS (split_finish_lds), as
//      decode_attn_split_kernel does for a one-split plan
//      (src/gpt2_engine.cu:496-504 / K13).
// Every value is produced by the same device code in the same order as the
// QKV GEMV + attention kernel pair, so the outputs are bit-identical to that
// pair (and to the step built from the C ABI).  One launch per layer fewer:
// GPT-2 Small, d = 768, D = 64, block size 16, a one-split plan.
#include <type_traits>

#include "attn_split.h"
#include "gemv_common.h"
#include "ie_internal.h"

namespace ie {
namespace {

constexpr int kQaWaves = 8;  // the 8-wave form of the one-split attention
constexpr int kQaK = 768;    // d_model (the projection's K)

// EMB: the first layer's launch builds x[b] itself (f.ids set): the
// embedding wte[ids[b]] + wpe[positions[b]], which head 0's workgroup also
// stores to x for the layer's residual adds; the embedding launch is saved.
// NTL: the cache walk reads with non-temporal loads (f.kv_stream).
template <int D, typename KV, bool EMB, bool NTL>
__global__ __launch_bounds__(64 * kQaWaves) void qkv_attn_kernel(const int32_t* __restrict__ BT,
                                                                 const float* __restrict__ sB,
                                                                 const float* __restrict__ bias, GemvFusion f,
                                                                 const KV* __restrict__ kcache,
                                                                 const KV* __restrict__ vcache, int H,
                                                                 float qscale, float* __restrict__ O) {
    constexpr int K16 = kQaK / 16, CPL = K16 / 16;  // 16-byte chunks per row, per lane
    constexpr int RPW = 3 * D / kQaWaves;           // projection rows per wave
    constexpr int G = RPW / 4;                      // 4-row groups per wave
    static_assert(RPW % 4 == 0 && K16 % 16 == 0, "head rows split into 4-row groups");
    constexpr int d = kQaK;
    __shared__ i32x4 a_lds[K16];
    __shared__ float s_sa[1];
    __shared__ float s_q[D];
    __shared__ __attribute__((aligned(16))) KV s_k[D], s_v[D];
    const int h = blockIdx.x, b = blockIdx.y;
    const int lane = threadIdx.x & 63, li = lane & 15;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // Row 0 of this view is sequence b.
    GemvFusion fb = f;
    fb.q = f.q + (size_t)b * d;
    fb.positions = f.positions + b;
    fb.table = f.table + (size_t)b * f.nbps;
    fb.ctx_lens = f.ctx_lens + b;

    // Projection row of lane group (wave wv, group g): q, k or v row i of head h.
    auto row_of = [&](int g) {
        const int lr = (wv * G + g) * 4 + (lane >> 4);
        const int which = lr / D;
        return which * d + h * D + (lr - which * D);
    };
    // Wave 0's activation row and LayerNorm parameters are requested first:
    // vector loads return in order, so behind the weights they would wait
    // for them; and before the position / block-table lookups below, scalar
    // loads in a dependent chain (a wait for any scalar load waits for all).
    float4 xv[kQaK / 256];
    LnVec<kQaK> lnp;
    if (wv == 0) {
        if constexpr (EMB) {
            const float4* e4 = reinterpret_cast<const float4*>(f.wte + (size_t)f.ids[b] * d);
            const float4* p4 = reinterpret_cast<const float4*>(f.wpe + (size_t)f.positions[b] * d);
            float4 ev[kQaK / 256], pv[kQaK / 256];
#pragma unroll
            for (int i = 0; i < kQaK / 256; ++i) {
                ev[i] = e4[lane + 64 * i];
                pv[i] = p4[lane + 64 * i];
            }
            ln_load<kQaK, kSrcLnQuant>(f, lnp, lane);
#pragma unroll
            for (int i = 0; i < kQaK / 256; ++i) {
                xv[i] = make_float4(ev[i].x + pv[i].x, ev[i].y + pv[i].y, ev[i].z + pv[i].z, ev[i].w + pv[i].w);
                if (h == 0) reinterpret_cast<float4*>(const_cast<float*>(f.x) + (size_t)b * d)[lane + 64 * i] = xv[i];
            }
        } else {
            stage_load<kQaK>(f.x + (size_t)b * d, xv, lane);
            ln_load<kQaK, kSrcLnQuant>(f, lnp, lane);
        }
    }
    const i32x4* w4 = reinterpret_cast<const i32x4*>(BT);
    i32x4 wreg[G][CPL];
    EpiIn ein[G];
#pragma unroll
    for (int g = 0; g < G; ++g) ein[g] = epi_load<IE_EPI_BIAS>(0, row_of(g), 3 * d, sB, bias, nullptr);
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const i32x4* w = w4 + (size_t)row_of(g) * K16 + li;
#pragma unroll
        for (int t = 0; t < CPL; ++t) wreg[g][t] = w[16 * t];
    }
    size_t slot[1];
    qkv_slots<1>(fb, 1, slot);

    // Tokens 0 .. pos of the sequence (never past its block-table row).
    const int pos = f.positions[b];
    const int tok1 = (int)min((long long)pos + 1, (long long)f.nbps * f.block_size);
    SplitWalk<D, 1, KV, kQaWaves, true, 2, NTL> walk;
    walk.begin(kcache, vcache, fb.table, h, H, f.block_size, 0, tok1, wv, lane);

    if (wv == 0) stage_compute<kQaK, kSrcLnQuant>(xv, f, lnp, reinterpret_cast<int32_t*>(a_lds), &s_sa[0], lane);
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
        int32_t acc[1] = {0};
#pragma unroll
        for (int t = 0; t < CPL; ++t) dot_chunk<1>(acc, wreg[g][t], a_lds, K16, li + 16 * t);
        // gemv_finish<1, kEpiQKV>, plus the LDS copy of the stored value.
        const int32_t tot = row16_sum(acc[0]);
        if (li == 0) {
            const int n = row_of(g);
            gemv_store<kEpiQKV>(nullptr, 0, n, 3 * d, tot, s_sa[0], ein[g], slot[0], fb);
            const float v = epilogue_value<IE_EPI_BIAS>(tot, s_sa[0], ein[g].sb, ein[g].bias, 0.0f);
            const int lr = (wv * G + g) * 4 + (lane >> 4);
            const int which = lr / D, r = lr - which * D;
            if (which == 0) {
                s_q[r] = v;
            } else {
                KV kv;
                if constexpr (sizeof(KV) == 2)
                    kv = f32_to_bf16_rne(v);
                else
                    kv = v;
                (which == 1 ? s_k : s_v)[r] = kv;
            }
        }
    }
    __syncthreads();

    constexpr int EPL = D / 16;
    float q[1][EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) q[0][e] = s_q[li * EPL + e] * qscale;
    const int grp = lane >> 4;
    auto patch = [&](Chunk<D, KV, 4>& c, int cs) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (min(cs + 4 * j + grp, tok1 - 1) == pos) {
                const uint32_t* kw = reinterpret_cast<const uint32_t*>(s_k + li * EPL);
                const uint32_t* vw = reinterpret_cast<const uint32_t*>(s_v + li * EPL);
#pragma unroll
                for (int w = 0; w < Slice<EPL, KV>::WORDS; ++w) {
                    c.k[j].w[w] = kw[w];
                    c.v[j].w[w] = vw[w];
                }
            }
        }
    };
    float m[1], l[1], o[1][EPL];
    walk.run(q, m, l, o, patch);
    split_finish_lds<D, 1, kQaWaves>(b, h, H, 0, 1, wv, lane, m, l, o, nullptr, O);
}

}  // namespace

bool qkv_attn_supported(int d_model, int n_heads, int d_head, int block_size) {
    return d_model == kQaK && d_head == 64 && n_heads * d_head == d_model && block_size == 16;
}

void launch_qkv_attn(int B, int H, const int32_t* BT, const float* sB, const float* bias, const GemvFusion& f,
                     float* O, hipStream_t s) {
    constexpr int D = 64;
    const float qscale = (1.0f / sqrtf((float)D)) * 1.4426950408889634f;
    const dim3 grid(H, B);
    auto go = [&](auto emb, auto ntl) {
        constexpr bool E = decltype(emb)::value, N = decltype(ntl)::value;
        if (f.kv_dtype == IE_KV_BF16)
            qkv_attn_kernel<D, uint16_t, E, N><<<grid, 64 * kQaWaves, 0, s>>>(
                BT, sB, bias, f, static_cast<const uint16_t*>(f.kc), static_cast<const uint16_t*>(f.vc), H, qscale,
                O);
        else
            qkv_attn_kernel<D, float, E, N><<<grid, 64 * kQaWaves, 0, s>>>(
                BT, sB, bias, f, static_cast<const float*>(f.kc), static_cast<const float*>(f.vc), H, qscale, O);
    };
    auto go_n = [&](auto emb) {
        if (f.kv_stream)
            go(emb, std::true_type{});
        else
            go(emb, std::false_type{});
    };
    if (f.ids)
        go_n(std::true_type{});
    else
        go_n(std::false_type{});
}

}  // namespace ie
