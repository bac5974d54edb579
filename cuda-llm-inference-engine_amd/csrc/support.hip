// support.hip — the non-GEMM, non-attention operations of the decode step:
// LayerNorm, token+position embedding, fp32 vocabulary projection and a
// device-side argmax.  They run once or twice per layer on [M, d] rows, so they
// are written for low latency, not as roofline kernels.
#include <algorithm>
#include <climits>

#include "device_util.h"
#include "ie_internal.h"

namespace ie {
namespace {

// kernels/layernorm/15_layernorm_residual.cu:59-103 (ln_accum / ln_finish /
// ln_apply).  One wave per row, four rows per workgroup, no barrier.  In
// place (out == x) is allowed: every element is read and written by the same
// lane.  VEC: cols % 4 == 0 and 16-byte aligned rows (the GEMV prologue's
// order); otherwise lanes take single elements l, l + 64, ...
template <bool VEC>
__global__ __launch_bounds__(256) void layernorm_kernel(int rows, int cols, const float* x,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta,
                                                        float* out, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    const float* xr = x + (size_t)row * cols;
    float* orow = out + (size_t)row * cols;
    float s = 0.0f, s2 = 0.0f, mean, rs;
    if constexpr (VEC) {
        const int n4 = cols >> 2;
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        for (int j = lane; j < n4; j += 64) ln_accum(x4[j], s, s2);
        ln_finish(s, s2, cols, eps, mean, rs);
        const float4* g4 = reinterpret_cast<const float4*>(gamma);
        const float4* b4 = reinterpret_cast<const float4*>(beta);
        float4* o4 = reinterpret_cast<float4*>(orow);
        for (int j = lane; j < n4; j += 64) o4[j] = ln_apply(x4[j], g4[j], b4[j], mean, rs);
    } else {
        for (int c = lane; c < cols; c += 64) {
            const float v = xr[c];
            s += v;
            s2 = fmaf(v, v, s2);
        }
        ln_finish(s, s2, cols, eps, mean, rs);
        for (int c = lane; c < cols; c += 64) orow[c] = fmaf(gamma[c] * (xr[c] - mean), rs, beta[c]);
    }
}

// kernels/layernorm/15_layernorm_residual.cu:6-57: y = x + residual (one fp32
// add), residual_out = y, out = LayerNorm(y) with the standalone LayerNorm's
// reduction order (ln_accum / ln_finish / ln_apply), so out equals
// layernorm(residual_out) bit for bit.  As in the reference, any of out and
// residual_out may alias x or residual (or each other): a lane reads an
// element's x and residual before it writes that element, and the second pass
// reads y back from residual_out, which the same lane wrote.
template <bool VEC>
__global__ __launch_bounds__(256) void layernorm_residual_kernel(int rows, int cols, const float* x,
                                                                 const float* res,
                                                                 const float* __restrict__ gamma,
                                                                 const float* __restrict__ beta,
                                                                 float* out, float* res_out, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lane = threadIdx.x & 63;
    const size_t off = (size_t)row * cols;
    float s = 0.0f, s2 = 0.0f, mean, rs;
    if constexpr (VEC) {
        const int n4 = cols >> 2;
        const float4* x4 = reinterpret_cast<const float4*>(x + off);
        const float4* r4 = reinterpret_cast<const float4*>(res + off);
        float4* y4 = reinterpret_cast<float4*>(res_out + off);
        for (int j = lane; j < n4; j += 64) {
            const float4 a = x4[j], b = r4[j];
            const float4 y = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
            y4[j] = y;
            ln_accum(y, s, s2);
        }
        ln_finish(s, s2, cols, eps, mean, rs);
        const float4* g4 = reinterpret_cast<const float4*>(gamma);
        const float4* b4 = reinterpret_cast<const float4*>(beta);
        float4* o4 = reinterpret_cast<float4*>(out + off);
        for (int j = lane; j < n4; j += 64) {
            const float4 y = y4[j];
            o4[j] = ln_apply(y, g4[j], b4[j], mean, rs);
        }
    } else {
        for (int c = lane; c < cols; c += 64) {
            const float v = x[off + c] + res[off + c];
            res_out[off + c] = v;
            s += v;
            s2 = fmaf(v, v, s2);
        }
        ln_finish(s, s2, cols, eps, mean, rs);
        for (int c = lane; c < cols; c += 64) {
            const float v = res_out[off + c];
            out[off + c] = fmaf(gamma[c] * (v - mean), rs, beta[c]);
        }
    }
}

// kernels/layernorm/15_embed.cu:4-21.
__global__ __launch_bounds__(256) void embedding_kernel(const int* __restrict__ ids, int seq_len,
                                                        int start_pos, int d,
                                                        const float* __restrict__ wte,
                                                        const float* __restrict__ wpe,
                                                        float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)seq_len * d) return;
    const int t = (int)(idx / d);
    const int i = (int)(idx - (size_t)t * d);
    out[idx] = wte[(size_t)ids[t] * d + i] + wpe[(size_t)(start_pos + t) * d + i];
}

__global__ __launch_bounds__(256) void embedding_batch_kernel(int B, const int* __restrict__ ids,
                                                              const int* __restrict__ positions,
                                                              int d, const float* __restrict__ wte,
                                                              const float* __restrict__ wpe,
                                                              float* __restrict__ out) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)B * d) return;
    const int b = (int)(idx / d);
    const int i = (int)(idx - (size_t)b * d);
    out[idx] = wte[(size_t)ids[b] * d + i] + wpe[(size_t)positions[b] * d + i];
}

// src/gpt2_engine.cu:391-403: logits[r][j] = hidden[r] . wte[j].  Each 16-lane
// row owns one vocabulary row and streams it with 16-byte loads (the
// reference gives each thread a whole row, which does not coalesce).
template <int RT>
__global__ __launch_bounds__(256) void vocab_proj_kernel(int rows, const float* __restrict__ h,
                                                         const float* __restrict__ wte,
                                                         float* __restrict__ logits, int d,
                                                         int V) {
    const int lane = threadIdx.x & 63, li = lane & 15;
    const int j = blockIdx.x * 16 + (threadIdx.x >> 6) * 4 + (lane >> 4);
    const bool ok = j < V;
    float acc[RT];
#pragma unroll
    for (int r = 0; r < RT; ++r) acc[r] = 0.0f;
    if (ok) {
        const float* w = wte + (size_t)j * d;
#pragma unroll 4
        for (int k = li * 4; k < d; k += 64) {
            const float4 wv = *reinterpret_cast<const float4*>(w + k);
#pragma unroll
            for (int r = 0; r < RT; ++r) {
                const int rr = r < rows ? r : rows - 1;
                const float4 hv = *reinterpret_cast<const float4*>(h + (size_t)rr * d + k);
                float a = acc[r];
                a = fmaf(wv.x, hv.x, a);
                a = fmaf(wv.y, hv.y, a);
                a = fmaf(wv.z, hv.z, a);
                a = fmaf(wv.w, hv.w, a);
                acc[r] = a;
            }
        }
    }
    float mine = 0.0f;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
        const float t = row16_sum(acc[r]);
        if (li == r) mine = t;
    }
    if (ok && li < rows && li < RT) logits[(size_t)li * V + j] = mine;
}

// The same projection on v_mfma_f32_16x16x4_f32 for any row count 1..16
// when d = 256 * NCH (GPT-2: NCH = 3): a 16-vocabulary-row tile of logits^T =
// wte tile (A) x hidden^T (B, zero past `rows`).
//   * Persistent workgroups walk the tiles (tile = blockIdx.x + n * gridDim.x)
//     with the next tile's weights loaded while the current one is computed
//     (the fused head, one workgroup per CU with its 512 registers per lane:
//     the next two tiles; batch-1 / 16 decode step -1.0 / -0.9 us, same bits).
//   * The four waves split K: wave w owns k in [w d/4, (w+1) d/4), NCH chunks
//     of 64.  It holds its quarter of the hidden rows in registers for the
//     whole kernel, so nothing is staged per tile, and its partial 16 x 16
//     tile is summed with the other three in LDS in a fixed order.
//   * MFMA operand layout: within chunk c, fragment e of lane (i, g)
//     (i = l % 16, g = l / 16) is vocabulary row v0 + i at k = 64c + 16e +
//     4g .. +3; MFMA step (e, s) sums k = 64c + 16e + 4g + s over g for A
//     and B alike, every k once.
//   * Loads: read in that layout, a wave instruction would cover 16 rows x
//     64 bytes, half of each 128-byte line, and with non-temporal loads that
//     pattern streams slower (a lab over the 154 MB GPT-2 wte: 5.3 TB/s
//     against 6.6 TB/s for 4 rows x 256 bytes per instruction).  So instruction (rg, c)
//     reads rows 4rg .. 4rg + 3 x 256 contiguous bytes (lane l: row 4rg +
//     l / 16, k = 64c + 4(l % 16)), and each wave passes its 12 fragments
//     through its own 12 KB of LDS into the operand layout (XOR-swizzled
//     slots: both the writes and the reads of 16 consecutive lanes cover 256
//     distinct bytes).  The MFMAs see the same values in the same order.
//   * Four accumulators (one per e) keep the MFMAs independent and are added
//     in a fixed order.
// A logit depends on its own hidden row only (zero columns add nothing to
// the others), so a batch of 16 and a batch of 1 give the same bits per row.
// Plain loads: non-temporal ones measured ~10% slower here.
//
// Key of a (logit, index) pair whose unsigned maximum is the first index of
// the largest logit: the value in an order-preserving bit pattern (-0 taken
// as +0, as a float comparison does) above the complement of the index.
__device__ __forceinline__ unsigned long long argmax_key(float v, int idx) {
    uint32_t u = __builtin_bit_cast(uint32_t, v == 0.0f ? 0.0f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (0xFFFFFFFFu - (uint32_t)idx);
}

// HEAD: the decode step's head in one launch.  h is then the hidden state x
// before the final LayerNorm: the workgroup first normalises the rows into
// LDS with the standalone LayerNorm's arithmetic (ln_*, one wave per row, the
// same lane order, so the same bits), and the argmax of each row (first index
// of the maximum) is folded in: every workgroup keeps its rows' best (value,
// index) while it writes the logits and merges it into keys[row] with one
// 64-bit atomic max (argmax_key).  The last workgroup to finish (a counter,
// `done`) turns the keys into token ids (finalize_row): every
// workgroup's atomic max has completed (vmcnt) before its counter increment,
// and keys and counter are only touched by atomics, so the last one to
// increment reads every row's final key.  It then clears keys and counter
// for the next launch.
struct HeadArgs {
    const float* gamma = nullptr;
    const float* beta = nullptr;
    float eps = 1e-5f;
    unsigned long long* keys = nullptr;
    unsigned* done = nullptr;  // 0 before the launch, 0 after it
    int* tokens = nullptr;
    int* positions = nullptr;
    int advance = 0;
    int* host_ids = nullptr;
};

// tokens[b] from keys[b] (cleared), the ids also to host_ids slot
// positions[b] & 1 (system-scope stores; pinned host memory [2][B]), and
// positions[b] += advance.
__device__ __forceinline__ void finalize_row(int B, int b, unsigned long long* keys, int* tokens, int* positions,
                                             int advance, int* host_ids) {
    const unsigned long long k = __hip_atomic_load(keys + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int tok = (int)(0xFFFFFFFFu - (uint32_t)k);
    tokens[b] = tok;
    __hip_atomic_store(keys + b, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int p = positions[b];
    if (host_ids) __hip_atomic_store(host_ids + (p & 1) * B + b, tok, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (advance) positions[b] = p + 1;
}

template <int NCH, bool HEAD = false>
__global__ __launch_bounds__(256, NCH >= 5 || HEAD ? 1 : 2) void vocab_proj_mfma_kernel(int rows, const float* __restrict__ h,
                                                                 const float* __restrict__ wte,
                                                                 float* __restrict__ logits, int d, int V,
                                                                 HeadArgs ha) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    __shared__ f32x4 red[2][4][64];
    __shared__ f32x4 tr[4][4 * NCH][64];  // each wave's fragments on their way to the operand layout
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int i = lane & 15, g = lane >> 4;
    const int kq = w * NCH * 64;
    const int ntiles = (V + 15) / 16;
    // provenance hidden, so the compiler keeps the first tile's loads where
    // they are issued instead of sinking them past the LayerNorm to their use
    const float* wsrc = HEAD ? opaque_global(wte) : wte;
    // b[rg][c]: row 4rg + l / 16, k = kq + 64c + 4(l % 16)
    auto load = [&](f32x4 (&b)[4][NCH], int t) {
        const int r0 = min(t, ntiles - 1) * 16 + (lane >> 4);
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
            const float* p = wsrc + (size_t)min(r0 + 4 * rg, V - 1) * d + kq + 4 * (lane & 15);
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                if constexpr (HEAD)
                    b[rg][c] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + 64 * c));
                else
                    b[rg][c] = *reinterpret_cast<const f32x4*>(p + 64 * c);
            }
        }
    };
    // Slot of fragment (row 4rg + r4, k = 64c + 16e + 4g) in block (rg, c)
    // of the wave's LDS: 16e + 4(r4 ^ e) + (g ^ rg).
    auto to_operands = [&](const f32x4 (&b)[4][NCH], float4 (&a)[NCH][4]) {
        {
            const int r4 = lane >> 4, e = (lane >> 2) & 3, gg = lane & 3;
#pragma unroll
            for (int rg = 0; rg < 4; ++rg)
#pragma unroll
                for (int c = 0; c < NCH; ++c) tr[w][rg * NCH + c][16 * e + 4 * (r4 ^ e) + (gg ^ rg)] = b[rg][c];
        }
        const int rg = i >> 2, r4 = i & 3;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f32x4 v = tr[w][rg * NCH + c][16 * e + 4 * (r4 ^ e) + (g ^ rg)];
                a[c][e] = make_float4(v.x, v.y, v.z, v.w);
            }
    };
    int t = blockIdx.x;
    if (t >= ntiles) return;  // uniform over the workgroup
    // HEAD: this wave's hidden rows (w, w + 4, ...; rows <= 16) and the
    // LayerNorm parameters are requested first, then the first tile's
    // weights, which do not depend on them: loads return in order, so the
    // rows arrive, and the LayerNorm runs, while the tile is in flight.
    constexpr int NV = HEAD ? NCH : 1;  // float4s of a row per lane (d = 256 NCH)
    float4 xr[HEAD ? 4 : 1][NV], gv[NV], bv[NV];
    if constexpr (HEAD) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int r = w + 4 * rr;
            if (r < rows) {
                const float4* x4 = reinterpret_cast<const float4*>(h + (size_t)r * d);
#pragma unroll
                for (int j = 0; j < NV; ++j) xr[rr][j] = x4[lane + 64 * j];
            }
        }
        const float4* g4 = reinterpret_cast<const float4*>(ha.gamma);
        const float4* b4 = reinterpret_cast<const float4*>(ha.beta);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            gv[j] = g4[lane + 64 * j];
            bv[j] = b4[lane + 64 * j];
        }
    }
    f32x4 wa[4][NCH], wb[4][NCH], wc[4][NCH];
    load(wa, t);
    if constexpr (HEAD) load(wb, t + gridDim.x);
    float4 hb[NCH][4];
    if constexpr (HEAD) {
        extern __shared__ float4 hs[];  // the normalised rows [rows][d / 4]
        const int d4 = d >> 2;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int r = w + 4 * rr;
            if (r < rows) {
                float s = 0.0f, s2 = 0.0f, mean, rs;
#pragma unroll
                for (int j = 0; j < NV; ++j) ln_accum(xr[rr][j], s, s2);
                ln_finish(s, s2, d, ha.eps, mean, rs);
#pragma unroll
                for (int j = 0; j < NV; ++j) hs[r * d4 + lane + 64 * j] = ln_apply(xr[rr][j], gv[j], bv[j], mean, rs);
            }
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                hb[c][e] = i < rows ? hs[i * d4 + ((kq + 64 * c + 16 * e + 4 * g) >> 2)]
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    } else {
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                hb[c][e] = i < rows ? *reinterpret_cast<const float4*>(h + (size_t)i * d + kq + 64 * c + 16 * e + 4 * g)
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    // this lane's best logit of row i so far (wave 0, HEAD): indices only grow
    // along a lane's walk, so a strict > keeps the first maximum
    float best = -INFINITY;
    int bi = INT_MAX;
    int par = 0;
    auto tile = [&](const f32x4 (&raw)[4][NCH], int t) {
        float4 b[NCH][4];
        to_operands(raw, b);
        f32x4 acc[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float4 a = b[c][e], hv = hb[c][e];
                acc[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, hv.x, acc[e], 0, 0, 0);
                acc[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, hv.y, acc[e], 0, 0, 0);
                acc[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, hv.z, acc[e], 0, 0, 0);
                acc[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, hv.w, acc[e], 0, 0, 0);
            }
        red[par][w][lane] = ((acc[0] + acc[1]) + acc[2]) + acc[3];
        // One barrier per tile: the buffer written here is next written two
        // tiles later, after every wave has passed the next tile's barrier,
        // which wave 0 reaches only once it has read this one.
        __syncthreads();
        if (w == 0 && i < rows) {
            const f32x4 s4 = ((red[par][0][lane] + red[par][1][lane]) + red[par][2][lane]) + red[par][3][lane];
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int vr = t * 16 + 4 * g + v;  // result row 4g + v, hidden row i
                if (vr < V) {
                    logits[(size_t)i * V + vr] = s4[v];
                    if constexpr (HEAD)
                        if (s4[v] > best || bi == INT_MAX) {
                            best = s4[v];
                            bi = vr;
                        }
                }
            }
        }
        par ^= 1;
    };
    if constexpr (HEAD) {
        // three tiles in the ring: two in flight while one is computed
        const int G3 = 2 * (int)gridDim.x;
        while (true) {
            load(wc, t + G3);
            tile(wa, t);
            t += gridDim.x;
            if (t >= ntiles) break;
            load(wa, t + G3);
            tile(wb, t);
            t += gridDim.x;
            if (t >= ntiles) break;
            load(wb, t + G3);
            tile(wc, t);
            t += gridDim.x;
            if (t >= ntiles) break;
        }
    } else {
        while (true) {
            load(wb, t + gridDim.x);
            tile(wa, t);
            t += gridDim.x;
            if (t >= ntiles) break;
            load(wa, t + gridDim.x);
            tile(wb, t);
            t += gridDim.x;
            if (t >= ntiles) break;
        }
    }
    if constexpr (HEAD) {
        if (w == 0) {
            // lanes i, i + 16, i + 32, i + 48 hold row i's candidates
            unsigned long long key = bi == INT_MAX ? 0ull : argmax_key(best, bi);
#pragma unroll
            for (int o = 16; o < 64; o <<= 1) {
                const unsigned long long other = __shfl_xor(key, o, 64);
                key = other > key ? other : key;
            }
            if (g == 0 && i < rows && key) atomicMax(ha.keys + i, key);
        }
        __shared__ int last;
        if (threadIdx.x == 0) {
            // wave 0's atomic maxima have completed before the increment
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            const unsigned prev = __hip_atomic_fetch_add(ha.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = prev == gridDim.x - 1;
        }
        __syncthreads();
        if (last) {
            if (threadIdx.x < rows)
                finalize_row(rows, threadIdx.x, ha.keys, ha.tokens, ha.positions, ha.advance, ha.host_ids);
            if (threadIdx.x == 0) __hip_atomic_store(ha.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// src/sampler.cu:10-14 on the device: first index of the maximum (ties go to
// the lower index, as std::max_element).  One 1024-thread workgroup per row
// reads the row as 16-byte chunks from its 16-byte-aligned base (a 50257-wide
// row is 12.3 chunks per thread, all in flight at once; 4-byte loads took
// 7.3 us for such a row against 2.8 us); the at most two chunks that straddle
// the row's ends are read element by element.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ void argmax_take(float& best, int& bi, float v, int i) {
    if (v > best || (v == best && i < bi)) {
        best = v;
        bi = i;
    }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ logits,
                                                                int n, int* __restrict__ out) {
    const float* x = logits + (size_t)blockIdx.x * n;
    const int s = (int)(((uintptr_t)x & 15u) >> 2);
    const float4* x4 = reinterpret_cast<const float4*>(x - s);
    const int cf = s == 0 ? 0 : 1, cl = (n + s) / 4 - 1;  // chunks wholly inside the row
    const int nch = (n + s + 3) / 4;
    float best = -INFINITY;
    int bi = INT_MAX;
    constexpr int U = 8;
    for (int c0 = threadIdx.x; c0 < nch; c0 += kArgmaxThreads * U) {
        float4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * kArgmaxThreads;
            v[u] = cf <= cl ? x4[min(max(c, cf), cl)] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + u * kArgmaxThreads, e0 = 4 * c - s;
            if (c >= nch) continue;
            if (c < cf || c > cl) {  // a chunk straddling an end of the row
                v[u].x = e0 >= 0 && e0 < n ? x[e0] : 0.f;
                v[u].y = e0 + 1 >= 0 && e0 + 1 < n ? x[e0 + 1] : 0.f;
                v[u].z = e0 + 2 >= 0 && e0 + 2 < n ? x[e0 + 2] : 0.f;
                v[u].w = e0 + 3 < n ? x[e0 + 3] : 0.f;
            }
            const float e[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
            // a thread's indices increase, so a strict > keeps its first
            // maximum; the first element it sees is always taken (an all
            // -inf row still reports an index)
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (e0 + k >= 0 && e0 + k < n && (e[k] > best || bi == INT_MAX)) {
                    best = e[k];
                    bi = e0 + k;
                }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        argmax_take(best, bi, __shfl_xor(best, off, 64), __shfl_xor(bi, off, 64));
    constexpr int W = kArgmaxThreads / 64;
    __shared__ float sb[W];
    __shared__ int si[W];
    if ((threadIdx.x & 63) == 0) {
        sb[threadIdx.x >> 6] = best;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        best = threadIdx.x < W ? sb[threadIdx.x] : -INFINITY;
        bi = threadIdx.x < W ? si[threadIdx.x] : INT_MAX;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1)
            argmax_take(best, bi, __shfl_xor(best, off, 64), __shfl_xor(bi, off, 64));
        if (threadIdx.x == 0) out[blockIdx.x] = bi < n ? bi : 0;
    }
}

}  // namespace

void launch_layernorm(int rows, int cols, const float* x, const float* g, const float* b,
                      float* out, float eps, hipStream_t s) {
    if (rows == 0) return;
    const bool vec = cols % 4 == 0 && (((uintptr_t)x | (uintptr_t)g | (uintptr_t)b |
                                        (uintptr_t)out) % 16) == 0;
    const unsigned blocks = (unsigned)((rows + 3) / 4);
    if (vec)
        layernorm_kernel<true><<<blocks, 256, 0, s>>>(rows, cols, x, g, b, out, eps);
    else
        layernorm_kernel<false><<<blocks, 256, 0, s>>>(rows, cols, x, g, b, out, eps);
}

void launch_layernorm_residual(int rows, int cols, const float* x, const float* res, const float* g,
                               const float* b, float* out, float* res_out, float eps, hipStream_t s) {
    if (rows == 0) return;
    const bool vec = cols % 4 == 0 && (((uintptr_t)x | (uintptr_t)res | (uintptr_t)g | (uintptr_t)b |
                                        (uintptr_t)out | (uintptr_t)res_out) % 16) == 0;
    const unsigned blocks = (unsigned)((rows + 3) / 4);
    if (vec)
        layernorm_residual_kernel<true><<<blocks, 256, 0, s>>>(rows, cols, x, res, g, b, out, res_out, eps);
    else
        layernorm_residual_kernel<false><<<blocks, 256, 0, s>>>(rows, cols, x, res, g, b, out, res_out, eps);
}

void launch_embedding(const int* ids, int seq_len, int start_pos, int d, const float* wte,
                      const float* wpe, float* out, hipStream_t s) {
    const size_t total = (size_t)seq_len * d;
    if (total == 0) return;
    embedding_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(ids, seq_len, start_pos, d,
                                                                     wte, wpe, out);
}

void launch_embedding_batch(int B, const int* ids, const int* positions, int d,
                            const float* wte, const float* wpe, float* out, hipStream_t s) {
    const size_t total = (size_t)B * d;
    if (total == 0) return;
    embedding_batch_kernel<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(B, ids, positions, d,
                                                                           wte, wpe, out);
}

void launch_vocab_proj(int rows, const float* h, const float* wte, float* logits, int d, int V,
                       hipStream_t s) {
    if (rows == 0 || V == 0) return;
    if (d % 256 == 0 && d <= 1280) {
        // one workgroup per CU: more measured no faster (the stream is
        // bandwidth-bound with four waves' tiles in flight per CU)
        const unsigned grid = (unsigned)std::min<long long>((V + 15) / 16, num_cus());
        const HeadArgs none{};
        switch (d / 256) {
            case 1: vocab_proj_mfma_kernel<1><<<grid, 256, 0, s>>>(rows, h, wte, logits, d, V, none); break;
            case 2: vocab_proj_mfma_kernel<2><<<grid, 256, 0, s>>>(rows, h, wte, logits, d, V, none); break;
            case 3: vocab_proj_mfma_kernel<3><<<grid, 256, 0, s>>>(rows, h, wte, logits, d, V, none); break;
            case 4: vocab_proj_mfma_kernel<4><<<grid, 256, 0, s>>>(rows, h, wte, logits, d, V, none); break;
            default: vocab_proj_mfma_kernel<5><<<grid, 256, 0, s>>>(rows, h, wte, logits, d, V, none); break;
        }
        return;
    }
    const unsigned blocks = (unsigned)((V + 15) / 16);
    if (rows == 1)
        vocab_proj_kernel<1><<<blocks, 256, 0, s>>>(rows, h, wte, logits, d, V);
    else
        vocab_proj_kernel<16><<<blocks, 256, 0, s>>>(rows, h, wte, logits, d, V);
}

bool vocab_head_supported(int rows, int d) { return rows >= 1 && rows <= 16 && d % 256 == 0 && d <= 1024; }

void launch_vocab_head(int rows, const float* x, const float* gamma, const float* beta, float eps,
                       const float* wte, float* logits, int d, int V, unsigned long long* keys, unsigned* done,
                       int* tokens, int* positions, bool advance, int* host_ids, hipStream_t s) {
    HeadArgs ha;
    ha.gamma = gamma;
    ha.beta = beta;
    ha.eps = eps;
    ha.keys = keys;
    ha.done = done;
    ha.tokens = tokens;
    ha.positions = positions;
    ha.advance = advance ? 1 : 0;
    ha.host_ids = host_ids;
    const unsigned grid = (unsigned)std::min<long long>((V + 15) / 16, num_cus());
    const size_t lds = (size_t)rows * d * sizeof(float);
    switch (d / 256) {
        case 1: vocab_proj_mfma_kernel<1, true><<<grid, 256, lds, s>>>(rows, x, wte, logits, d, V, ha); break;
        case 2: vocab_proj_mfma_kernel<2, true><<<grid, 256, lds, s>>>(rows, x, wte, logits, d, V, ha); break;
        case 3: vocab_proj_mfma_kernel<3, true><<<grid, 256, lds, s>>>(rows, x, wte, logits, d, V, ha); break;
        default: vocab_proj_mfma_kernel<4, true><<<grid, 256, lds, s>>>(rows, x, wte, logits, d, V, ha); break;
    }
}


void launch_argmax(int rows, const float* logits, int n, int* out, hipStream_t s) {
    if (rows == 0) return;
    argmax_kernel<<<rows, kArgmaxThreads, 0, s>>>(logits, n, out);
}

}  // namespace ie
