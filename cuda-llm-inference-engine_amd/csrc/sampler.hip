// Device half of the top-k sampler (src/sampler.cu:16-45): the k largest
// logits of each row with their indices, sorted by value descending and, for
// equal values, by index ascending (std::partial_sort leaves the order of
// equal values unspecified; this is the order a stable sort gives).  Only
// these k pairs cross PCIe; the reference copies the whole row (201 KB for
// GPT-2) and partial-sorts it on the host.  The draw itself (temperature
// softmax over the k values and the rand() threshold) stays on the host,
// where it is the same float arithmetic as the reference's.
//
// One 1024-thread workgroup per row.  Rows of up to 65533 logits (GPT-2's
// 50257 among them) are read once, as 16-byte chunks, into registers (64 keys
// per thread):
//   1. a lower bound M of the k-th largest key: the k-th largest of the 1024
//      per-thread maxima (a radix select over one key per thread);
//   2. the keys >= M (typically a few more than k) gathered into LDS;
//   3. each gathered key ranked by counting those before it (larger key, or
//      equal key and lower index), and the first k written.
// Longer rows, and rows where more than 2048 keys reach M (many equal
// values, or k near 1024), are streamed from memory (L2 after the first
// pass) through an exact radix select of the k-th largest key, 8 bits per
// pass (the histogram in LDS; each wave instruction adds its leading lane's
// bin with one atomic, the other lanes' bins lane by lane), a gather of the
// keys above it plus the lowest-index keys equal to it (ranked in index order
// only when some equal keys are left out), and a bitonic sort of those k.
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "ie_internal.h"

namespace ie {
namespace {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / 64;
constexpr int kTopkUnroll = 8;
constexpr int kTopkRegPer = 64;  // keys per thread in the register-resident kernel
constexpr int kTopkCand = 2048;  // candidates (keys >= the lower bound) sorted directly

// Unsigned key with the order of the floats; -0.0 is keyed as +0.0 so that
// values the reference compares equal are equal here.
__device__ __forceinline__ uint32_t order_key(float x) {
    uint32_t b = __float_as_uint(x);
    if (b == 0x80000000u) b = 0;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct TopkShared {
    uint32_t hist[256];
    uint32_t prefix, remaining, eqcount, gt, eq;
    uint32_t wave_tot[kTopkWaves];
    uint32_t ckey[kTopkCand];
    int cidx[kTopkCand];
};

// Adds one key per lane (where `match`) to bin `digit`: the leading lane's
// bin in one atomic for every lane that shares it.
__device__ __forceinline__ void hist_add(uint32_t* hist, bool match, uint32_t digit, int lane) {
    const uint64_t mm = __ballot(match);
    if (!mm) return;
    const int lead = __ffsll((unsigned long long)mm) - 1;
    const uint32_t d0 = __shfl(digit, lead, 64);
    const uint64_t same = __ballot(match && digit == d0);
    if (match && digit != d0) atomicAdd(&hist[digit], 1u);
    if (lane == lead) atomicAdd(&hist[d0], (uint32_t)__popcll(same));
}

// Wave 0 finds the bin holding the remaining-th largest key among those with
// the current prefix and publishes the longer prefix, the keys still needed
// within it and its count.  Called by every thread between two barriers.
__device__ __forceinline__ void select_digit(TopkShared& sh, uint32_t prefix, uint32_t remaining, int shift,
                                             int lane, int wid) {
    if (wid != 0) return;
    uint32_t c[4], s = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // lane l holds bins 255-4l .. 252-4l: lanes run from the top
        c[j] = sh.hist[255 - 4 * lane - j];
        s += c[j];
    }
    uint32_t incl = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
    }
    uint32_t acc = incl - s;
    if (acc < remaining && remaining <= incl) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (acc < remaining && remaining <= acc + c[j]) {
                sh.prefix = prefix | ((uint32_t)(255 - 4 * lane - j) << shift);
                sh.remaining = remaining - acc;
                sh.eqcount = c[j];
            }
            acc += c[j];
        }
    }
}

__device__ __forceinline__ void put(TopkShared& sh, uint32_t slot, uint32_t key, int i) {
    sh.ckey[slot] = key;
    sh.cidx[slot] = i;
}

// Radix select of the k-th largest key, 8 bits per pass from the top:
// add(hmask, prefix, shift) puts every candidate key whose bits under hmask
// equal prefix into bin (key >> shift) & 255.  Returns the key; `remaining`
// = how many keys equal to it belong to the top k, `eqcount` = how many
// candidates equal it.  Called by every thread.
template <typename Add>
__device__ __forceinline__ uint32_t radix_kth(TopkShared& sh, uint32_t k, Add&& add, int lane, int wid,
                                              uint32_t& remaining, uint32_t& eqcount) {
    uint32_t prefix = 0;
    remaining = k;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        const uint32_t hmask = pass == 0 ? 0u : (0xffffffffu << (shift + 8));
        if (threadIdx.x < 256) sh.hist[threadIdx.x] = 0;
        __syncthreads();
        add(hmask, prefix, shift);
        __syncthreads();
        select_digit(sh, prefix, remaining, shift, lane, wid);
        __syncthreads();
        prefix = sh.prefix;
        remaining = sh.remaining;
        eqcount = sh.eqcount;
        __syncthreads();  // all have read before the next pass publishes
    }
    return prefix;
}

// Bitonic sort of the `count` gathered entries (larger key first, then
// lower index); the first k are the output row.
__device__ __forceinline__ void sort_and_write(TopkShared& sh, int count, int k, float* out_vals, int* out_idx) {
    int KP = 1;
    while (KP < count) KP <<= 1;
    for (int t = count + threadIdx.x; t < KP; t += kTopkThreads) put(sh, t, 0u, INT_MAX);
    __syncthreads();
    for (int size = 2; size <= KP; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < KP / 2; t += kTopkThreads) {
                const int i = 2 * stride * (t / stride) + (t % stride), j = i + stride;
                const bool desc = (i & size) == 0;
                const uint32_t ka = sh.ckey[i], kb = sh.ckey[j];
                const int ia = sh.cidx[i], ib = sh.cidx[j];
                const bool a_first = ka > kb || (ka == kb && ia < ib);
                if (a_first != desc) {
                    put(sh, i, kb, ib);
                    put(sh, j, ka, ia);
                }
            }
            __syncthreads();
        }
    }
    for (int t = threadIdx.x; t < k; t += kTopkThreads) {
        out_vals[(size_t)blockIdx.x * k + t] = key_value(sh.ckey[t]);
        out_idx[(size_t)blockIdx.x * k + t] = sh.cidx[t];
    }
}

// Streams one row (every pass re-reads it: L2 after the first).
__device__ __forceinline__ void topk_stream_row(TopkShared& sh, const float* __restrict__ x, int n, int k,
                                                float* __restrict__ out_vals, int* __restrict__ out_idx, int lane,
                                                int wid) {
    // visits every index in rounds of kTopkUnroll coalesced loads per thread
    auto for_each = [&](auto&& f) {
        for (int base = threadIdx.x; base < n; base += kTopkThreads * kTopkUnroll) {
            float v[kTopkUnroll];
#pragma unroll
            for (int u = 0; u < kTopkUnroll; ++u) {
                const int i = base + u * kTopkThreads;
                v[u] = x[min(i, n - 1)];
            }
#pragma unroll
            for (int u = 0; u < kTopkUnroll; ++u) f(base + u * kTopkThreads, order_key(v[u]));
        }
    };

    uint32_t remaining, eqcount;
    const uint32_t prefix = radix_kth(
        sh, (uint32_t)k,
        [&](uint32_t hmask, uint32_t prefix, int shift) {
            for_each([&](int i, uint32_t key) {
                hist_add(sh.hist, i < n && (key & hmask) == prefix, (key >> shift) & 255u, lane);
            });
        },
        lane, wid, remaining, eqcount);
    const uint32_t T = prefix, kgt = (uint32_t)k - remaining;

    if (threadIdx.x == 0) sh.gt = sh.eq = 0;
    if (eqcount == remaining) {
        __syncthreads();
        for_each([&](int i, uint32_t key) {
            if (i < n && key >= T) put(sh, key > T ? atomicAdd(&sh.gt, 1u) : kgt + atomicAdd(&sh.eq, 1u), key, i);
        });
    } else {
        // Wave w walks indices [w S, (w+1) S) in order; a first walk counts
        // its equal keys so that every equal key gets its global rank.
        const int S = ((n + kTopkWaves - 1) / kTopkWaves + 63) & ~63;
        const int lo = wid * S, hi = min(n, lo + S);
        uint32_t cnt = 0;
        for (int i0 = lo; i0 < hi; i0 += 64) {
            const int i = i0 + lane;
            cnt += (uint32_t)__popcll(__ballot(i < hi && order_key(x[i]) == T));
        }
        if (lane == 0) sh.wave_tot[wid] = cnt;
        __syncthreads();
        uint32_t rank = 0;
        for (int w = 0; w < wid; ++w) rank += sh.wave_tot[w];
        const uint64_t below = (1ull << lane) - 1;
        for (int i0 = lo; i0 < hi; i0 += 64) {
            const int i = i0 + lane;
            const uint32_t key = i < hi ? order_key(x[i]) : 0u;
            const uint64_t eq = __ballot(i < hi && key == T);
            if (i < hi && key > T) put(sh, atomicAdd(&sh.gt, 1u), key, i);
            const uint32_t r = rank + (uint32_t)__popcll(eq & below);
            if (i < hi && key == T && r < remaining) put(sh, kgt + r, key, i);
            rank += (uint32_t)__popcll(eq);
        }
    }
    __syncthreads();
    sort_and_write(sh, k, k, out_vals, out_idx);
}

// Rows whose 16-byte chunks number at most 16 x 1024 (n + 3 <= 65536): the
// row is read once as 16-byte chunks from its 16-byte-aligned base, thread t
// holding chunks t + 1024 q (q < 16), i.e. indices 4 (t + 1024 q) + c - s
// where s = the row start's float offset within its chunk.  Key 0 (the bit
// pattern of a NaN, which rows do not hold) marks slots outside the row.
__global__ __launch_bounds__(kTopkThreads) void topk_reg_kernel(const float* __restrict__ logits, int n, int k,
                                                                float* __restrict__ out_vals,
                                                                int* __restrict__ out_idx) {
    __shared__ TopkShared sh;
    const float* x = logits + (size_t)blockIdx.x * n;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int s = (int)(((uintptr_t)x & 15u) >> 2);
    const float4* x4 = reinterpret_cast<const float4*>(x - s);
    // chunks wholly inside the row: [cf, cl]; the (at most two) others that
    // touch it are read element by element by the one lane that holds each
    const int cf = s == 0 ? 0 : 1, cl = (n + s) / 4 - 1;
    uint32_t key[kTopkRegPer];
#pragma unroll
    for (int q = 0; q < kTopkRegPer / 4; ++q) {
        const int c = (int)threadIdx.x + q * kTopkThreads, e0 = 4 * c - s;
        // branch-free for whole chunks, so all 16 loads are in flight together
        float4 v = cf <= cl ? x4[min(max(c, cf), cl)] : make_float4(0.f, 0.f, 0.f, 0.f);
        const bool whole = c >= cf && c <= cl;
        if (!whole && e0 < n && e0 + 3 >= 0) {
            v.x = e0 >= 0 && e0 < n ? x[e0] : 0.f;
            v.y = e0 + 1 >= 0 && e0 + 1 < n ? x[e0 + 1] : 0.f;
            v.z = e0 + 2 >= 0 && e0 + 2 < n ? x[e0 + 2] : 0.f;
            v.w = e0 + 3 < n ? x[e0 + 3] : 0.f;
        }
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) key[4 * q + u] = e0 + u >= 0 && e0 + u < n ? order_key(e[u]) : 0u;
    }
    // index of key[j]: one base per thread plus a constant per slot (written
    // this way the compiler does not keep 64 precomputed indices live)
    const int ibase = 4 * (int)threadIdx.x - s;
    auto index = [&](int j) { return ibase + (j >> 2) * (4 * kTopkThreads) + (j & 3); };

    // Lower bound M: the k-th largest of the 1024 per-thread maxima (k <=
    // 1024).  Those k maxima are k keys >= M, so every key of the top k is
    // >= M.  The keys >= M (typically a few more than k) are gathered into
    // LDS and ranked there; only when more than kTopkCand keys reach M (many
    // ties, or k near 1024) is the row streamed through the radix select.
    // (every loop over key[] is fully unrolled: an early exit would leave the
    // array indexed at run time, i.e. in scratch memory)
    uint32_t tmax = 0;
#pragma unroll
    for (int j = 0; j < kTopkRegPer; ++j) tmax = max(tmax, key[j]);
    uint32_t remaining, eqcount;
    const uint32_t M = radix_kth(
        sh, (uint32_t)k,
        [&](uint32_t hmask, uint32_t prefix, int shift) {
            hist_add(sh.hist, (tmax & hmask) == prefix, (tmax >> shift) & 255u, lane);
        },
        lane, wid, remaining, eqcount);
    if (threadIdx.x == 0) sh.gt = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kTopkRegPer; ++j)
        if (key[j] != 0u && key[j] >= M) {
            const uint32_t slot = atomicAdd(&sh.gt, 1u);
            if (slot < (uint32_t)kTopkCand) put(sh, slot, key[j], index(j));
        }
    __syncthreads();
    const uint32_t cnt = sh.gt;
    if (cnt > (uint32_t)kTopkCand) {  // uniform
        __syncthreads();  // all have read the count before the stream resets it
        topk_stream_row(sh, x, n, k, out_vals, out_idx, lane, wid);
        return;
    }
    // rank sort: a candidate's place is the number of candidates before it
    // (larger key, or equal key and lower index); places are distinct
    for (int t = threadIdx.x; t < (int)cnt; t += kTopkThreads) {
        const uint32_t kt = sh.ckey[t];
        const int it = sh.cidx[t];
        int rank = 0;
        for (int u = 0; u < (int)cnt; ++u) {
            const uint32_t ku = sh.ckey[u];
            rank += ku > kt || (ku == kt && sh.cidx[u] < it);
        }
        if (rank < k) {
            out_vals[(size_t)blockIdx.x * k + rank] = key_value(kt);
            out_idx[(size_t)blockIdx.x * k + rank] = it;
        }
    }
}

// Longer rows.
__global__ __launch_bounds__(kTopkThreads) void topk_stream_kernel(const float* __restrict__ logits, int n, int k,
                                                                   float* __restrict__ out_vals,
                                                                   int* __restrict__ out_idx) {
    __shared__ TopkShared sh;
    topk_stream_row(sh, logits + (size_t)blockIdx.x * n, n, k, out_vals, out_idx, threadIdx.x & 63,
                    threadIdx.x >> 6);
}

}  // namespace

void launch_topk(int rows, const float* logits, int n, int k, float* out_vals, int* out_idx, hipStream_t s) {
    if (rows == 0) return;
    if (n + 3 <= kTopkRegPer * kTopkThreads)
        topk_reg_kernel<<<rows, kTopkThreads, 0, s>>>(logits, n, k, out_vals, out_idx);
    else
        topk_stream_kernel<<<rows, kTopkThreads, 0, s>>>(logits, n, k, out_vals, out_idx);
}

}  // namespace ie
