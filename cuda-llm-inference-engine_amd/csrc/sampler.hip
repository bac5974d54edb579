// Device half of the top-k sampler (src/sampler.cu:16-45): the k largest
// logits of each row with their indices, sorted by value descending and, for
// equal values, by index ascending (std::partial_sort leaves the order of
// equal values unspecified; this is the order a stable sort gives).  Only
// these k pairs cross PCIe; the reference copies the whole row (201 KB for
// GPT-2) and partial-sorts it on the host.  The draw itself (temperature
// softmax over the k values and the rand() threshold) stays on the host,
// where it is the same float arithmetic as the reference's.
//
// One 1024-thread workgroup per row:
//   1. radix select of the k-th largest order key, 8 bits per pass from the
//      top.  The histogram lives in LDS; logits cluster in a few exponent
//      bins, so each wave instruction adds its leading lane's bin with one
//      atomic and only the other lanes' bins lane by lane;
//   2. gather: every key above the threshold, plus the lowest-index keys equal
//      to it (ranked in index order only when some equal keys are left out),
//      k entries in LDS;
//   3. bitonic sort of the k entries (padded to a power of two) in LDS.
// Rows of up to 64 x 1024 logits (GPT-2's 50257 among them) are read once
// into registers, 64 keys per thread, and every pass runs from there; longer
// rows are streamed from memory (L2 after the first pass) with 8 loads in
// flight per thread.
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
    uint32_t scan[kTopkThreads];  // tie ranks: counts per (column, wave), then their exclusive prefix
    uint64_t emask[kTopkThreads];  // tie ranks: lanes holding a key equal to the threshold, per (column, wave)
    uint32_t wave_tot[kTopkWaves];
    uint32_t ckey[kTopkMax];
    int cidx[kTopkMax];
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

// Exclusive prefix of sh.scan[0 .. 1024) in place (all threads).
__device__ __forceinline__ void block_exclusive_scan(TopkShared& sh, int lane, int wid) {
    const uint32_t v = sh.scan[threadIdx.x];
    uint32_t incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off, 64);
        if (lane >= off) incl += t;
    }
    if (lane == 63) sh.wave_tot[wid] = incl;
    __syncthreads();
    uint32_t base = 0;
    for (int w = 0; w < wid; ++w) base += sh.wave_tot[w];
    sh.scan[threadIdx.x] = base + incl - v;
    __syncthreads();
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

// Bitonic sort of the k gathered entries (larger key first, then lower
// index) and the output row.
__device__ __forceinline__ void sort_and_write(TopkShared& sh, int k, float* out_vals, int* out_idx) {
    int KP = 1;
    while (KP < k) KP <<= 1;
    for (int t = k + threadIdx.x; t < KP; t += kTopkThreads) put(sh, t, 0u, INT_MAX);
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

// Rows of n <= 64 x 1024: thread t holds keys of indices t + 1024 j; key 0
// (the bit pattern of a NaN, which rows do not hold) marks indices past n.
__global__ __launch_bounds__(kTopkThreads) void topk_reg_kernel(const float* __restrict__ logits, int n, int k,
                                                                float* __restrict__ out_vals,
                                                                int* __restrict__ out_idx) {
    __shared__ TopkShared sh;
    const float* x = logits + (size_t)blockIdx.x * n;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    uint32_t key[kTopkRegPer];
#pragma unroll
    for (int j = 0; j < kTopkRegPer; ++j) {
        const int i = (int)threadIdx.x + j * kTopkThreads;
        key[j] = i < n ? order_key(x[i]) : 0u;
    }
    auto valid = [&](int j) { return key[j] != 0u; };

    // Lower bound M: the k-th largest of the 1024 per-thread maxima (k <=
    // 1024).  Those k maxima are k keys >= M, so every key of the top k is
    // >= M, and only keys >= M (typically a few more than k) reach the
    // histogram below: GPT-2's logits otherwise spread over some 60 bins in
    // the second pass and nearly every key costs an LDS atomic.
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
    // (every loop over key[] is fully unrolled: an early exit would leave the
    // array indexed at run time, i.e. in scratch memory)
    const uint32_t prefix = radix_kth(
        sh, (uint32_t)k,
        [&](uint32_t hmask, uint32_t prefix, int shift) {
#pragma unroll
            for (int j = 0; j < kTopkRegPer; ++j)
                hist_add(sh.hist, valid(j) && key[j] >= M && (key[j] & hmask) == prefix, (key[j] >> shift) & 255u,
                         lane);
        },
        lane, wid, remaining, eqcount);
    const uint32_t T = prefix, kgt = (uint32_t)k - remaining;

    if (threadIdx.x == 0) sh.gt = sh.eq = 0;
    if (eqcount == remaining) {  // every key equal to T is taken
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kTopkRegPer; ++j)
            if (valid(j) && key[j] >= T)
                put(sh, key[j] > T ? atomicAdd(&sh.gt, 1u) : kgt + atomicAdd(&sh.eq, 1u), key[j], threadIdx.x + j * kTopkThreads);
    } else {
        // rank of each equal key in index order: index t + 1024 j orders by
        // column j, then wave, then lane
        const uint64_t below = (1ull << lane) - 1;
        sh.scan[threadIdx.x] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kTopkRegPer; ++j) {
            const uint64_t m = __ballot(valid(j) && key[j] == T);
            if (lane == 0) {
                sh.scan[j * kTopkWaves + wid] = (uint32_t)__popcll(m);
                sh.emask[j * kTopkWaves + wid] = m;  // kept in LDS, not in 64 scalar register pairs
            }
        }
        __syncthreads();
        block_exclusive_scan(sh, lane, wid);
#pragma unroll
        for (int j = 0; j < kTopkRegPer; ++j) {
            const bool eq = valid(j) && key[j] == T;
            const uint64_t m = sh.emask[j * kTopkWaves + wid];
            const uint32_t r = sh.scan[j * kTopkWaves + wid] + (uint32_t)__popcll(m & below);
            if (valid(j) && key[j] > T) put(sh, atomicAdd(&sh.gt, 1u), key[j], threadIdx.x + j * kTopkThreads);
            if (eq && r < remaining) put(sh, kgt + r, key[j], threadIdx.x + j * kTopkThreads);
        }
    }
    __syncthreads();
    sort_and_write(sh, k, out_vals, out_idx);
}

// Longer rows, streamed: every pass re-reads the row (L2 after the first).
__global__ __launch_bounds__(kTopkThreads) void topk_stream_kernel(const float* __restrict__ logits, int n, int k,
                                                                   float* __restrict__ out_vals,
                                                                   int* __restrict__ out_idx) {
    __shared__ TopkShared sh;
    const float* x = logits + (size_t)blockIdx.x * n;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    // visits every index in rounds of kTopkUnroll coalesced loads per thread
    auto for_each = [&](auto&& f) {
        for (int base = threadIdx.x; base < n; base += kTopkThreads * kTopkUnroll) {
            float v[kTopkUnroll];
#pragma unroll
            for (int u = 0; u < kTopkUnroll; ++u) {
                const int i = base + u * kTopkThreads;
                v[u] = i < n ? x[i] : 0.0f;
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
    sort_and_write(sh, k, out_vals, out_idx);
}

}  // namespace

void launch_topk(int rows, const float* logits, int n, int k, float* out_vals, int* out_idx, hipStream_t s) {
    if (rows == 0) return;
    if (n <= kTopkRegPer * kTopkThreads)
        topk_reg_kernel<<<rows, kTopkThreads, 0, s>>>(logits, n, k, out_vals, out_idx);
    else
        topk_stream_kernel<<<rows, kTopkThreads, 0, s>>>(logits, n, k, out_vals, out_idx);
}

}  // namespace ie
