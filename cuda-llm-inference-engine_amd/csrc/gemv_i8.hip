// gemv_i8.hip — INT8 GEMV for decode-sized M (1..16) on gfx950.
//
// Computes the same sum as the reference's K14 dp4a GEMM
// (kernels/quantization/14_int8_gemm.cu:96-140) followed by its epilogue
// (:142-169), for C[M,N] = A[M,K] * BT[N,K]^T with M <= 16.
//
// The weights BT dominate the traffic (N*K bytes, read once), so the kernel is
// laid out for HBM streaming:
//   * a workgroup owns 16 output features; each wave owns 4 of them and each
//     16-lane DPP row owns one, so a wave's load instruction fetches 4 rows x
//     256 contiguous bytes with 16-byte vector loads;
//   * activations (M*K bytes, tiny) are staged in LDS in 2 KiB-of-K chunks and
//     read back with 16-byte LDS loads, so the weight stream is the only
//     global traffic;
//   * v_dot4_i32_i8 accumulates four byte products per instruction in exact
//     int32 (sum order does not matter for integers);
//   * the 16 partial sums of a feature are combined with four DPP row
//     rotations (no LDS round trip), then lane m of the row stores output m.
// Requires K % 16 == 0 and 16-byte aligned A/BT; other shapes use the generic
// kernel at the end of this file.
#include "device_util.h"
#include "epilogue.h"
#include "ie_internal.h"

namespace ie {
namespace {

constexpr int kRowsPerWG = 16;
constexpr int kChunk = 128;  // 16-byte columns of A per LDS chunk (2 KiB of K)

template <int MT, int EPI>
__global__ __launch_bounds__(256) void gemv_i8_kernel(
    int M, int N, int K, const int32_t* __restrict__ A,
    const int32_t* __restrict__ BT, const float* __restrict__ sA,
    const float* __restrict__ sB, const float* bias, const float* residual,
    void* C) {
    __shared__ i32x4 a_lds[MT * kChunk];
    const int lane = threadIdx.x & 63;
    const int li = lane & 15;
    const int n = blockIdx.x * kRowsPerWG + (threadIdx.x >> 6) * 4 + (lane >> 4);
    const bool row_ok = n < N;
    const int K16 = K >> 4;
    const i32x4* w = reinterpret_cast<const i32x4*>(BT) + (size_t)(row_ok ? n : 0) * K16;
    const i32x4* a4 = reinterpret_cast<const i32x4*>(A);

    int32_t acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0;

    for (int c0 = 0; c0 < K16; c0 += kChunk) {
        const int cw = min(kChunk, K16 - c0);
        __syncthreads();
        for (int i = threadIdx.x; i < MT * cw; i += 256) {
            const int m = i / cw;
            const int c = i - m * cw;
            const int mm = m < M ? m : M - 1;  // padded rows re-read a real row
            a_lds[m * kChunk + c] = a4[(size_t)mm * K16 + c0 + c];
        }
        __syncthreads();
        if (row_ok) {
#pragma unroll 4
            for (int c = li; c < cw; c += 16) {
                const i32x4 wv = w[c0 + c];
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const i32x4 av = a_lds[m * kChunk + c];
                    int32_t s = acc[m];
                    s = dot4_i8(wv.x, av.x, s);
                    s = dot4_i8(wv.y, av.y, s);
                    s = dot4_i8(wv.z, av.z, s);
                    s = dot4_i8(wv.w, av.w, s);
                    acc[m] = s;
                }
            }
        }
    }

    int32_t mine = 0;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int32_t t = row16_sum(acc[m]);
        if (li == m) mine = t;
    }
    if (row_ok && li < M) {
        const size_t idx = (size_t)li * N + n;
        float sa = 0.0f, sb = 0.0f;
        if constexpr (EPI != IE_EPI_I32) {
            sa = sA[li];
            sb = sB[n];
        }
        store_epilogue<EPI>(C, idx, mine, sa, sb, bias, residual, n);
    }
}

// Any K % 4 == 0 and any alignment: one thread per output element.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_i8_generic_kernel(
    int M, int N, int K, const int32_t* __restrict__ A,
    const int32_t* __restrict__ BT, const float* __restrict__ sA,
    const float* __restrict__ sB, const float* bias, const float* residual,
    void* C) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (size_t)M * N) return;
    const int m = (int)(idx / N);
    const int n = (int)(idx - (size_t)m * N);
    const int K4 = K >> 2;
    const int32_t* a = A + (size_t)m * K4;
    const int32_t* b = BT + (size_t)n * K4;
    int32_t s = 0;
    for (int k = 0; k < K4; ++k) s = dot4_i8(a[k], b[k], s);
    float sa = 0.0f, sb = 0.0f;
    if constexpr (EPI != IE_EPI_I32) {
        sa = sA[m];
        sb = sB[n];
    }
    store_epilogue<EPI>(C, idx, s, sa, sb, bias, residual, n);
}

template <int EPI>
struct GemvLaunch {
    static void run(const GemmArgs& a, hipStream_t s) {
        const dim3 grid((a.N + kRowsPerWG - 1) / kRowsPerWG);
#define IE_GEMV(MT)                                                                 \
    gemv_i8_kernel<MT, EPI><<<grid, 256, 0, s>>>(a.M, a.N, a.K, a.A, a.BT, a.sA, a.sB, \
                                                 a.bias, a.residual, a.C)
        if (a.M <= 1) IE_GEMV(1);
        else if (a.M <= 2) IE_GEMV(2);
        else if (a.M <= 4) IE_GEMV(4);
        else if (a.M <= 8) IE_GEMV(8);
        else IE_GEMV(16);
#undef IE_GEMV
    }
};

template <int EPI>
struct GenericLaunch {
    static void run(const GemmArgs& a, hipStream_t s) {
        const size_t total = (size_t)a.M * a.N;
        const unsigned blocks = (unsigned)((total + 255) / 256);
        gemm_i8_generic_kernel<EPI><<<blocks, 256, 0, s>>>(a.M, a.N, a.K, a.A, a.BT, a.sA,
                                                           a.sB, a.bias, a.residual, a.C);
    }
};

bool vec_ok(const GemmArgs& a) {
    return (a.K % 16) == 0 && ((uintptr_t)a.A % 16) == 0 && ((uintptr_t)a.BT % 16) == 0;
}

}  // namespace

void launch_gemv_i8(const GemmArgs& a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    if (vec_ok(a))
        dispatch_epilogue<GemvLaunch>(a.epi, a, s);
    else
        dispatch_epilogue<GenericLaunch>(a.epi, a, s);
}

// Used by the MFMA path for shapes its vector loads cannot cover.
void launch_gemm_i8_generic(const GemmArgs& a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    dispatch_epilogue<GenericLaunch>(a.epi, a, s);
}

}  // namespace ie
