// epilogue.h — dequantization epilogues of the INT8 GEMM kernels.
//
// kernels/quantization/14_int8_gemm.cu:142-169 of the reference:
//   t = (float)acc * scale_A[m]                        (left to right, :154)
//   Plain         C = t * scale_B[n]
//   BiasOnly      C = t * scale_B[n] + bias[n]
//   BiasGELU      v = t * scale_B[n] + bias[n];
//                 C = 0.5 v (1 + tanh(0.7978845608 (v + 0.044715 v^3)))
//   BiasResidual  C = t * scale_B[n] + bias[n] + residual[m][n]
// The reference's compiler fuses "t * sB + bias" and "v + 0.044715 v^3" into
// single-rounding multiply-adds; they are written as fmaf here so the result
// does not depend on this compiler's contraction choices.  GELU constants:
// sqrt(2/pi) and 0.044715 from the tanh approximation of Hendrycks & Gimpel.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "ie_amd.h"

namespace ie {

// NT = true writes C with non-temporal stores: used where C is far larger
// than the caches (it would otherwise evict the operand panels other
// workgroups are still reading).
template <int EPI, bool NT = false>
__device__ __forceinline__ void store_epilogue(void* C, size_t idx, int32_t acc,
                                               float sa, float sb,
                                               const float* bias,
                                               const float* residual, int n) {
    if constexpr (EPI == IE_EPI_I32) {
        if constexpr (NT)
            __builtin_nontemporal_store(acc, static_cast<int32_t*>(C) + idx);
        else
            static_cast<int32_t*>(C)[idx] = acc;
    } else {
        const float t = (float)acc * sa;
        float out;
        if constexpr (EPI == IE_EPI_PLAIN) {
            out = t * sb;
        } else if constexpr (EPI == IE_EPI_BIAS) {
            out = fmaf(t, sb, bias[n]);
        } else if constexpr (EPI == IE_EPI_BIAS_GELU) {
            const float v = fmaf(t, sb, bias[n]);
            const float x3 = v * v * v;
            const float u = 0.7978845608f * fmaf(0.044715f, x3, v);
            out = 0.5f * v * (1.0f + tanhf(u));
        } else {
            out = fmaf(t, sb, bias[n]) + residual[idx];
        }
        if constexpr (NT)
            __builtin_nontemporal_store(out, static_cast<float*>(C) + idx);
        else
            static_cast<float*>(C)[idx] = out;
    }
}

// Runtime-to-compile-time epilogue dispatch.
template <template <int> class F, typename... Args>
inline void dispatch_epilogue(int epi, Args&&... args) {
    switch (epi) {
        case IE_EPI_PLAIN: F<IE_EPI_PLAIN>::run(args...); break;
        case IE_EPI_BIAS: F<IE_EPI_BIAS>::run(args...); break;
        case IE_EPI_BIAS_GELU: F<IE_EPI_BIAS_GELU>::run(args...); break;
        case IE_EPI_BIAS_RESIDUAL: F<IE_EPI_BIAS_RESIDUAL>::run(args...); break;
        default: F<IE_EPI_I32>::run(args...); break;
    }
}

}  // namespace ie
