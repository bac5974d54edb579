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

#include "device_util.h"
#include "ie_amd.h"
#include "ie_internal.h"

namespace ie {

// The epilogue value for a float output, from the bias and residual values.
template <int EPI>
__device__ __forceinline__ float epilogue_value(int32_t acc, float sa, float sb, float bias_v,
                                                float res_v) {
    const float t = (float)acc * sa;
    if constexpr (EPI == IE_EPI_PLAIN) {
        return t * sb;
    } else if constexpr (EPI == IE_EPI_BIAS_GELU) {
        const float v = fmaf(t, sb, bias_v);
        const float x3 = v * v * v;
        const float u = 0.7978845608f * fmaf(0.044715f, x3, v);
        return 0.5f * v * (1.0f + tanhf(u));
    } else if constexpr (EPI == IE_EPI_BIAS_RESIDUAL) {
        return fmaf(t, sb, bias_v) + res_v;
    } else {  // IE_EPI_BIAS and the routed bias epilogues
        return fmaf(t, sb, bias_v);
    }
}

// Stores one output with its epilogue, the bias and residual values given.
// NT = true writes C with non-temporal stores: used where C is far larger
// than the caches (it would otherwise evict the operand panels other
// workgroups are still reading).
template <int EPI, bool NT = false>
__device__ __forceinline__ void store_epilogue_v(void* C, size_t idx, int32_t acc, float sa,
                                                 float sb, float bias_v, float res_v) {
    if constexpr (EPI == IE_EPI_I32) {
        if constexpr (NT)
            __builtin_nontemporal_store(acc, static_cast<int32_t*>(C) + idx);
        else
            static_cast<int32_t*>(C)[idx] = acc;
    } else {
        const float out = epilogue_value<EPI>(acc, sa, sb, bias_v, res_v);
        if constexpr (NT)
            __builtin_nontemporal_store(out, static_cast<float*>(C) + idx);
        else
            static_cast<float*>(C)[idx] = out;
    }
}

// As store_epilogue_v, reading bias[n] and residual[idx] as the epilogue needs.
template <int EPI, bool NT = false>
__device__ __forceinline__ void store_epilogue(void* C, size_t idx, int32_t acc,
                                               float sa, float sb,
                                               const float* bias,
                                               const float* residual, int n) {
    float bias_v = 0.0f, res_v = 0.0f;
    if constexpr (EPI == IE_EPI_BIAS || EPI == IE_EPI_BIAS_GELU || EPI == IE_EPI_BIAS_RESIDUAL)
        bias_v = bias[n];
    if constexpr (EPI == IE_EPI_BIAS_RESIDUAL) res_v = residual[idx];
    store_epilogue_v<EPI, NT>(C, idx, acc, sa, sb, bias_v, res_v);
}

// kEpiQKVRoute: one routed store of the bias epilogue's value for row m,
// column n, the row's cache slot given (row_slot[m], gathered before the
// stores like the other epilogue operands).
__device__ __forceinline__ void route_store(const QkvRoute& r, int m, int n, int slot, int32_t acc, float sa,
                                            float sb, float bias_v) {
    const float v = epilogue_value<IE_EPI_BIAS>(acc, sa, sb, bias_v, 0.0f);
    if (n < r.d) {
        r.q[(size_t)m * r.d + n] = v;
        return;
    }
    const bool is_k = n < 2 * r.d;
    const size_t i = (size_t)slot * r.d + (is_k ? n - r.d : n - 2 * r.d);
    void* base = is_k ? r.kc : r.vc;
    if (r.kv_dtype == IE_KV_BF16)
        static_cast<uint16_t*>(base)[i] = f32_to_bf16_rne(v);
    else
        static_cast<float*>(base)[i] = v;
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
