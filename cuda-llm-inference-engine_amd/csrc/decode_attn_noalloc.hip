// decode_attn_noalloc.hip — ie_decode_attn_noalloc (include/ie_amd.h): split-K
// paged decode attention whose split partials live in a file-scope device
// array instead of a caller workspace, for callers that cannot allocate.
//
// The array is a device symbol: in host code its name is only a stand-in, so
// its device address is looked up once per device (hipGetSymbolAddress with
// that device current) and only that address reaches kernels.  Each device
// holds its own copy for the life of the process.  Every call on a device
// shares it; the kernels write every split slot before the merge reads it, so
// nothing needs clearing between calls, but overlapping calls race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "ie_internal.h"

static __device__ __align__(256) float scratch[IE_DECODE_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
float* g_scratch[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up on first use.
int scratch_on_current_device(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return ie::fail(IE_ERR_HIP, "decode_attn_noalloc: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return ie::fail(IE_ERR_UNSUPPORTED, "decode_attn_noalloc: device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return ie::fail(IE_ERR_HIP, "decode_attn_noalloc: scratch address on device %d: %s", dev,
                            hipGetErrorString(e));
        g_scratch[dev] = static_cast<float*>(p);
    }
    *out = g_scratch[dev];
    return IE_OK;
}

}  // namespace

namespace ie {
int decode_scratch_init() {
    float* p = nullptr;
    return scratch_on_current_device(&p);
}
}  // namespace ie

extern "C" int ie_decode_attn_noalloc(int B, int H_q, int H_kv, int d, const float* Q, const void* k_cache,
                                      const void* v_cache, int kv_dtype, const int* block_table,
                                      const int* context_lens, int max_context_len, int block_size,
                                      int num_blocks_per_seq, float* O, int num_splits, ie_stream_t stream) {
    size_t need = 0;
    int S = 1;
    const int st = ie::check_decode_attn(B, H_q, H_kv, d, Q, k_cache, v_cache, kv_dtype, block_table, context_lens,
                                         max_context_len, block_size, num_blocks_per_seq, O, num_splits, &need, &S);
    if (st != IE_OK || B == 0) return st;
    if (need > IE_DECODE_SCRATCH_BYTES)
        return ie::fail(IE_ERR_WORKSPACE,
                        "decode_attn_noalloc: %zu bytes of split partials (B*H_q*splits*(d+2)*4 with %d splits) "
                        "exceed the %zu-byte scratch",
                        need, S, (size_t)IE_DECODE_SCRATCH_BYTES);
    float* ws = nullptr;
    const int sst = scratch_on_current_device(&ws);
    if (sst != IE_OK) return sst;
    return ie_decode_attn(B, H_q, H_kv, d, Q, k_cache, v_cache, kv_dtype, block_table, context_lens, max_context_len,
                          block_size, num_blocks_per_seq, O, ws, IE_DECODE_SCRATCH_BYTES, num_splits, stream);
}
