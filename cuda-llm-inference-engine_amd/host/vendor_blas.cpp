// vendor_blas.cpp — the fp32 GEMM of the engine's vendor comparison backend
// (the reference's CUBLAS_FP32 backend, src/gpt2_engine.cu:530-610, which
// calls cublasSgemm on fp32 [K, N] weights).  Here rocBLAS's rocblas_sgemm,
// loaded with dlopen on first use so that the library itself keeps no link
// dependency on rocBLAS (only engines built with that backend load it).
#include "vendor_blas.h"

#include <dlfcn.h>

#include <mutex>
#include <stdexcept>
#include <string>

namespace ie {
namespace {

// rocblas.h types, restated so the header need not be on the include path of
// every translation unit: handles and streams are opaque pointers, the
// operation enum's "none" value is 111, the status enum's success is 0.
using rb_handle = void*;
using rb_status = int;
constexpr int kRbOpNone = 111;
using create_fn = rb_status (*)(rb_handle*);
using destroy_fn = rb_status (*)(rb_handle);
using set_stream_fn = rb_status (*)(rb_handle, hipStream_t);
using sgemm_fn = rb_status (*)(rb_handle, int, int, int, int, int, const float*, const float*, int, const float*,
                               int, const float*, float*, int);

struct Api {
    void* lib = nullptr;
    create_fn create = nullptr;
    destroy_fn destroy = nullptr;
    set_stream_fn set_stream = nullptr;
    sgemm_fn sgemm = nullptr;
};

const Api& api() {
    static std::once_flag once;
    static Api a;
    static std::string err;
    std::call_once(once, [] {
        for (const char* name : {"librocblas.so.5", "librocblas.so", "/opt/rocm/lib/librocblas.so.5"}) {
            a.lib = dlopen(name, RTLD_NOW | RTLD_LOCAL);
            if (a.lib) break;
        }
        if (!a.lib) {
            err = std::string("cannot load rocBLAS: ") + dlerror();
            return;
        }
        a.create = reinterpret_cast<create_fn>(dlsym(a.lib, "rocblas_create_handle"));
        a.destroy = reinterpret_cast<destroy_fn>(dlsym(a.lib, "rocblas_destroy_handle"));
        a.set_stream = reinterpret_cast<set_stream_fn>(dlsym(a.lib, "rocblas_set_stream"));
        a.sgemm = reinterpret_cast<sgemm_fn>(dlsym(a.lib, "rocblas_sgemm"));
        if (!a.create || !a.destroy || !a.set_stream || !a.sgemm) err = "rocBLAS lacks a required symbol";
    });
    if (!err.empty()) throw std::runtime_error(err);
    return a;
}

}  // namespace

VendorSgemm::VendorSgemm(hipStream_t stream) {
    const Api& a = api();
    rb_handle h = nullptr;
    if (a.create(&h) != 0 || !h) throw std::runtime_error("rocblas_create_handle failed");
    if (a.set_stream(h, stream) != 0) {
        a.destroy(h);
        throw std::runtime_error("rocblas_set_stream failed");
    }
    handle_ = h;
}

VendorSgemm::~VendorSgemm() {
    if (handle_) (void)api().destroy(handle_);
}

// Row-major C[M, N] = A[M, K] . W[K, N]: in column-major terms
// C^T[N, M] = W^T[N, K] . A^T[K, M], the reference's own call shape
// (cublasSgemm(N, N, n = N, m = M, k = K, W, ldw = N, A, lda = K, C, ldc = N)).
void VendorSgemm::rowmajor(int M, int N, int K, const float* A, const float* W, float* C) {
    const float alpha = 1.0f, beta = 0.0f;
    if (api().sgemm(handle_, kRbOpNone, kRbOpNone, N, M, K, &alpha, W, N, A, K, &beta, C, N) != 0)
        throw std::runtime_error("rocblas_sgemm failed");
}

}  // namespace ie
