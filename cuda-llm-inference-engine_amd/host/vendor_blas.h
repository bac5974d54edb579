// vendor_blas.h — fp32 GEMM from the vendor library (rocBLAS, loaded on first
// use) for the engine's fp32 comparison backend.
#ifndef IE_VENDOR_BLAS_H
#define IE_VENDOR_BLAS_H

#include <hip/hip_runtime.h>

namespace ie {

class VendorSgemm {
public:
    explicit VendorSgemm(hipStream_t stream);  // throws std::runtime_error
    ~VendorSgemm();
    VendorSgemm(const VendorSgemm&) = delete;
    VendorSgemm& operator=(const VendorSgemm&) = delete;
    // Row-major C[M, N] = A[M, K] . W[K, N] (W in the exporter's fp32 [K, N]
    // layout), on the stream given at construction.
    void rowmajor(int M, int N, int K, const float* A, const float* W, float* C);

private:
    void* handle_ = nullptr;
};

}  // namespace ie

#endif
