// Y = X W^T + b through rocBLAS: a plain library GEMM (weights are the
// reference's [out_features, in_features] row-major layout, README.md:195-210).
//
// Row-major Y[M,N] = X[M,K] W[N,K]^T is, read column-major, Y^T = W^T' X^T'
// with W's buffer as a K x N column-major matrix used transposed and X's as
// K x M used as is: one "TN" GEMM, m = N, n = M, k = K, fp32 accumulation.
#include "launch.hpp"

#include "../device/hip_check.hpp"

#include <rocblas/rocblas.h>

#include <unordered_map>

namespace llaisys::kernels {

namespace {

#define ROCBLAS_CHECK(expr)                                                                  \
    do {                                                                                     \
        rocblas_status s__ = (expr);                                                         \
        if (s__ != rocblas_status_success) LLAISYS_RAISE("rocBLAS error " << rocblas_status_to_string(s__) << " from " #expr); \
    } while (0)

// One handle per (thread, device); never destroyed (handles outlive any
// thread-exit ordering against the HIP runtime's own teardown).
rocblas_handle handleFor() {
    thread_local std::unordered_map<int, rocblas_handle> handles;
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    auto it = handles.find(dev);
    if (it != handles.end()) return it->second;
    rocblas_handle h = nullptr;
    ROCBLAS_CHECK(rocblas_create_handle(&h));
    handles.emplace(dev, h);
    return h;
}

rocblas_datatype typeOf(ElemType t) {
    switch (t) {
    case ElemType::F32: return rocblas_datatype_f32_r;
    case ElemType::F16: return rocblas_datatype_f16_r;
    case ElemType::BF16: return rocblas_datatype_bf16_r;
    }
    return rocblas_datatype_f32_r;
}

} // namespace

void linear(void *y, const void *x, const void *w, const void *bias, ElemType t, int M, int N, int K, void *stream,
            bool accumulate) {
    if (M == 0 || N == 0) return;
    rocblas_handle h = handleFor();
    ROCBLAS_CHECK(rocblas_set_stream(h, static_cast<hipStream_t>(stream)));
    // The bias enters as C (Y preset to bias, beta = 1) so the result is rounded once.
    if (bias) {
        if (accumulate) {
            addBias(y, bias, t, size_t(M), size_t(N), stream);
        } else {
            fillRows(y, bias, t, size_t(M), size_t(N), stream);
        }
    }
    const float alpha = 1.f, beta = (accumulate || bias) ? 1.f : 0.f;
    const rocblas_datatype dt = typeOf(t);
    ROCBLAS_CHECK(rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, N, M, K, &alpha, w, dt, K, x,
                                  dt, K, &beta, y, dt, N, y, dt, N, rocblas_datatype_f32_r, rocblas_gemm_algo_standard,
                                  0, 0));
}

} // namespace llaisys::kernels
