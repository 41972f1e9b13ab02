// Contiguous causal GQA attention: the reference's self_attention op
// (spec README.md:244-266; formula test/ops/self_attention.py:11-28).
//
//   out[i, h, :] = sum_j softmax_j(scale * q[i,h] . k[j, h/G]) v[j, h/G],
//   keys j <= i + S - L (bottom-right causal alignment), G = nh / nkvh.
//
// One wave per (query, head). Keys stream in chunks of 64, one key per lane
// for the scores; the value pass puts output dims on lanes. Online softmax in
// base 2, fp32 throughout, one rounding to the output type at the end.
// This is the general path (any head dim up to 256, f32/f16/bf16); the paged
// kernels carry the Qwen2 decode and prefill traffic.
#include "launch.hpp"

#include "../device/hip_check.hpp"

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

namespace llaisys::kernels {

namespace {

constexpr int kMaxDim = 256;

template <typename T> __device__ __forceinline__ float toF32(T x);
template <> __device__ __forceinline__ float toF32<float>(float x) { return x; }
template <> __device__ __forceinline__ float toF32<__half>(__half x) { return __half2float(x); }
template <> __device__ __forceinline__ float toF32<__hip_bfloat16>(__hip_bfloat16 x) { return __bfloat162float(x); }

template <typename T> __device__ __forceinline__ T fromF32(float x);
template <> __device__ __forceinline__ float fromF32<float>(float x) { return x; }
template <> __device__ __forceinline__ __half fromF32<__half>(float x) { return __float2half_rn(x); }
template <> __device__ __forceinline__ __hip_bfloat16 fromF32<__hip_bfloat16>(float x) { return __float2bfloat16(x); }

__device__ __forceinline__ float waveMax(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}
__device__ __forceinline__ float waveSum(float x) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

template <typename T>
__global__ void __launch_bounds__(64) selfAttentionKernel(T *__restrict__ out, const T *__restrict__ q,
                                                          const T *__restrict__ k, const T *__restrict__ v, int L,
                                                          int S, int nh, int nkvh, int d, int dv, float scale_log2) {
    __shared__ float qs[kMaxDim];
    __shared__ float ps[64];
    const int i = blockIdx.x;
    const int h = blockIdx.y;
    const int lane = threadIdx.x;
    const int kh = h / (nh / nkvh);
    for (int e = lane; e < d; e += 64) qs[e] = toF32(q[(size_t(i) * nh + h) * d + e]) * scale_log2;
    __syncthreads();

    const int n_keys = i + S - L + 1; // keys 0 .. i+S-L
    float m = -INFINITY;
    float l = 0.f;
    float acc[kMaxDim / 64] = {0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < n_keys; j0 += 64) {
        const int j = j0 + lane;
        float s = -INFINITY;
        if (j < n_keys) {
            const T *kr = k + (size_t(j) * nkvh + kh) * d;
            float dot = 0.f;
            for (int e = 0; e < d; ++e) dot = fmaf(qs[e], toF32(kr[e]), dot);
            s = dot;
        }
        const float m_new = fmaxf(m, waveMax(s));
        const float alpha = exp2f(m - m_new); // m_new is finite: key j0 is always valid
        const float p = (j < n_keys) ? exp2f(s - m_new) : 0.f;
        l = l * alpha + waveSum(p);
        m = m_new;
        ps[lane] = p;
        __syncthreads();
        const int cnt = min(64, n_keys - j0);
#pragma unroll
        for (int c = 0; c < kMaxDim / 64; ++c) {
            const int e = c * 64 + lane;
            float a = acc[c] * alpha;
            if (e < dv) {
                const T *vc = v + size_t(j0) * nkvh * dv + size_t(kh) * dv + e;
                for (int jj = 0; jj < cnt; ++jj) a = fmaf(ps[jj], toF32(vc[size_t(jj) * nkvh * dv]), a);
            }
            acc[c] = a;
        }
        __syncthreads();
    }
    const float inv = 1.f / l;
#pragma unroll
    for (int c = 0; c < kMaxDim / 64; ++c) {
        const int e = c * 64 + lane;
        if (e < dv) out[(size_t(i) * nh + h) * dv + e] = fromF32<T>(acc[c] * inv);
    }
}

template <typename T>
void launch(void *out, const void *q, const void *k, const void *v, int L, int S, int nh, int nkvh, int d, int dv,
            float scale, hipStream_t stream) {
    const float scale_log2 = scale * 1.4426950408889634f;
    hipLaunchKernelGGL(selfAttentionKernel<T>, dim3(L, nh), dim3(64), 0, stream, static_cast<T *>(out),
                       static_cast<const T *>(q), static_cast<const T *>(k), static_cast<const T *>(v), L, S, nh,
                       nkvh, d, dv, scale_log2);
    HIP_CHECK(hipGetLastError());
}

} // namespace

void selfAttention(void *out, const void *q, const void *k, const void *v, ElemType type, int L, int S, int nh,
                   int nkvh, int d, int dv, float scale, void *stream) {
    LLAISYS_CHECK(d <= kMaxDim && dv <= kMaxDim, "self_attention: head dims above " << kMaxDim << " not supported");
    if (L == 0 || nh == 0) return;
    auto s = static_cast<hipStream_t>(stream);
    switch (type) {
    case ElemType::F32: return launch<float>(out, q, k, v, L, S, nh, nkvh, d, dv, scale, s);
    case ElemType::F16: return launch<__half>(out, q, k, v, L, S, nh, nkvh, d, dv, scale, s);
    case ElemType::BF16: return launch<__hip_bfloat16>(out, q, k, v, L, S, nh, nkvh, d, dv, scale, s);
    }
}

} // namespace llaisys::kernels
