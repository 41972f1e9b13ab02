// Fused glue kernels of the Qwen2 decode/prefill step (bf16 activations,
// fp32 math, one rounding per output):
//  * qkvRope: split the fused QKV projection rows into q [T, nh, d] and
//    k/v [T, nkvh, d], rotating q and k by the token's position (the
//    reference's rope formula, test/ops/rope.py:11-33);
//  * swigluRows: act = up * silu(gate) over fused [gate | up] rows
//    (test/ops/swiglu.py:11-12);
//  * rmsNormRows: rms_norm of selected rows only (the last position of each
//    sequence before the LM head; test/ops/rms_norm.py:11-17).
#include "launch.hpp"

#include "../device/hip_check.hpp"

#include <hip/hip_bf16.h>

#include <algorithm>

namespace llaisys::kernels {

namespace {

using bf16 = __hip_bfloat16;
constexpr int kThreads = 256;

__device__ __forceinline__ float f(bf16 v) { return __bfloat162float(v); }

// One block per token. Rotation pairs (j, j + d/2), angle pos / theta^(2j/d).
__global__ void __launch_bounds__(kThreads) qkvRopeKernel(bf16 *q, bf16 *k, bf16 *v, const bf16 *qkv, const int64_t *pos,
                                                          int nh, int nkvh, int d, float theta) {
    const size_t t = blockIdx.x;
    const int half = d / 2;
    const int width = (nh + 2 * nkvh) * d;
    const bf16 *row = qkv + t * size_t(width);
    const float p = float(pos[t]);
    // rotated heads: nh query heads then nkvh key heads, half-pairs each
    for (int i = threadIdx.x; i < (nh + nkvh) * half; i += kThreads) {
        const int h = i / half, j = i - h * half;
        const float phi = p / powf(theta, float(2 * j) / float(d));
        float s, c;
        sincosf(phi, &s, &c);
        const bf16 *src = row + h * d;
        const float a = f(src[j]), b = f(src[j + half]);
        bf16 *dst = h < nh ? q + (t * nh + h) * size_t(d) : k + (t * nkvh + (h - nh)) * size_t(d);
        dst[j] = __float2bfloat16(a * c - b * s);
        dst[j + half] = __float2bfloat16(b * c + a * s);
    }
    const bf16 *vsrc = row + (nh + nkvh) * d;
    for (int i = threadIdx.x; i < nkvh * d; i += kThreads) v[t * size_t(nkvh) * d + i] = vsrc[i];
}

__global__ void swigluRowsKernel(bf16 *act, const bf16 *gu, size_t T, int di) {
    const size_t n = T * size_t(di);
    for (size_t i = blockIdx.x * size_t(kThreads) + threadIdx.x; i < n; i += size_t(gridDim.x) * kThreads) {
        const size_t r = i / di, c = i - r * di;
        const float g = f(gu[r * 2 * di + c]), u = f(gu[r * 2 * di + di + c]);
        act[i] = __float2bfloat16(u * g / (1.f + expf(-g)));
    }
}

__global__ void __launch_bounds__(kThreads) rmsNormRowsKernel(bf16 *out, const bf16 *x, const int64_t *rows, const bf16 *w,
                                                              int d, float eps) {
    __shared__ float red[kThreads / 64];
    const bf16 *src = x + size_t(rows[blockIdx.x]) * d;
    float ss = 0.f;
    for (int c = threadIdx.x; c < d; c += kThreads) ss += f(src[c]) * f(src[c]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < kThreads / 64; ++i) tot += red[i];
    const float inv = rsqrtf(tot / float(d) + eps);
    for (int c = threadIdx.x; c < d; c += kThreads)
        out[size_t(blockIdx.x) * d + c] = __float2bfloat16(f(src[c]) * inv * f(w[c]));
}

} // namespace

void qkvRope(uint16_t *q, uint16_t *k, uint16_t *v, const uint16_t *qkv, const int64_t *pos, size_t T, int nh, int nkvh,
             int d, float theta, void *stream) {
    if (!T) return;
    hipLaunchKernelGGL(qkvRopeKernel, dim3(unsigned(T)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<bf16 *>(q), reinterpret_cast<bf16 *>(k), reinterpret_cast<bf16 *>(v),
                       reinterpret_cast<const bf16 *>(qkv), pos, nh, nkvh, d, theta);
    HIP_CHECK(hipGetLastError());
}

void swigluRows(uint16_t *act, const uint16_t *gate_up, size_t T, int di, void *stream) {
    const size_t n = T * size_t(di);
    if (!n) return;
    const unsigned grid = unsigned(std::min<size_t>((n + kThreads - 1) / kThreads, 65536));
    hipLaunchKernelGGL(swigluRowsKernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<bf16 *>(act), reinterpret_cast<const bf16 *>(gate_up), T, di);
    HIP_CHECK(hipGetLastError());
}

void rmsNormRows(uint16_t *out, const uint16_t *x, const int64_t *rows, const uint16_t *w, size_t R, int d, float eps,
                 void *stream) {
    if (!R) return;
    hipLaunchKernelGGL(rmsNormRowsKernel, dim3(unsigned(R)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<bf16 *>(out), reinterpret_cast<const bf16 *>(x), rows,
                       reinterpret_cast<const bf16 *>(w), d, eps);
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
