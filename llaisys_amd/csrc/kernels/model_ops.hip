// Elementwise / normalisation / indexing kernels of the reference's model ops
// (README.md:157-292; formulas test/ops/{add,argmax,embedding,rms_norm,rope,
// swiglu}.py), for the Qwen2 decode step built on the paged KV path. All math
// is fp32; results are rounded once to the tensor dtype.
#include "launch.hpp"

#include "../device/hip_check.hpp"

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <algorithm>

namespace llaisys::kernels {

namespace {

template <typename T> __device__ __forceinline__ float ld(const T *p, size_t i);
template <> __device__ __forceinline__ float ld<float>(const float *p, size_t i) { return p[i]; }
template <> __device__ __forceinline__ float ld<__half>(const __half *p, size_t i) { return __half2float(p[i]); }
template <> __device__ __forceinline__ float ld<__hip_bfloat16>(const __hip_bfloat16 *p, size_t i) {
    return __bfloat162float(p[i]);
}
template <typename T> __device__ __forceinline__ void st(T *p, size_t i, float v);
template <> __device__ __forceinline__ void st<float>(float *p, size_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void st<__half>(__half *p, size_t i, float v) { p[i] = __float2half_rn(v); }
template <> __device__ __forceinline__ void st<__hip_bfloat16>(__hip_bfloat16 *p, size_t i, float v) {
    p[i] = __float2bfloat16(v);
}

constexpr int kThreads = 256;

template <typename T> __global__ void addKernel(T *c, const T *a, const T *b, size_t n) {
    for (size_t i = blockIdx.x * size_t(kThreads) + threadIdx.x; i < n; i += size_t(gridDim.x) * kThreads)
        st(c, i, ld(a, i) + ld(b, i));
}

// out = up * gate / (1 + exp(-gate))
template <typename T> __global__ void swigluKernel(T *out, const T *gate, const T *up, size_t n) {
    for (size_t i = blockIdx.x * size_t(kThreads) + threadIdx.x; i < n; i += size_t(gridDim.x) * kThreads) {
        const float g = ld(gate, i);
        st(out, i, ld(up, i) * g / (1.f + expf(-g)));
    }
}

// out[r, c] = x[r, c] + bias[c]
template <typename T> __global__ void biasKernel(T *x, const T *bias, size_t rows, size_t cols) {
    const size_t n = rows * cols;
    for (size_t i = blockIdx.x * size_t(kThreads) + threadIdx.x; i < n; i += size_t(gridDim.x) * kThreads)
        st(x, i, ld(x, i) + ld(bias, i % cols));
}

__device__ float blockSum(float v, float *red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
    for (int w = 0; w < kThreads / 64; ++w) s += red[w];
    __syncthreads();
    return s;
}

// One block per row: y = x * w / sqrt(mean(x^2) + eps).
template <typename T> __global__ void __launch_bounds__(kThreads) rmsNormKernel(T *out, const T *x, const T *w, int d, float eps) {
    __shared__ float red[kThreads / 64];
    const size_t row = blockIdx.x;
    float ss = 0.f;
    for (int c = threadIdx.x; c < d; c += kThreads) {
        const float v = ld(x, row * d + c);
        ss += v * v;
    }
    const float inv = rsqrtf(blockSum(ss, red) / float(d) + eps);
    for (int c = threadIdx.x; c < d; c += kThreads) st(out, row * d + c, ld(x, row * d + c) * inv * ld(w, c));
}

// Rotate halves: for j < d/2, phi = pos / theta^(2j/d) computed in fp32 as the
// reference formula does; a' = a cos - b sin, b' = b cos + a sin.
template <typename T>
__global__ void ropeKernel(T *out, const T *in, const int64_t *pos, int nhead, int d, float theta) {
    const size_t tok = blockIdx.x;
    const int half = d / 2;
    const float p = float(pos[tok]);
    for (int t = threadIdx.x; t < nhead * half; t += kThreads) {
        const int h = t / half, j = t - h * half;
        const float phi = p / powf(theta, float(2 * j) / float(d));
        float s, c;
        sincosf(phi, &s, &c);
        const size_t base = (tok * nhead + h) * size_t(d);
        const float a = ld(in, base + j), b = ld(in, base + half + j);
        st(out, base + j, a * c - b * s);
        st(out, base + half + j, b * c + a * s);
    }
}

template <typename T>
__global__ void embeddingKernel(T *out, const int64_t *idx, const T *weight, int64_t vocab, int d, int *err) {
    const size_t r = blockIdx.x;
    const int64_t i = idx[r];
    if (i < 0 || i >= vocab) {
        if (threadIdx.x == 0) atomicOr(err, 4);
        return;
    }
    for (int c = threadIdx.x; c < d; c += kThreads) out[r * d + c] = weight[size_t(i) * d + c];
}

// One block per row: the first index of the maximum (NaN compares false, as
// a plain > scan would).
template <typename T>
__global__ void __launch_bounds__(kThreads) argmaxKernel(int64_t *idx, T *val, const T *vals, int64_t n) {
    __shared__ float sv[kThreads];
    __shared__ int64_t si[kThreads];
    const size_t row = blockIdx.x;
    float best = -INFINITY;
    int64_t bi = -1;
    for (int64_t c = threadIdx.x; c < n; c += kThreads) {
        const float v = ld(vals, row * n + c);
        if (bi < 0 || v > best) {
            best = v;
            bi = c;
        }
    }
    sv[threadIdx.x] = best;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            const float ov = sv[threadIdx.x + s];
            const int64_t oi = si[threadIdx.x + s];
            const float mv = sv[threadIdx.x];
            const int64_t mi = si[threadIdx.x];
            if (oi >= 0 && (mi < 0 || ov > mv || (ov == mv && oi < mi))) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        idx[row] = si[0];
        if (val) st(val, row, sv[0]);
    }
}

// Strided copy of equal-shaped tensors (up to kMaxDims dims), element size esz.
struct StridedDesc {
    int ndim;
    int64_t shape[kMaxDims];
    int64_t out_stride[kMaxDims];
    int64_t in_stride[kMaxDims];
};

template <typename E> __global__ void rearrangeKernel(E *out, const E *in, StridedDesc d, size_t n) {
    for (size_t i = blockIdx.x * size_t(kThreads) + threadIdx.x; i < n; i += size_t(gridDim.x) * kThreads) {
        size_t rem = i;
        int64_t oo = 0, io = 0;
        for (int k = d.ndim - 1; k >= 0; --k) {
            const int64_t c = int64_t(rem % size_t(d.shape[k]));
            rem /= size_t(d.shape[k]);
            oo += c * d.out_stride[k];
            io += c * d.in_stride[k];
        }
        out[oo] = in[io];
    }
}

unsigned gridFor(size_t n) { return unsigned(std::min<size_t>((n + kThreads - 1) / kThreads, 65536)); }

template <template <typename> class F, typename... Args> void byType(ElemType t, Args &&...args) {
    switch (t) {
    case ElemType::F32: return F<float>::run(args...);
    case ElemType::F16: return F<__half>::run(args...);
    case ElemType::BF16: return F<__hip_bfloat16>::run(args...);
    }
}

template <typename T> struct AddL {
    static void run(void *c, const void *a, const void *b, size_t n, hipStream_t s) {
        if (n) hipLaunchKernelGGL(addKernel<T>, dim3(gridFor(n)), dim3(kThreads), 0, s, (T *)c, (const T *)a, (const T *)b, n);
    }
};
template <typename T> struct SwigluL {
    static void run(void *o, const void *g, const void *u, size_t n, hipStream_t s) {
        if (n) hipLaunchKernelGGL(swigluKernel<T>, dim3(gridFor(n)), dim3(kThreads), 0, s, (T *)o, (const T *)g, (const T *)u, n);
    }
};
template <typename T> struct BiasL {
    static void run(void *x, const void *b, size_t rows, size_t cols, hipStream_t s) {
        if (rows * cols)
            hipLaunchKernelGGL(biasKernel<T>, dim3(gridFor(rows * cols)), dim3(kThreads), 0, s, (T *)x, (const T *)b, rows, cols);
    }
};
template <typename T> struct RmsL {
    static void run(void *o, const void *x, const void *w, size_t rows, int d, float eps, hipStream_t s) {
        if (rows) hipLaunchKernelGGL(rmsNormKernel<T>, dim3(rows), dim3(kThreads), 0, s, (T *)o, (const T *)x, (const T *)w, d, eps);
    }
};
template <typename T> struct RopeL {
    static void run(void *o, const void *x, const int64_t *pos, size_t ntok, int nhead, int d, float theta, hipStream_t s) {
        if (ntok) hipLaunchKernelGGL(ropeKernel<T>, dim3(ntok), dim3(kThreads), 0, s, (T *)o, (const T *)x, pos, nhead, d, theta);
    }
};
template <typename T> struct EmbL {
    static void run(void *o, const int64_t *idx, const void *w, size_t rows, int64_t vocab, int d, int *err, hipStream_t s) {
        if (rows) hipLaunchKernelGGL(embeddingKernel<T>, dim3(rows), dim3(kThreads), 0, s, (T *)o, idx, (const T *)w, vocab, d, err);
    }
};
template <typename T> struct ArgmaxL {
    static void run(int64_t *idx, void *val, const void *vals, size_t rows, int64_t n, hipStream_t s) {
        if (rows) hipLaunchKernelGGL(argmaxKernel<T>, dim3(rows), dim3(kThreads), 0, s, idx, (T *)val, (const T *)vals, n);
    }
};

} // namespace

void add(void *c, const void *a, const void *b, ElemType t, size_t n, void *stream) {
    byType<AddL>(t, c, a, b, n, static_cast<hipStream_t>(stream));
    HIP_CHECK(hipGetLastError());
}
void swiglu(void *out, const void *gate, const void *up, ElemType t, size_t n, void *stream) {
    byType<SwigluL>(t, out, gate, up, n, static_cast<hipStream_t>(stream));
    HIP_CHECK(hipGetLastError());
}
void addBias(void *x, const void *bias, ElemType t, size_t rows, size_t cols, void *stream) {
    byType<BiasL>(t, x, bias, rows, cols, static_cast<hipStream_t>(stream));
    HIP_CHECK(hipGetLastError());
}
void rmsNorm(void *out, const void *x, const void *w, ElemType t, size_t rows, int d, float eps, void *stream) {
    byType<RmsL>(t, out, x, w, rows, d, eps, static_cast<hipStream_t>(stream));
    HIP_CHECK(hipGetLastError());
}
void rope(void *out, const void *in, const int64_t *pos, ElemType t, size_t ntok, int nhead, int d, float theta,
          void *stream) {
    byType<RopeL>(t, out, in, pos, ntok, nhead, d, theta, static_cast<hipStream_t>(stream));
    HIP_CHECK(hipGetLastError());
}
void embedding(void *out, const int64_t *idx, const void *weight, ElemType t, size_t rows, int64_t vocab, int d,
               int *err, void *stream) {
    byType<EmbL>(t, out, idx, weight, rows, vocab, d, err, static_cast<hipStream_t>(stream));
    HIP_CHECK(hipGetLastError());
}
void argmax(int64_t *idx, void *val, const void *vals, ElemType t, size_t rows, int64_t n, void *stream) {
    byType<ArgmaxL>(t, idx, val, vals, rows, n, static_cast<hipStream_t>(stream));
    HIP_CHECK(hipGetLastError());
}
void rearrange(void *out, const void *in, size_t esz, int ndim, const int64_t *shape, const int64_t *out_strides,
               const int64_t *in_strides, void *stream) {
    LLAISYS_CHECK(ndim >= 0 && ndim <= kMaxDims, "rearrange: at most " << kMaxDims << " dims");
    StridedDesc d{};
    d.ndim = ndim;
    size_t n = 1;
    for (int k = 0; k < ndim; ++k) {
        d.shape[k] = shape[k];
        d.out_stride[k] = out_strides[k];
        d.in_stride[k] = in_strides[k];
        n *= size_t(shape[k]);
    }
    if (!n) return;
    auto s = static_cast<hipStream_t>(stream);
    switch (esz) {
    case 1: hipLaunchKernelGGL(rearrangeKernel<uint8_t>, dim3(gridFor(n)), dim3(kThreads), 0, s, (uint8_t *)out, (const uint8_t *)in, d, n); break;
    case 2: hipLaunchKernelGGL(rearrangeKernel<uint16_t>, dim3(gridFor(n)), dim3(kThreads), 0, s, (uint16_t *)out, (const uint16_t *)in, d, n); break;
    case 4: hipLaunchKernelGGL(rearrangeKernel<uint32_t>, dim3(gridFor(n)), dim3(kThreads), 0, s, (uint32_t *)out, (const uint32_t *)in, d, n); break;
    case 8: hipLaunchKernelGGL(rearrangeKernel<uint64_t>, dim3(gridFor(n)), dim3(kThreads), 0, s, (uint64_t *)out, (const uint64_t *)in, d, n); break;
    default: LLAISYS_RAISE("rearrange: element size " << esz << " not supported");
    }
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
