// Elementwise / normalisation / indexing kernels of the reference's model ops
// (README.md:157-292; formulas test/ops/{add,argmax,embedding,rms_norm,rope,
// swiglu}.py), for the Qwen2 decode step built on the paged KV path. All math
// is fp32; results are rounded once to the tensor dtype.
#include "launch.hpp"
#include "step_common.hpp"

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

template <typename T> __global__ void fillRowsKernel(T *x, const T *row, size_t rows, size_t cols) {
    const size_t n = rows * cols;
    for (size_t i = blockIdx.x * size_t(kThreads) + threadIdx.x; i < n; i += size_t(gridDim.x) * kThreads)
        x[i] = row[i % cols];
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

// One block per row: y = x * w / sqrt(mean(x^2) + eps). Rows of 2-byte
// elements with d % 8 == 0 move as 16 B vectors.
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

template <typename T> __device__ __forceinline__ float half8(const uint4 &v, int e) {
    const uint16_t h = uint16_t((&v.x)[e >> 1] >> ((e & 1) * 16));
    return ld(reinterpret_cast<const T *>(&h), 0);
}

template <typename T>
__global__ void __launch_bounds__(kThreads) rmsNormVecKernel(T *out, const T *x, const T *w, int d, float eps) {
    __shared__ float red[kThreads / 64];
    const size_t row = blockIdx.x;
    const uint4 *xr = reinterpret_cast<const uint4 *>(x + row * d);
    const int nv = d / 8;
    float ss = 0.f;
    for (int c = threadIdx.x; c < nv; c += kThreads) {
        const uint4 v = xr[c];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float f = half8<T>(v, e);
            ss += f * f;
        }
    }
    const float inv = rsqrtf(blockSum(ss, red) / float(d) + eps);
    const uint4 *wr = reinterpret_cast<const uint4 *>(w);
    uint4 *orow = reinterpret_cast<uint4 *>(out + row * d);
    for (int c = threadIdx.x; c < nv; c += kThreads) {
        const uint4 v = xr[c], g = wr[c];
        uint4 o;
        uint16_t *oh = reinterpret_cast<uint16_t *>(&o);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            T r;
            st(&r, 0, half8<T>(v, e) * inv * half8<T>(g, e));
            oh[e] = *reinterpret_cast<const uint16_t *>(&r);
        }
        orow[c] = o;
    }
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

// argmax over the last dim, split over columns: stage 1 reduces chunks of
// kArgmaxChunk columns of one row to a 64-bit key, stage 2 reduces a row's
// chunk keys. key = order-preserving bits of the value (NaN above +inf, as
// torch.max propagates NaN) << 32 | ~column, so the maximum key is the
// largest value at its first column.
constexpr int kArgmaxChunk = 4096;


__device__ __forceinline__ uint64_t waveMax(uint64_t k) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t o = __shfl_xor(k, off);
        k = o > k ? o : k;
    }
    return k;
}

// grid (chunks, rows): keys[row * chunks + chunk]. vec: 2-byte values, n % 8
// == 0 and a 16 B aligned base, read as 16 B vectors (8 columns) per load.
template <typename T>
__global__ void __launch_bounds__(kThreads) argmaxChunkKernel(uint64_t *keys, const T *vals, int64_t n, int chunks,
                                                              int vec) {
    __shared__ uint64_t red[kThreads / 64];
    const size_t row = blockIdx.y;
    const int64_t c0 = int64_t(blockIdx.x) * kArgmaxChunk;
    const int64_t c1 = min(n, c0 + kArgmaxChunk);
    uint64_t best = 0;
    if (vec) {
        const uint4 *v = reinterpret_cast<const uint4 *>(vals + row * n);
        for (int64_t c = c0 + 8 * threadIdx.x; c < c1; c += 8 * kThreads) {
            const uint4 u = v[c / 8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint16_t bits = uint16_t((&u.x)[e >> 1] >> ((e & 1) * 16));
                const uint64_t k = argmaxKey(ld(reinterpret_cast<const T *>(&bits), 0), c + e);
                best = k > best ? k : best;
            }
        }
    } else {
        for (int64_t c = c0 + threadIdx.x; c < c1; c += kThreads) {
            const uint64_t k = argmaxKey(ld(vals, row * n + c), c);
            best = k > best ? k : best;
        }
    }
    best = waveMax(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kThreads / 64; ++w) best = red[w] > best ? red[w] : best;
        keys[row * chunks + blockIdx.x] = best;
    }
}

// one wave per row
template <typename T>
__global__ void __launch_bounds__(64) argmaxFinishKernel(int64_t *idx, T *val, const uint64_t *keys, const T *vals,
                                                        int64_t n, int chunks) {
    const size_t row = blockIdx.x;
    uint64_t best = 0;
    for (int c = threadIdx.x; c < chunks; c += 64) best = keys[row * chunks + c] > best ? keys[row * chunks + c] : best;
    best = waveMax(best);
    if (threadIdx.x == 0) {
        const int64_t col = int64_t(~uint32_t(best & 0xffffffffu));
        idx[row] = col;
        if (val) val[row] = vals[row * n + col];
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
template <typename T> struct FillRowsL {
    static void run(void *x, const void *r, size_t rows, size_t cols, hipStream_t s) {
        if (rows * cols)
            hipLaunchKernelGGL(fillRowsKernel<T>, dim3(gridFor(rows * cols)), dim3(kThreads), 0, s, (T *)x, (const T *)r, rows, cols);
    }
};
template <typename T> struct RmsL {
    static void run(void *o, const void *x, const void *w, size_t rows, int d, float eps, hipStream_t s) {
        if (!rows) return;
        const bool vec = sizeof(T) == 2 && d % 8 == 0 && (reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(x) |
                                                          reinterpret_cast<uintptr_t>(w)) % 16 == 0;
        if (vec)
            hipLaunchKernelGGL(rmsNormVecKernel<T>, dim3(rows), dim3(kThreads), 0, s, (T *)o, (const T *)x, (const T *)w, d, eps);
        else
            hipLaunchKernelGGL(rmsNormKernel<T>, dim3(rows), dim3(kThreads), 0, s, (T *)o, (const T *)x, (const T *)w, d, eps);
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
    static void run(int64_t *idx, void *val, const void *vals, size_t rows, int64_t n, uint64_t *keys, hipStream_t s) {
        if (!rows) return;
        const int chunks = int((n + kArgmaxChunk - 1) / kArgmaxChunk);
        const int vec = sizeof(T) == 2 && n % 8 == 0 && reinterpret_cast<uintptr_t>(vals) % 16 == 0;
        hipLaunchKernelGGL(argmaxChunkKernel<T>, dim3(chunks, unsigned(rows)), dim3(kThreads), 0, s, keys, (const T *)vals, n,
                           chunks, vec);
        hipLaunchKernelGGL(argmaxFinishKernel<T>, dim3(unsigned(rows)), dim3(64), 0, s, idx, (T *)val, keys, (const T *)vals, n, chunks);
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
void fillRows(void *x, const void *row, ElemType t, size_t rows, size_t cols, void *stream) {
    byType<FillRowsL>(t, x, row, rows, cols, static_cast<hipStream_t>(stream));
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
void argmaxFinishKeys(int64_t *idx, const uint64_t *keys, size_t rows, int chunks, void *stream) {
    if (!rows) return;
    hipLaunchKernelGGL(argmaxFinishKernel<__hip_bfloat16>, dim3(unsigned(rows)), dim3(64), 0,
                       static_cast<hipStream_t>(stream), idx, nullptr, keys, nullptr, int64_t(0), chunks);
    HIP_CHECK(hipGetLastError());
}

size_t argmaxWorkspaceBytes(size_t rows, int64_t n) {
    return rows * size_t((n + kArgmaxChunk - 1) / kArgmaxChunk) * sizeof(uint64_t);
}
void argmax(int64_t *idx, void *val, const void *vals, ElemType t, size_t rows, int64_t n, void *workspace,
            void *stream) {
    byType<ArgmaxL>(t, idx, val, vals, rows, n, static_cast<uint64_t *>(workspace), static_cast<hipStream_t>(stream));
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
