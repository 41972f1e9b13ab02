// Contiguous causal GQA attention: the reference's self_attention op
// (spec README.md:244-266; formula test/ops/self_attention.py:11-28).
//
//   out[i, h, :] = sum_j softmax_j(scale * q[i,h] . k[j, h/G]) v[j, h/G],
//   keys j <= i + S - L (bottom-right causal alignment), G = nh / nkvh.
//
// One workgroup of kWaves waves per (query, head, key split); the keys are
// cut into chunks of 64, split z of NS takes chunks z, z + NS, ... and wave
// w of it every kWaves-th of those (a wave per (query, head) walked all S
// keys alone: 56.6 us at L = 1, S = 513). A grid of few query rows x heads
// splits the keys over workgroups (each CU then streams a part of K and V
// instead of all of it); the splits leave (m, l, o) partials that a second
// kernel merges.
// Scores: one key per lane, its row read in 16 B pieces when the rows
// allow. Values: the 64 lanes are 4 groups of 16; group g takes keys
// g, g + 4, ... of the chunk and lane t of a group dims t, t + 16, ...
// (or 16 B pieces of them), so one load instruction reads 4 key rows.
// Online softmax in base 2 per wave, fp32 throughout; the waves' states
// (m, l, o) meet in LDS and one rounding to the output type ends it.
#include "launch.hpp"

#include "../device/hip_check.hpp"

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <algorithm>

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

constexpr int kWaves = 8;
constexpr int kDimsPerLane = kMaxDim / 16; // value accumulators per lane

// 16 B of a row: VEC elements widened to fp32.
template <typename T> struct Vec16 {
    static constexpr int N = 16 / sizeof(T);
    __device__ __forceinline__ static void load(const T *p, float (&f)[16 / sizeof(T)]) {
        typedef uint32_t u4 __attribute__((ext_vector_type(4)));
        const u4 w = *reinterpret_cast<const u4 *>(p);
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) f[e] = __uint_as_float(w[e]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t lo = w[e] & 0xffffu, hi = w[e] >> 16;
                f[2 * e] = toF32(__builtin_bit_cast(T, uint16_t(lo)));
                f[2 * e + 1] = toF32(__builtin_bit_cast(T, uint16_t(hi)));
            }
        }
    }
};

// VECK: key rows in 16 B pieces (d % VEC == 0, rows 16 B aligned);
// VECV: value rows likewise with dv % (16 VEC) == 0.
template <typename T, bool VECK, bool VECV>
__global__ void __launch_bounds__(64 * kWaves) selfAttentionKernel(T *__restrict__ out, const T *__restrict__ q,
                                                                   const T *__restrict__ k, const T *__restrict__ v,
                                                                   int L, int S, int nh, int nkvh, int d, int dv,
                                                                   float scale_log2, float *part) {
    constexpr int VEC = Vec16<T>::N;
    __shared__ float ps[kWaves][64];
    __shared__ float wo[kWaves][kMaxDim];
    __shared__ float wml[kWaves][2];
    const int i = blockIdx.x, h = blockIdx.y, z = blockIdx.z, NS = gridDim.z;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = lane >> 4, t = lane & 15;
    const int kh = h / (nh / nkvh);
    // q is the same for every lane: read through the scalar cache inside the
    // dot products (no LDS copy and no barrier ahead of the key loads).
    const T *qr = q + (size_t(i) * nh + h) * d;

    const int n_keys = i + S - L + 1; // keys 0 .. i+S-L
    const size_t kstride = size_t(nkvh) * d, vstride = size_t(nkvh) * dv;
    float m = -INFINITY, l = 0.f;
    float acc[kDimsPerLane];
#pragma unroll
    for (int c = 0; c < kDimsPerLane; ++c) acc[c] = 0.f;
    for (int j0 = 64 * (z + NS * wave); j0 < n_keys; j0 += 64 * NS * kWaves) {
        const int j = j0 + lane;
        float s = -INFINITY;
        if (j < n_keys) {
            const T *kr = k + size_t(j) * kstride + size_t(kh) * d;
            float dot = 0.f;
            if constexpr (VECK) {
#pragma unroll 16
                for (int e0 = 0; e0 < d; e0 += VEC) {
                    float f[VEC];
                    Vec16<T>::load(kr + e0, f);
#pragma unroll
                    for (int e = 0; e < VEC; ++e) dot = fmaf(toF32(qr[e0 + e]), f[e], dot);
                }
            } else {
                for (int e = 0; e < d; ++e) dot = fmaf(toF32(qr[e]), toF32(kr[e]), dot);
            }
            s = dot * scale_log2;
        }
        const float m_new = fmaxf(m, waveMax(s)); // finite: key j0 is valid
        const float alpha = exp2f(m - m_new);
        const float p = j < n_keys ? exp2f(s - m_new) : 0.f;
        l = l * alpha + waveSum(p);
        m = m_new;
        ps[wave][lane] = p; // read back by this wave only (LDS keeps a wave's order)
        const int cnt = min(64, n_keys - j0);
#pragma unroll
        for (int c = 0; c < kDimsPerLane; ++c) acc[c] *= alpha;
        const T *vb = v + size_t(j0) * vstride + size_t(kh) * dv;
        // 16 keys per group, every load unconditional (past cnt: the last
        // key again, weight 0) so the compiler issues them all up front.
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int jj = grp + 4 * u;
            const float pj = jj < cnt ? ps[wave][jj] : 0.f;
            const T *vr = vb + size_t(min(jj, cnt - 1)) * vstride;
            if constexpr (VECV) {
                // lane t: dims VEC t .. + VEC - 1 of each 16 VEC block
#pragma unroll
                for (int b = 0; b < kDimsPerLane / VEC; ++b) {
                    const int e0 = 16 * VEC * b + VEC * t;
                    if (e0 < dv) {
                        float f[VEC];
                        Vec16<T>::load(vr + e0, f);
#pragma unroll
                        for (int e = 0; e < VEC; ++e) acc[VEC * b + e] = fmaf(pj, f[e], acc[VEC * b + e]);
                    }
                }
            } else {
#pragma unroll
                for (int c = 0; c < kDimsPerLane; ++c) {
                    const int e = t + 16 * c;
                    if (e < dv) acc[c] = fmaf(pj, toF32(vr[e]), acc[c]);
                }
            }
        }
    }
    // The 4 key groups of the wave hold the same dims: sum them.
#pragma unroll
    for (int c = 0; c < kDimsPerLane; ++c) {
        acc[c] += __shfl_xor(acc[c], 16);
        acc[c] += __shfl_xor(acc[c], 32);
    }
    if (grp == 0) {
#pragma unroll
        for (int c = 0; c < kDimsPerLane; ++c) {
            const int e = VECV ? 16 * VEC * (c / VEC) + VEC * t + c % VEC : t + 16 * c;
            if (e < dv) wo[wave][e] = acc[c];
        }
    }
    if (lane == 0) {
        wml[wave][0] = m;
        wml[wave][1] = l;
    }
    __syncthreads();
    // Merge the waves: weights 2^(m_w - M) (a wave without keys: m = -inf,
    // weight 0).
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, wml[w][0]);
    float Lsum = 0.f, wt[kWaves];
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        wt[w] = exp2f(wml[w][0] - M);
        Lsum += wml[w][1] * wt[w];
    }
    if (NS > 1) {
        // Partial (m, l, o) of this split; a split without keys for this
        // query leaves m = -inf, l = 0, o = 0 (weight 0 in the merge).
        float *rec = part + ((size_t(i) * nh + h) * NS + z) * (dv + 2);
        const bool none = M == -INFINITY;
        if (threadIdx.x == 0) {
            rec[0] = M;
            rec[1] = none ? 0.f : Lsum;
        }
        for (int e = threadIdx.x; e < dv; e += 64 * kWaves) {
            float o = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) o += none ? 0.f : wt[w] * wo[w][e];
            rec[2 + e] = o;
        }
        return;
    }
    const float inv = 1.f / Lsum;
    for (int e = threadIdx.x; e < dv; e += 64 * kWaves) {
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) o += wt[w] * wo[w][e];
        out[(size_t(i) * nh + h) * dv + e] = fromF32<T>(o * inv);
    }
}

constexpr int kSplitGrid = 1024, kMaxSplits = 16;

// Merge the NS key splits of (query i, head h): weights 2^(m_z - M); one
// thread per output dim (dv <= 256).
template <typename T>
__global__ void __launch_bounds__(256) selfAttentionMergeKernel(T *__restrict__ out, const float *__restrict__ part,
                                                                int nh, int dv, int NS) {
    const int i = blockIdx.x, h = blockIdx.y;
    const float *recs = part + (size_t(i) * nh + h) * NS * (dv + 2);
    // Every split's (m, l) and this thread's o values requested at once.
    float m[kMaxSplits], lz[kMaxSplits], o[kMaxSplits];
    const int e = threadIdx.x;
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z) {
        const float *r = recs + size_t(min(z, NS - 1)) * (dv + 2);
        m[z] = z < NS ? r[0] : -INFINITY;
        lz[z] = r[1];
        o[z] = r[2 + min(e, dv - 1)];
    }
    float M = -INFINITY;
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z) M = fmaxf(M, m[z]);
    float Lsum = 0.f, acc = 0.f;
#pragma unroll
    for (int z = 0; z < kMaxSplits; ++z) {
        if (z >= NS) break;
        const float w = exp2f(m[z] - M);
        Lsum += lz[z] * w;
        acc += o[z] * w;
    }
    if (e < dv) out[(size_t(i) * nh + h) * dv + e] = fromF32<T>(acc / Lsum);
}

// Key splits: grids of under kSplitGrid (query, head) workgroups split the
// S / 64 key chunks over up to kMaxSplits workgroups each.
int splitsFor(int L, int S, int nh) {
    const long base = long(L) * nh;
    if (base >= kSplitGrid) return 1;
    const int chunks = (S + 63) / 64;
    return int(std::max<long>(1, std::min<long>({long(chunks), long(kMaxSplits), kSplitGrid / base})));
}

template <typename T>
void launch(void *out, const void *q, const void *k, const void *v, int L, int S, int nh, int nkvh, int d, int dv,
            float scale, hipStream_t stream, float *part) {
    const float scale_log2 = scale * 1.4426950408889634f;
    constexpr int VEC = 16 / int(sizeof(T));
    const bool veck = d % VEC == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0;
    const bool vecv = dv % (16 * VEC) == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0;
    auto *o = static_cast<T *>(out);
    const auto *qq = static_cast<const T *>(q), *kk = static_cast<const T *>(k), *vv = static_cast<const T *>(v);
    const int ns = splitsFor(L, S, nh);
    LLAISYS_CHECK(ns == 1 || part, "self_attention: this shape needs selfAttentionWorkspaceBytes() of workspace");
    const dim3 grid(L, nh, ns), block(64 * kWaves);
    if (veck && vecv)
        hipLaunchKernelGGL((selfAttentionKernel<T, true, true>), grid, block, 0, stream, o, qq, kk, vv, L, S, nh, nkvh,
                           d, dv, scale_log2, part);
    else if (veck)
        hipLaunchKernelGGL((selfAttentionKernel<T, true, false>), grid, block, 0, stream, o, qq, kk, vv, L, S, nh,
                           nkvh, d, dv, scale_log2, part);
    else if (vecv)
        hipLaunchKernelGGL((selfAttentionKernel<T, false, true>), grid, block, 0, stream, o, qq, kk, vv, L, S, nh,
                           nkvh, d, dv, scale_log2, part);
    else
        hipLaunchKernelGGL((selfAttentionKernel<T, false, false>), grid, block, 0, stream, o, qq, kk, vv, L, S, nh,
                           nkvh, d, dv, scale_log2, part);
    HIP_CHECK(hipGetLastError());
    if (ns > 1) {
        hipLaunchKernelGGL(selfAttentionMergeKernel<T>, dim3(L, nh), dim3(dv > 128 ? 256 : 128), 0, stream, o, part,
                           nh, dv, ns);
        HIP_CHECK(hipGetLastError());
    }
}

} // namespace

size_t selfAttentionWorkspaceBytes(int L, int S, int nh, int dv) {
    if (L <= 0 || nh <= 0) return 0;
    const int ns = splitsFor(L, S, nh);
    return ns > 1 ? size_t(L) * nh * ns * (dv + 2) * sizeof(float) : 0;
}

void selfAttention(void *out, const void *q, const void *k, const void *v, ElemType type, int L, int S, int nh,
                   int nkvh, int d, int dv, float scale, void *stream, void *workspace) {
    LLAISYS_CHECK(d <= kMaxDim && dv <= kMaxDim, "self_attention: head dims above " << kMaxDim << " not supported");
    if (L == 0 || nh == 0) return;
    auto s = static_cast<hipStream_t>(stream);
    auto *part = static_cast<float *>(workspace);
    switch (type) {
    case ElemType::F32: return launch<float>(out, q, k, v, L, S, nh, nkvh, d, dv, scale, s, part);
    case ElemType::F16: return launch<__half>(out, q, k, v, L, S, nh, nkvh, d, dv, scale, s, part);
    case ElemType::BF16: return launch<__hip_bfloat16>(out, q, k, v, L, S, nh, nkvh, d, dv, scale, s, part);
    }
}

} // namespace llaisys::kernels
