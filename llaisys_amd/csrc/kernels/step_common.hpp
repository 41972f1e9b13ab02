// Device helpers shared by the decode step's kernels: where a token's k/v
// element sits inside its (block, kv head) page, the RoPE angle, and a
// row's sum of squares for the RMSNorm factor.
#pragma once

#include <hip/hip_runtime.h>

namespace llaisys::kernels {

// Element (token t, dim d) of a K page: 8-dim chunks of all 16 tokens, then
// the next chunk ([d / 8][t][d % 8]).
__device__ __forceinline__ int kPageIndex(int t, int d) { return (d >> 3) * 128 + t * 8 + (d & 7); }
// Element (t, d) of a V page: [d / 32][t / 4][d % 16][(d / 16) % 2][t % 4].
__device__ __forceinline__ int vPageIndex(int t, int d) {
    return (d >> 5) * 512 + (t >> 2) * 128 + (d & 15) * 8 + ((d >> 4) & 1) * 4 + (t & 3);
}

// Angle by which the reference's rope turns the pair (j, j + d/2) at
// position pos (test/ops/rope.py:11-33): pos / theta^(2j/d).
__device__ __forceinline__ float ropePhi(int pos, int j, int d, float theta) {
    return float(pos) / powf(theta, float(2 * j) / float(d));
}

// A row of d bf16 values (d % 8 == 0) as lane-strided 16 B chunks (chunk c
// to lane c % 64 of a wave) for its sum of squares. load() issues all the
// lane's chunks of the first kRowChunks * 512 values at once, so a caller can
// start them beside its other loads; sumSquares() adds the lane's chunks in
// ascending order (reading any further ones then) and returns the wave's
// total, which every lane gets.
constexpr int kRowChunks = 4;
struct RowChunks {
    uint4 v[kRowChunks];
    __device__ __forceinline__ void load(const uint16_t *row, int d) {
        const int lane = threadIdx.x & 63;
        const uint4 *src = reinterpret_cast<const uint4 *>(row);
        // Clamped loads, no branch (a branch around a load makes later waits
        // count conservatively); sumSquares skips chunks past the row.
#pragma unroll
        for (int u = 0; u < kRowChunks; ++u) v[u] = src[min(lane + 64 * u, d / 8 - 1)];
    }
    __device__ __forceinline__ static void add(float &ss, const uint4 &x) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t w = (&x.x)[e];
            const float lo = __uint_as_float(w << 16), hi = __uint_as_float(w & 0xffff0000u);
            ss += lo * lo + hi * hi;
        }
    }
    __device__ __forceinline__ float sumSquares(const uint16_t *row, int d) const {
        const int lane = threadIdx.x & 63;
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < kRowChunks; ++u)
            if (lane + 64 * u < d / 8) add(ss, v[u]);
        const uint4 *src = reinterpret_cast<const uint4 *>(row);
        for (int c = lane + 64 * kRowChunks; c < d / 8; c += 64) add(ss, src[c]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
        return ss;
    }
};

// Row-wise argmax key: order-preserving bits of the value (NaN above +inf,
// as torch.max propagates NaN) << 32 | ~column, so the maximum key is the
// largest value at its first column.
__device__ __forceinline__ uint64_t argmaxKey(float v, int64_t col) {
    uint32_t u = __float_as_uint(v);
    if (v != v) u = 0x7fc00000u; // any NaN: the canonical positive NaN
    const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (uint64_t(ord) << 32) | uint32_t(~uint32_t(col));
}

} // namespace llaisys::kernels
