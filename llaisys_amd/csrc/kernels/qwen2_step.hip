// Fused glue kernels of the Qwen2 decode/prefill step (bf16 activations,
// fp32 math, one rounding per output):
//  * qkvRopeAppend: split the fused QKV projection rows (plus bias) into q
//    [T, nh, d] and k/v, rotating q and k by the token's position (the
//    reference's rope formula, test/ops/rope.py:11-33), with k/v written
//    straight into their slots of the paged pool (the append of paged_kv.hip
//    fused in);
//  * swigluRows: act = up * silu(gate) over fused [gate | up] rows
//    (test/ops/swiglu.py:11-12);
//  * rmsNormRows: rms_norm of all or selected rows (the last position of each
//    sequence before the LM head; test/ops/rms_norm.py:11-17);
//  * foldNormColumns: W' = W diag(w), the RMSNorm weight folded into the
//    columns of the projection that consumes the normalised rows. With it,
//    rms_norm(x) W^T = r(x) * (x W'^T), r(x) = 1/sqrt(mean(x^2) + eps), and
//    the per-row factor r is applied by the kernel that reads the GEMM's
//    output (qkvRopeAppend, swigluRows take the residual rows x for it), so
//    the layer runs no separate rms_norm launch.
#include "launch.hpp"
#include "step_common.hpp"

#include "../common.hpp"
#include "../device/hip_check.hpp"

#include <hip/hip_bf16.h>

#include <algorithm>

namespace llaisys::kernels {

namespace {

using bf16 = __hip_bfloat16;
constexpr int kThreads = 256;

__device__ __forceinline__ float f(bf16 v) { return __bfloat162float(v); }

// 1/sqrt(mean(x^2) + eps) of one row of d (% 8 == 0) bf16 values, computed
// by the whole 64-lane wave (every lane gets the result), as rmsNormRows
// does, from a RowChunks load the caller issued beside its other loads.
__device__ __forceinline__ float rowInvRms(const RowChunks &xr, const bf16 *xrow, int d, float eps) {
    const float ss = xr.sumSquares(reinterpret_cast<const uint16_t *>(xrow), d);
    return rsqrtf(ss / float(d) + eps);
}

// out[r, c] = bf16(w[r, c] * g[c]) over rows x cols (cols % 8 == 0); the
// product of two bf16 values is exact in fp32, so this is one rounding.
__global__ void foldNormColumnsKernel(uint4 *out, const uint4 *w, const uint4 *g, size_t n, int nv) {
    for (size_t i = blockIdx.x * size_t(kThreads) + threadIdx.x; i < n; i += size_t(gridDim.x) * kThreads) {
        const uint4 a = w[i], b = g[i % nv];
        uint4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t aw = (&a.x)[e], bw = (&b.x)[e];
            const uint32_t lo = __builtin_bit_cast(uint16_t, __float2bfloat16(__uint_as_float(aw << 16) *
                                                                               __uint_as_float(bw << 16)));
            const uint32_t hi = __builtin_bit_cast(uint16_t, __float2bfloat16(__uint_as_float(aw & 0xffff0000u) *
                                                                               __uint_as_float(bw & 0xffff0000u)));
            (&o.x)[e] = lo | (hi << 16);
        }
        out[i] = o;
    }
}

// Row r = blockIdx.y, 8 columns per thread (di % 8 == 0): 16 B loads of gate
// and up, one 16 B store. x (may be null): the residual rows whose RMSNorm
// weight was folded into the gate/up projection; gate and up are then scaled
// by the row's 1/rms (each wave works it out itself: no barrier).
__global__ void __launch_bounds__(kThreads) swigluRowsKernel(bf16 *act, const bf16 *gu, const bf16 *x, int di, int hs,
                                                             float eps, int interleaved) {
    const int nv = di / 8;
    const size_t r = blockIdx.y;
    const int c = blockIdx.x * kThreads + threadIdx.x;
    // Every load first (gate, up and the row's x, clamped rather than
    // branched), so the latencies overlap.
    const int cc = min(c, nv - 1);
    // 8 columns: gate chunk cc and up chunk cc, side by side when interleaved.
    const uint4 *row = reinterpret_cast<const uint4 *>(gu + r * 2 * di);
    const uint4 g = interleaved ? row[2 * cc] : row[cc];
    const uint4 u = interleaved ? row[2 * cc + 1] : row[cc + di / 8];
    RowChunks xr; // (without x the gate row stands in: read, not used)
    xr.load(reinterpret_cast<const uint16_t *>(x ? x + r * hs : gu + r * 2 * di), x ? hs : 8);
    const float rs = x ? rowInvRms(xr, x + r * hs, hs, eps) : 1.f;
    if (c < nv) {
        uint4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t gw = (&g.x)[e], uw = (&u.x)[e];
            const float g0 = rs * __uint_as_float(gw << 16), g1 = rs * __uint_as_float(gw & 0xffff0000u);
            const float u0 = rs * __uint_as_float(uw << 16), u1 = rs * __uint_as_float(uw & 0xffff0000u);
            const uint32_t lo = __builtin_bit_cast(uint16_t, __float2bfloat16(u0 * g0 / (1.f + expf(-g0))));
            const uint32_t hi = __builtin_bit_cast(uint16_t, __float2bfloat16(u1 * g1 / (1.f + expf(-g1))));
            (&o.x)[e] = lo | (hi << 16);
        }
        reinterpret_cast<uint4 *>(act)[r * nv + c] = o;
    }
}


// One 256-thread block (4 waves) per token row r over its nh query, nkvh key
// and nkvh value heads; row r belongs to sequence b (cu: varlen offsets, else
// r == b) at position pos = ctx[b] + (r - cu[b]). Wave w takes heads w,
// w + 4, ...: lane j rotates the pair (j, j + d/2) of a q or k head, or moves
// dims 2j, 2j + 1 of a v head. The row's sequence, position, RoPE angle and
// page slot are worked out once for all its heads (a launch per (row, head)
// spent most of its time looking them up: 194 us for 8192 rows). Error bits
// as the append kernel: 1 bad block id, 2 position past the block table.
constexpr int kRopeRowWaves = 4;
constexpr int kRopeHeadsPerPass = 4; // heads per wave whose loads go out together
__global__ void __launch_bounds__(64 * kRopeRowWaves) qkvRopeAppendKernel(
    bf16 *q, uint16_t *k_pool, uint16_t *v_pool, const bf16 *qkv, const bf16 *bias, const int32_t *table,
    const int32_t *ctx, const int32_t *cu, int B, int nh, int nkvh, int d, int max_pages, int num_blocks, float theta,
    int *err, const bf16 *x, int hs, float eps) {
    const int r = blockIdx.x, wave = threadIdx.x >> 6, j = threadIdx.x & 63;
    const int half = d / 2, H = nh + 2 * nkvh;
    const bf16 *row = qkv + size_t(r) * H * d;
    // Every load that depends on no other is issued first: the row's x for
    // the 1/rms of the RMSNorm folded into the QKV weights (x null: none),
    // this lane's projection values and biases of the first heads (q/k: dims
    // j and j + d/2; v: dims 2j and 2j + 1), the sequence offsets.
    // (Without x the projection row stands in: read, not used; a branch
    // around the load would make later waits count conservatively.)
    RowChunks xr;
    xr.load(reinterpret_cast<const uint16_t *>(x ? x + size_t(r) * hs : row), x ? hs : 8);
    float pv[kRopeHeadsPerPass][4];
    auto loadPass = [&](int h0) {
#pragma unroll
        for (int u = 0; u < kRopeHeadsPerPass; ++u) {
            const int h = min(h0 + kRopeRowWaves * u, H - 1);
            const int c0 = h < nh + nkvh ? h * d + j : (nh + nkvh) * d + (h - nh - nkvh) * d + 2 * j;
            const int c1 = h < nh + nkvh ? c0 + half : c0 + 1;
            pv[u][0] = f(row[c0]);
            pv[u][1] = f(row[c1]);
            pv[u][2] = f(bias[c0]);
            pv[u][3] = f(bias[c1]);
        }
    };
    loadPass(wave);
    // The row's sequence: the number of offsets cu[0..B] at most r, counted
    // 64 at a time by ballots (cu is non-decreasing, cu[0] = 0 <= r < cu[B]).
    int b = r;
    if (cu) {
        int cnt = 0;
        for (int c0 = 0; c0 <= B; c0 += 256) {
            int v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = c0 + 64 * u + j;
                v[u] = i <= B ? cu[i] : 0x7fffffff;
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) cnt += int(__popcll(__ballot(v[u] <= r)));
        }
        b = min(max(cnt - 1, 0), B - 1);
    }
    const int pos = ctx[b] + (cu ? r - cu[b] : 0);
    const float rs = x ? rowInvRms(xr, x + size_t(r) * hs, hs, eps) : 1.f;
    // Every q and k head of the row turns pair j by the same angle.
    float sn, cs;
    sincosf(ropePhi(pos, j, d, theta), &sn, &cs);
    // The new token's page slot, for every k and v head of the row.
    const int page = pos >> 4, slot = pos & 15;
    const bool in_table = pos >= 0 && page < max_pages;
    const int blk = in_table ? table[size_t(b) * max_pages + page] : -1;
    const bool slot_ok = in_table && blk >= 0 && blk < num_blocks;
    for (int h0 = wave; h0 < H; h0 += kRopeRowWaves * kRopeHeadsPerPass) {
        if (h0 != wave) loadPass(h0);
#pragma unroll
        for (int u = 0; u < kRopeHeadsPerPass; ++u) {
            const int h = h0 + kRopeRowWaves * u;
            if (h >= H) break;
            const float a = rs * pv[u][0] + pv[u][2], bb = rs * pv[u][1] + pv[u][3];
            if (h < nh) {
                bf16 *dst = q + (size_t(r) * nh + h) * d;
                dst[j] = __float2bfloat16(a * cs - bb * sn);
                dst[j + half] = __float2bfloat16(bb * cs + a * sn);
            } else if (!slot_ok) {
                if (j == 0 && h == nh) atomicOr(err, in_table ? 1 : 2);
            } else if (h < nh + nkvh) {
                uint16_t *pg = k_pool + (size_t(blk) * nkvh + (h - nh)) * kPageElems;
                pg[kPageIndex(slot, j)] = __builtin_bit_cast(uint16_t, __float2bfloat16(a * cs - bb * sn));
                pg[kPageIndex(slot, j + half)] = __builtin_bit_cast(uint16_t, __float2bfloat16(bb * cs + a * sn));
            } else {
                uint16_t *pg = v_pool + (size_t(blk) * nkvh + (h - nh - nkvh)) * kPageElems;
                pg[vPageIndex(slot, 2 * j)] = __builtin_bit_cast(uint16_t, __float2bfloat16(a));
                pg[vPageIndex(slot, 2 * j + 1)] = __builtin_bit_cast(uint16_t, __float2bfloat16(bb));
            }
        }
    }
}

// One wave per output row r (source row rows[r], or r), VPL 16-byte vectors
// (8 columns) per lane: the row and the norm weights are loaded together and
// kept in registers, the sum of squares is a wave reduction (no LDS, no
// barrier), then each element is scaled and rounded once.
template <int VPL>
__global__ void __launch_bounds__(64) rmsNormRowsKernel(uint16_t *out, const bf16 *x, const int64_t *rows,
                                                        const bf16 *w, int d, float eps) {
    const int r = blockIdx.x, lane = threadIdx.x;
    const uint4 *src = reinterpret_cast<const uint4 *>(x + size_t(rows ? rows[r] : r) * d);
    const uint4 *wr = reinterpret_cast<const uint4 *>(w);
    const int nv = d / 8;
    uint4 v[VPL], g[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int c = lane + i * 64;
        v[i] = c < nv ? src[c] : uint4{0, 0, 0, 0};
        g[i] = c < nv ? wr[c] : uint4{0, 0, 0, 0};
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t u = (&v[i].x)[e];
            const float lo = __uint_as_float(u << 16), hi = __uint_as_float(u & 0xffff0000u);
            ss += lo * lo + hi * hi;
        }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float inv = rsqrtf(ss / float(d) + eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int c = lane + i * 64;
        if (c >= nv) break;
        uint4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t u = (&v[i].x)[e], gw = (&g[i].x)[e];
            const uint32_t lo = __builtin_bit_cast(uint16_t, __float2bfloat16(__uint_as_float(u << 16) * inv *
                                                                               __uint_as_float(gw << 16)));
            const uint32_t hi = __builtin_bit_cast(uint16_t, __float2bfloat16(__uint_as_float(u & 0xffff0000u) * inv *
                                                                               __uint_as_float(gw & 0xffff0000u)));
            (&o.x)[e] = lo | (hi << 16);
        }
        reinterpret_cast<uint4 *>(out)[size_t(r) * nv + c] = o;
    }
}
constexpr int kRowMaxVecs = 16; // d <= 16 * 64 * 8 = 8192

// Multi-step decode: step s reads s from a device counter (steps started).
// Advance, at the start of step s: the previous step's argmax (next) goes
// into history[s - 1], lengths = base + s (before) and base + s + 1 (after),
// tokens = first at s = 0 else next, then the counter moves to s + 1 (after
// every thread has read it). After the last step, decodeRecordLast writes
// the final argmax into history[counter - 1]. One block each.
__global__ void __launch_bounds__(kThreads) decodeAdvanceKernel(int32_t *ctx_before, int32_t *ctx_after, int64_t *tok,
                                                                int64_t *history, const int32_t *base,
                                                                const int64_t *first, const int64_t *next,
                                                                int32_t *counter, int B) {
    const int s = *counter;
    for (int b = threadIdx.x; b < B; b += kThreads) {
        if (s > 0) history[size_t(s - 1) * B + b] = next[b];
        ctx_before[b] = base[b] + s;
        ctx_after[b] = base[b] + s + 1;
        tok[b] = s == 0 ? first[b] : next[b];
    }
    __syncthreads();
    if (threadIdx.x == 0) *counter = s + 1;
}

__global__ void __launch_bounds__(kThreads) decodeRecordLastKernel(int64_t *history, const int64_t *next,
                                                                   const int32_t *counter, int B) {
    const int s = *counter;
    for (int b = threadIdx.x; b < B; b += kThreads) history[size_t(s - 1) * B + b] = next[b];
}

} // namespace

void decodeAdvance(int32_t *ctx_before, int32_t *ctx_after, int64_t *tok, int64_t *history, const int32_t *base,
                   const int64_t *first, const int64_t *next, int32_t *counter, int B, void *stream) {
    hipLaunchKernelGGL(decodeAdvanceKernel, dim3(1), dim3(kThreads), 0, static_cast<hipStream_t>(stream), ctx_before,
                       ctx_after, tok, history, base, first, next, counter, B);
    HIP_CHECK(hipGetLastError());
}

namespace {
// One block per row, 16 B (8 columns) per thread, stored twice: row-major and
// packed (an 8-column chunk is one contiguous 16 B piece of both).
__global__ void __launch_bounds__(kThreads) embedRowsPackedKernel(uint16_t *x, uint16_t *xp, const int64_t *idx,
                                                                  const uint16_t *w, int64_t vocab, int d, int *err) {
    const int r = blockIdx.x;
    const int64_t i = idx[r];
    if (i < 0 || i >= vocab) {
        if (threadIdx.x == 0) atomicOr(err, 4);
        return;
    }
    for (int c = 8 * threadIdx.x; c < d; c += 8 * kThreads) {
        const uint4 v = *reinterpret_cast<const uint4 *>(w + size_t(i) * d + c);
        *reinterpret_cast<uint4 *>(x + size_t(r) * d + c) = v;
        *reinterpret_cast<uint4 *>(xp + packedRowIndex(r, c, d)) = v;
    }
}
} // namespace

void embedRowsPacked(uint16_t *x, uint16_t *x_packed, const int64_t *idx, const uint16_t *weight, int T,
                     int64_t vocab, int d, int *err, void *stream) {
    LLAISYS_CHECK(d > 0 && d % 32 == 0, "embedRowsPacked: row length must be a positive multiple of 32, got " << d);
    if (T <= 0) return;
    hipLaunchKernelGGL(embedRowsPackedKernel, dim3(T), dim3(kThreads), 0, static_cast<hipStream_t>(stream), x,
                       x_packed, idx, weight, vocab, d, err);
    HIP_CHECK(hipGetLastError());
}

void decodeRecordLast(int64_t *history, const int64_t *next, const int32_t *counter, int B, void *stream) {
    hipLaunchKernelGGL(decodeRecordLastKernel, dim3(1), dim3(kThreads), 0, static_cast<hipStream_t>(stream), history,
                       next, counter, B);
    HIP_CHECK(hipGetLastError());
}

void qkvRopeAppend(uint16_t *q, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *qkv, const uint16_t *bias,
                   const int32_t *table, const int32_t *ctx, const int32_t *cu, int T, int B, int nh, int nkvh, int d,
                   int max_pages, int num_blocks, float theta, int *err, const uint16_t *x, int hs, float eps,
                   void *stream) {
    if (!T) return;
    LLAISYS_CHECK(d == 128, "qkvRopeAppend: head dim must be 128, got " << d);
    LLAISYS_CHECK(!x || (hs > 0 && hs % 8 == 0), "qkvRopeAppend: hidden size must be a positive multiple of 8");
    hipLaunchKernelGGL(qkvRopeAppendKernel, dim3(unsigned(T)), dim3(64 * kRopeRowWaves), 0,
                       static_cast<hipStream_t>(stream),
                       reinterpret_cast<bf16 *>(q), k_pool, v_pool, reinterpret_cast<const bf16 *>(qkv),
                       reinterpret_cast<const bf16 *>(bias), table, ctx, cu, B, nh, nkvh, d, max_pages, num_blocks,
                       theta, err, reinterpret_cast<const bf16 *>(x), hs, eps);
    HIP_CHECK(hipGetLastError());
}

void swigluRows(uint16_t *act, const uint16_t *gate_up, const uint16_t *x, size_t T, int di, int hs, float eps,
                void *stream, bool interleaved) {
    LLAISYS_CHECK(di % 8 == 0, "swigluRows: di must be a multiple of 8, got " << di);
    LLAISYS_CHECK(!x || (hs > 0 && hs % 8 == 0), "swigluRows: hidden size must be a positive multiple of 8");
    constexpr size_t kMaxRows = 65535; // grid y limit: longer batches take several launches
    for (size_t r0 = 0; r0 < T; r0 += kMaxRows) {
        const size_t rows = std::min(kMaxRows, T - r0);
        const dim3 grid(unsigned((di / 8 + kThreads - 1) / kThreads), unsigned(rows));
        hipLaunchKernelGGL(swigluRowsKernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                           reinterpret_cast<bf16 *>(act + r0 * di), reinterpret_cast<const bf16 *>(gate_up + r0 * 2 * di),
                           x ? reinterpret_cast<const bf16 *>(x + r0 * hs) : nullptr, di, hs, eps, interleaved ? 1 : 0);
        HIP_CHECK(hipGetLastError());
    }
}

void foldNormColumns(uint16_t *out, const uint16_t *w, const uint16_t *g, size_t rows, int cols, void *stream) {
    LLAISYS_CHECK(cols % 8 == 0, "foldNormColumns: cols must be a multiple of 8, got " << cols);
    const size_t n = rows * size_t(cols / 8);
    if (!n) return;
    const unsigned grid = unsigned(std::min<size_t>((n + kThreads - 1) / kThreads, 65536));
    hipLaunchKernelGGL(foldNormColumnsKernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<uint4 *>(out), reinterpret_cast<const uint4 *>(w),
                       reinterpret_cast<const uint4 *>(g), n, cols / 8);
    HIP_CHECK(hipGetLastError());
}

void swigluInterleave(uint16_t *out, const uint16_t *w, int di, int cols, void *stream) {
    LLAISYS_CHECK(di % 16 == 0 && cols % 8 == 0,
                  "swigluInterleave: di % 16 and cols % 8 must be 0 (di=" << di << ", cols=" << cols << ")");
    const size_t row_bytes = size_t(cols) * 2;
    // Block 2j <- gate rows 16j .., block 2j + 1 <- up rows 16j ..: one 2-D
    // copy per half, rows of 16-row blocks strided by two blocks.
    for (int half = 0; half < 2; ++half)
        HIP_CHECK(hipMemcpy2DAsync(reinterpret_cast<char *>(out) + size_t(half) * 16 * row_bytes, 32 * row_bytes,
                                   reinterpret_cast<const char *>(w) + size_t(half) * di * row_bytes, 16 * row_bytes,
                                   16 * row_bytes, size_t(di / 16), hipMemcpyDeviceToDevice,
                                   static_cast<hipStream_t>(stream)));
}

void rmsNormRows(uint16_t *out, const uint16_t *x, const int64_t *rows, const uint16_t *w, size_t R, int d, float eps,
                 void *stream) {
    LLAISYS_CHECK(d % 8 == 0 && d <= kRowMaxVecs * 64 * 8,
                  "rmsNormRows: d must be a multiple of 8 and at most " << kRowMaxVecs * 64 * 8 << ", got " << d);
    if (!R) return;
    const int vpl = (d / 8 + 63) / 64;
    const auto s = static_cast<hipStream_t>(stream);
    const auto *xb = reinterpret_cast<const bf16 *>(x);
    const auto *wb = reinterpret_cast<const bf16 *>(w);
    const dim3 grid{unsigned(R)}, block{64};
    if (vpl <= 1)
        hipLaunchKernelGGL(rmsNormRowsKernel<1>, grid, block, 0, s, out, xb, rows, wb, d, eps);
    else if (vpl <= 2)
        hipLaunchKernelGGL(rmsNormRowsKernel<2>, grid, block, 0, s, out, xb, rows, wb, d, eps);
    else if (vpl <= 4)
        hipLaunchKernelGGL(rmsNormRowsKernel<4>, grid, block, 0, s, out, xb, rows, wb, d, eps);
    else if (vpl <= 8)
        hipLaunchKernelGGL(rmsNormRowsKernel<8>, grid, block, 0, s, out, xb, rows, wb, d, eps);
    else
        hipLaunchKernelGGL(rmsNormRowsKernel<16>, grid, block, 0, s, out, xb, rows, wb, d, eps);
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
