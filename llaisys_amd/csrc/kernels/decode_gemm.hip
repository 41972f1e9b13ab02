// Decode-sized projections for gfx950: Y[M, N] (+)= X[M, K] . W[N, K]^T with
// M <= 128 token rows, bf16 in and out, fp32 accumulation (the reference's
// linear, README.md:181-198, at the shapes of a batched decode step).
//
// The weights are streamed from HBM exactly once, so the kernel is built
// around that stream:
//  * W is kept pre-packed in MFMA operand order: tile (nb, kb) = rows
//    16 nb .. 16 nb + 15, k 32 kb .. 32 kb + 31 is 1 KiB, one coalesced
//    64-lane x 16 B load that is the A operand of v_mfma_f32_16x16x32_bf16 as
//    loaded (lane l: row l % 16, k 8 (l / 16) .. + 7). Row blocks are
//    contiguous runs of tiles.
//  * A workgroup is 4 waves, one per SIMD. Wave w owns the k range
//    [w K / 4, (w + 1) K / 4) and holds X for that range and all M rows in
//    registers for the whole launch (KS x MB x 16 B per lane; 384 registers at
//    K = 1536, M = 128), loaded once.
//  * The workgroup walks its 16-row blocks of W (blocks g, g + grid, ...);
//    each wave streams its KS tiles of a block through a KS-deep register
//    ring, the next block's tile j issued as soon as tile j is consumed, so
//    a block's loads are in flight while the previous block computes and
//    nothing in the loop waits on another wave.
//  * Per block, each wave's partial C^T[16 rows x M] goes to LDS; after one
//    barrier wave w sums the four partials of m blocks w, w + 4 and writes
//    bf16 rows (+ the old Y when accumulating, before the one rounding; a
//    bias enters the same way, preset as the rows of Y).
// Double-buffered partials make that the only barrier per block.
#include "launch.hpp"

#include "../device/hip_check.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <vector>

namespace llaisys::kernels {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));


struct GemmArgs {
    uint16_t *y;
    const uint16_t *x;
    const u32x4 *wp;     // packed W
    int M, N, K, nblocks, accumulate;
    int mgroups; // workgroups per row block, each on its own 16 MB rows of X and Y
};

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
}

// MB: 16-row blocks of X (M <= 16 MB). KS: k tiles (32 each) per wave
// (K = 32 kWaves KS). ACC: add the old Y before the rounding.
template <int MB, int KS, bool ACC, int kWaves>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(kWaves / 4, kWaves / 4)))
decodeGemmKernel(GemmArgs a) {
    extern __shared__ f32x4 part[]; // [2][kWaves][MB][64] partial sums
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int KT = a.K / 32; // tiles per row block
    const int kb0 = wave * KS;
    // M split over mgroups workgroups per row block (small N, large M: the
    // weights are read mgroups times, each workgroup's X is that much smaller).
    const int mg = int(blockIdx.x) % a.mgroups;
    const int first = int(blockIdx.x) / a.mgroups, stride = int(gridDim.x) / a.mgroups;
    a.x += size_t(mg) * 16 * MB * a.K;
    a.y += size_t(mg) * 16 * MB * a.N;
    a.M = min(16 * MB, a.M - mg * 16 * MB);

    // X for the wave's k range and all 16 MB rows, loaded before anything
    // else (loads complete in order, so a later wait on the W ring never has
    // to wait on these). Rows past M read row M - 1; their output columns
    // are computed and dropped, and no other column depends on them.
    // Every workgroup reads all of X at once: rotate which m block and k
    // tile each register slot holds by the workgroup id, so the workgroups
    // of an XCD do not all ask one L2 channel for the same lines. Slot
    // (j, mb) holds k tile kb0 + (j + rk) % KS of m block (mb + rm) % MB;
    // the W ring uses the same k rotation and the epilogue the same m one.
    const int rk = int(blockIdx.x % KS), rm = int((blockIdx.x / KS) % MB);
    auto ktile = [&](int j) { return kb0 + (j + rk) % KS; };
    auto mblock = [&](int mb) { return (mb + rm) % MB; };
    u32x4 xr[KS][MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = min(16 * mblock(mb) + (lane & 15), a.M - 1);
        const uint16_t *xrow = a.x + size_t(m) * a.K + 8 * (lane >> 4);
#pragma unroll
        for (int j = 0; j < KS; ++j) xr[j][mb] = *reinterpret_cast<const u32x4 *>(xrow + 32 * ktile(j));
    }
    // W ring: tile j of the wave's range of the current block.
    u32x4 ring[KS];
    const u32x4 *wbase = a.wp + lane;
#pragma unroll
    for (int j = 0; j < KS; ++j) ring[j] = __builtin_nontemporal_load(wbase + (size_t(first) * KT + ktile(j)) * 64);

    constexpr int kOut = (MB + kWaves - 1) / kWaves; // m blocks this wave finalises (mb = wave + kWaves i)
    int it = 0;
    for (int nb = first; nb < a.nblocks; nb += stride, ++it) {
        const int nxt = nb + stride < a.nblocks ? nb + stride : nb; // past the end: re-read (L2 hit)
        const int n0 = 16 * nb + 4 * (lane >> 4);
        // The epilogue's own loads (old Y) go out before the ring's next
        // loads, so waiting for them never drains the ring.
        uint2 old_y[kOut]; // raw bf16 pairs, widened in the epilogue
#pragma unroll
        for (int i = 0; i < kOut; ++i) {
            old_y[i] = make_uint2(0, 0);
            const int mb = wave + kWaves * i;
            const int m = min(16 * mblock(mb) + (lane & 15), a.M - 1);
            if (ACC && mb < MB) old_y[i] = *reinterpret_cast<const uint2 *>(a.y + size_t(m) * a.N + n0);
        }
        f32x4 acc[MB];
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < KS; ++j) {
            const u32x4 w = ring[j];
            ring[j] = __builtin_nontemporal_load(wbase + (size_t(nxt) * KT + ktile(j)) * 64);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) acc[mb] = mfma(w, xr[j][mb], acc[mb]);
            // one refill, then the tile's MFMAs, in this order
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, MB, 0);
        }
        // Cross-wave sum of the k ranges, in the LDS buffer of this parity.
        f32x4 *buf = part + size_t(it & 1) * kWaves * MB * 64;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) buf[(wave * MB + mb) * 64 + lane] = acc[mb];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kOut; ++i) {
            const int mb = wave + kWaves * i;
            if (mb >= MB) break;
            f32x4 sum = f32x4{__uint_as_float(old_y[i].x << 16), __uint_as_float(old_y[i].x & 0xffff0000u),
                              __uint_as_float(old_y[i].y << 16), __uint_as_float(old_y[i].y & 0xffff0000u)};
#pragma unroll
            for (int v = 0; v < kWaves; ++v) sum += buf[(v * MB + mb) * 64 + lane];
            // lane holds C^T rows n0 + 0..3 of column m
            const int m = 16 * mblock(mb) + (lane & 15);
            if (m < a.M) {
                const __bf16 e0 = (__bf16)sum[0], e1 = (__bf16)sum[1], e2 = (__bf16)sum[2], e3 = (__bf16)sum[3];
                const uint32_t w0 = uint32_t(__builtin_bit_cast(uint16_t, e0)) |
                                    (uint32_t(__builtin_bit_cast(uint16_t, e1)) << 16);
                const uint32_t w1 = uint32_t(__builtin_bit_cast(uint16_t, e2)) |
                                    (uint32_t(__builtin_bit_cast(uint16_t, e3)) << 16);
                *reinterpret_cast<uint2 *>(a.y + size_t(m) * a.N + n0) = make_uint2(w0, w1);
            }
        }
    }
}

// One thread per 16 B of the packed layout: tile (nb, kb), lane l holds
// W[16 nb + l % 16][32 kb + 8 (l / 16) .. + 7], times g[k] when g is given
// (an RMSNorm weight folded into the columns, rounded once to bf16).
__global__ void packKernel(u32x4 *wp, const uint16_t *w, const uint16_t *g, int N, int K) {
    const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int KT = K / 32;
    const size_t total = size_t(N / 16) * KT * 64;
    if (idx >= total) return;
    const int lane = int(idx & 63);
    const size_t tile = idx >> 6;
    const int kb = int(tile % KT);
    const int nb = int(tile / KT);
    const int row = 16 * nb + (lane & 15);
    const int k = 32 * kb + 8 * (lane >> 4);
    u32x4 v = *reinterpret_cast<const u32x4 *>(w + size_t(row) * K + k);
    if (g) {
        const u32x4 gv = *reinterpret_cast<const u32x4 *>(g + k);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float lo = __uint_as_float(v[e] << 16) * __uint_as_float(gv[e] << 16);
            const float hi = __uint_as_float(v[e] & 0xffff0000u) * __uint_as_float(gv[e] & 0xffff0000u);
            const __bf16 blo = (__bf16)lo, bhi = (__bf16)hi;
            v[e] = uint32_t(__builtin_bit_cast(uint16_t, blo)) | (uint32_t(__builtin_bit_cast(uint16_t, bhi)) << 16);
        }
    }
    wp[idx] = v;
}

int computeUnitsOf() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    if (size_t(dev) >= cache.size()) cache.resize(dev + 1, 0);
    if (!cache[dev]) HIP_CHECK(hipDeviceGetAttribute(&cache[dev], hipDeviceAttributeMultiprocessorCount, dev));
    return cache[dev];
}

// Waves per workgroup: the K range splits over them; each holds MB x K / W
// of X in registers. 8 waves (two per SIMD) while that fits in 256
// registers, else 4 (one per SIMD, 512 registers).
template <int MB> constexpr int wavesFor() { return MB <= 4 ? 8 : 4; }

template <int MB> void launchGemm(const GemmArgs &a, hipStream_t s) {
    constexpr int W = wavesFor<MB>();
    constexpr int KS = kDecodeGemmK / (32 * W);
    static const int gdiv = std::getenv("LLAISYS_GEMM_GDIV") ? std::atoi(std::getenv("LLAISYS_GEMM_GDIV")) : 1;
    const int grid = std::max(1, std::min(a.nblocks / gdiv, computeUnitsOf()));
    const size_t lds = size_t(2) * W * MB * 64 * sizeof(f32x4);
    if (a.accumulate)
        hipLaunchKernelGGL((decodeGemmKernel<MB, KS, true, W>), dim3(grid), dim3(64 * W), lds, s, a);
    else
        hipLaunchKernelGGL((decodeGemmKernel<MB, KS, false, W>), dim3(grid), dim3(64 * W), lds, s, a);
}

// Weights of fewer rows than this are latency-bound: past 64 rows of X the
// M range splits over workgroups (4 m blocks each) instead of growing the
// per-workgroup X.
constexpr int kSplitMaxN = 8192;

void launchByM(GemmArgs a, hipStream_t s) {
    if (a.M > 64 && a.N < kSplitMaxN) {
        a.mgroups = (a.M + 63) / 64;
        return launchGemm<4>(a, s);
    }
    a.mgroups = 1;
    switch ((a.M + 15) / 16) {
    case 1: return launchGemm<1>(a, s);
    case 2: return launchGemm<2>(a, s);
    case 3: return launchGemm<3>(a, s);
    case 4: return launchGemm<4>(a, s);
    case 5: return launchGemm<5>(a, s);
    case 6: return launchGemm<6>(a, s);
    case 7: return launchGemm<7>(a, s);
    default: return launchGemm<8>(a, s);
    }
}

} // namespace

bool decodeGemmSupported(int M, int N, int K) {
    return M >= 1 && M <= kDecodeGemmMaxM && N >= 16 && N % 16 == 0 && K == kDecodeGemmK;
}

size_t packedWeightElems(int N, int K) { return size_t(N) * K; }

void packWeight(uint16_t *packed, const uint16_t *w, const uint16_t *fold_g, int N, int K, void *stream) {
    LLAISYS_CHECK(N % 16 == 0 && K % 32 == 0, "packWeight: N % 16 and K % 32 must be 0 (N=" << N << ", K=" << K << ")");
    const size_t total = size_t(N / 16) * (K / 32) * 64;
    if (!total) return;
    hipLaunchKernelGGL(packKernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<u32x4 *>(packed), w, fold_g, N, K);
    HIP_CHECK(hipGetLastError());
}

void decodeGemm(uint16_t *y, const uint16_t *x, const uint16_t *packed, int M, int N, int K, bool accumulate,
                void *stream) {
    LLAISYS_CHECK(decodeGemmSupported(M, N, K),
                  "decodeGemm: unsupported shape M=" << M << " N=" << N << " K=" << K);
    GemmArgs a{y, x, reinterpret_cast<const u32x4 *>(packed), M, N, K, N / 16, accumulate ? 1 : 0, 1};
    launchByM(a, static_cast<hipStream_t>(stream));
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
