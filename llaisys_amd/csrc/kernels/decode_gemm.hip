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
// Double-buffered partials make that the only barrier per block. Given
// argmax_keys, the epilogue also keeps each row's maximum (the LM head).
//
// Further down, the kernels of the batched decode step whose X comes packed
// in the same operand order (packedRowIndex; its producers write that copy):
// packedXGemm (32 x 32 tiles, qkv and o), qkvRopeGemm (qkv with the QKV
// epilogue), gateUpSwiglu (gate-up, row 1/rms and SwiGLU over interleaved
// gate/up weights) and splitKPackedGemm (the down projection); and the
// LDS-staged split-K GEMM for long K with row-major X.
#include "lanes.hpp"
#include "launch.hpp"
#include "step_common.hpp"

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
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// ss + x.lo^2 + x.hi^2 for a word of two bf16 values (one v_dot2 instruction).
__device__ __forceinline__ float addSquares(float ss, uint32_t w) {
    const bf16x2 v = __builtin_bit_cast(bf16x2, w);
    return __builtin_amdgcn_fdot2_f32_bf16(v, v, ss, false);
}


// silu(g) * u with the hardware exp2 and reciprocal (each ~1 ulp; the
// result is rounded to bf16, 2^-9).
__device__ __forceinline__ float siluTimes(float g, float u) {
    return u * g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

struct GemmArgs {
    uint16_t *y;
    const uint16_t *x;
    const u32x4 *wp;     // packed W
    int M, N, K, nblocks, accumulate;
    int mgroups; // workgroups per row block, each on its own 16 MB rows of X and Y
    uint64_t *keys; // non-null (mgroups == 1): argmax key of each row over the workgroup's columns,
                    // keys[m * gridDim.x + blockIdx.x]
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
    // The mgroups workgroups of one row-block walk sit on one XCD (ids
    // congruent mod 8), so the walk's W tiles come from HBM once and from
    // that XCD's L2 for the other row groups.
    int mg, first;
    const int stride = int(gridDim.x) / a.mgroups;
    if (stride % 8 == 0) {
        const int j = int(blockIdx.x) / 8;
        mg = j % a.mgroups;
        first = (j / a.mgroups) * 8 + int(blockIdx.x) % 8;
    } else {
        mg = int(blockIdx.x) % a.mgroups;
        first = int(blockIdx.x) / a.mgroups;
    }
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
    // Running maximum of the rounded outputs and its column, per m block
    // (a.keys): a lane's columns only grow, so a strict > keeps the first
    // maximum, and a NaN beats any number (torch's argmax).
    float best_v[kOut];
    int best_c[kOut];
#pragma unroll
    for (int i = 0; i < kOut; ++i) {
        best_v[i] = -INFINITY;
        best_c[i] = -1;
    }
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
                if (a.keys) {
                    const float ev[4] = {float(e0), float(e1), float(e2), float(e3)};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const bool take = ev[q] != ev[q] ? best_v[i] == best_v[i] : ev[q] > best_v[i];
                        best_v[i] = take ? ev[q] : best_v[i];
                        best_c[i] = take ? n0 + q : best_c[i];
                    }
                }
            }
        }
    }
    if (a.keys) {
        // Lanes l, l ^ 16, l ^ 32, l ^ 48 hold the same row m.
#pragma unroll
        for (int i = 0; i < kOut; ++i) {
            uint64_t k = best_c[i] < 0 ? 0 : argmaxKey(best_v[i], best_c[i]);
            uint64_t o = __shfl_xor(k, 16);
            k = o > k ? o : k;
            o = __shfl_xor(k, 32);
            k = o > k ? o : k;
            const int mb = wave + kWaves * i;
            const int m = 16 * mblock(mb) + (lane & 15);
            if (mb < MB && lane < 16 && m < a.M) a.keys[size_t(m) * gridDim.x + blockIdx.x] = k;
        }
    }
}

// One thread per 16 B of the packed layout: tile (nb, kb), lane l holds
// W[16 nb + l % 16][32 kb + 8 (l / 16) .. + 7], times g[k] when g is given
// (an RMSNorm weight folded into the columns, rounded once to bf16).
__global__ void packKernel(u32x4 *wp, const uint16_t *w, const uint16_t *g, int N, int K, int interleave_di) {
    const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int KT = K / 32;
    const size_t total = size_t(N / 16) * KT * 64;
    if (idx >= total) return;
    const int lane = int(idx & 63);
    const size_t tile = idx >> 6;
    const int kb = int(tile % KT);
    const int nb = int(tile / KT);
    // interleave_di > 0: block nb takes gate rows 8 nb .. + 7 and the up
    // rows interleave_di + 8 nb .. + 7 of a [gate; up] weight.
    const int r16 = lane & 15;
    const int row = interleave_di ? (r16 < 8 ? 8 * nb + r16 : interleave_di + 8 * nb + r16 - 8) : 16 * nb + r16;
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
    const int grid = std::max(1, std::min(a.nblocks, computeUnitsOf()));
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


// ---- Split-K variant for long K (the down projection, K = 8960).
//
// With K long and N short the 16-row blocks are too few to fill the chip, so
// K splits over workgroups instead: workgroup (t, s) computes the partial
// C[128 rows of N, all M] over k tiles [s KT / S, (s + 1) KT / S) into fp32
// partials part[s][m][n], and a reduce kernel sums the S partials in order
// (deterministic), adds the old Y when accumulating and rounds once to bf16.
//  * Each of the 4 waves (one per SIMD) owns 2 of the 8 row blocks of the
//    tile and streams their packed W tiles through a register ring of kRing
//    k steps (2 tiles each), issued first.
//  * X for the workgroup's k range and all M rows is then copied into LDS by
//    global_load_lds, one instruction per row (no registers, no index
//    arithmetic): a row is 64 chunks of 16 B (up to 16 k tiles), chunk c of
//    row m holding k chunk c ^ (m % 16), so the B-operand reads of one k step
//    (16 rows, one chunk column) hit 16 different bank groups.
//  * Per k step a wave reads the next step's MB B operands from LDS, issues
//    2 MB MFMAs on the current ones, then refills the ring slot.
constexpr int kSplitTileRows = 128; // rows of W (N) per workgroup
constexpr int kRing = 8;            // k steps of W in flight per wave
constexpr int kSplitMaxTiles = 16;  // k tiles per split: one 1 KiB LDS row of X

struct SplitKArgs {
    const uint16_t *x;
    const u32x4 *wp;
    float *part;
    int M, N, K, KT, S;
};

template <int MB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) splitKGemmKernel(SplitKArgs a) {
    extern __shared__ u32x4 xs[]; // [16 MB][64] chunks, swizzled
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int t = int(blockIdx.x) / a.S, s = int(blockIdx.x) % a.S;
    const int kt0 = s * a.KT / a.S, nk = (s + 1) * a.KT / a.S - kt0;

    // W ring: row blocks nb0 and nb0 + 1, k step j in slot j % kRing. Past
    // the range a slot re-reads the last step (an L2 hit), so every step
    // issues the same loads.
    const int nb0 = (kSplitTileRows / 16) * t + 2 * wave;
    const u32x4 *w0 = a.wp + (size_t(nb0) * a.KT + kt0) * 64 + lane;
    const u32x4 *w1 = w0 + size_t(a.KT) * 64;
    u32x4 r0[kRing], r1[kRing];
#pragma unroll
    for (int j = 0; j < kRing; ++j) {
        const int jj = min(j, nk - 1);
        r0[j] = __builtin_nontemporal_load(w0 + size_t(jj) * 64);
        r1[j] = __builtin_nontemporal_load(w1 + size_t(jj) * 64);
    }
    // X rows (clamped to M - 1: their columns are computed and dropped);
    // wave w copies rows w, w + 4, ... Lanes past the range fetch the row's
    // first chunk into an unused slot.
    for (int row = wave; row < 16 * MB; row += 4) {
        const int kc = lane ^ (row & 15); // lane l fills chunk l of the row
        const int m = min(row, a.M - 1);
        const int k = 32 * kt0 + 8 * (kc < 4 * nk ? kc : 0);
        __builtin_amdgcn_global_load_lds((const void *)(a.x + size_t(m) * a.K + k),
                                         (__attribute__((address_space(3))) void *)(xs + 64 * row), 16, 0, 0);
    }
    // The compiler does not track these copies: wait for every load of this
    // wave (the ring's too, needed first anyway), then the barrier covers
    // every wave's copies.
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");

    f32x4 acc[2][MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[0][mb] = acc[1][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const u32x4 *xrow = xs + (lane & 15) * 64;
    auto readX = [&](int j, u32x4 (&xv)[MB]) {
        const int c = (4 * j + (lane >> 4)) ^ (lane & 15);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) xv[mb] = xrow[16 * 64 * mb + c];
    };
    // Step j: read step j + 1's B operands, the MFMAs of step j on ring slot
    // r, then the slot's refill with step j + kRing into the same registers
    // (pinned in this order: a refill issued before the MFMAs read the slot
    // would need a second register set, and the loop latch would then copy
    // in-flight load results, draining the ring).
    auto stepK = [&](int j, u32x4 &s0, u32x4 &s1, const u32x4 (&xc)[MB], u32x4 (&xn)[MB]) {
        readX(min(j + 1, nk - 1), xn);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            acc[0][mb] = mfma(s0, xc[mb], acc[0][mb]);
            acc[1][mb] = mfma(s1, xc[mb], acc[1][mb]);
        }
        const int jn = min(j + kRing, nk - 1);
        s0 = __builtin_nontemporal_load(w0 + size_t(jn) * 64);
        s1 = __builtin_nontemporal_load(w1 + size_t(jn) * 64);
        __builtin_amdgcn_sched_group_barrier(0x100, MB, 0);     // next step's B operands
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * MB, 0); // the MFMAs
        __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);      // then the refill
    };
    static_assert(kRing % 2 == 0, "B-operand buffers alternate by slot parity");
    u32x4 xa[MB], xb[MB];
    readX(0, xa);
    // Whole ring passes with no guard, then the remainder.
    const int nfull = nk - nk % kRing;
    for (int j0 = 0; j0 < nfull; j0 += kRing) {
#pragma unroll
        for (int r = 0; r < kRing; r += 2) {
            stepK(j0 + r, r0[r], r1[r], xa, xb);
            stepK(j0 + r + 1, r0[r + 1], r1[r + 1], xb, xa);
        }
    }
#pragma unroll
    for (int r = 0; r < kRing; r += 2) {
        if (nfull + r < nk) stepK(nfull + r, r0[r], r1[r], xa, xb);
        if (nfull + r + 1 < nk) stepK(nfull + r + 1, r0[r + 1], r1[r + 1], xb, xa);
    }
    // Lane holds C rows n0 + 0..3 (of row block nb0 + h) for column m.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int n0 = 16 * (nb0 + h) + 4 * (lane >> 4);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const int m = 16 * mb + (lane & 15);
            if (m < a.M) *reinterpret_cast<f32x4 *>(a.part + (size_t(s) * a.M + m) * a.N + n0) = acc[h][mb];
        }
    }
}

// Y[m, n .. n + 3] = (old Y +) sum over s of part[s][m][n .. n + 3], rounded
// once. Loads of 16 partials are in flight at a time; the sum runs in split
// order.
// (With 10 splits a batch of exactly 10 measured slower, 5.03 against 4.91
// us: the re-reads past S are L2 hits.)
constexpr int kReduceBatch = 16;

__global__ void splitKReduceKernel(uint16_t *y, const float *part, int M, int N, int S, int accumulate,
                                   uint16_t *y_packed) {
    const size_t idx = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int n4 = N / 4;
    if (idx >= size_t(M) * n4) return;
    const int m = int(idx / n4), n = 4 * int(idx % n4);
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    if (accumulate) {
        const uint2 old = *reinterpret_cast<const uint2 *>(y + size_t(m) * N + n);
        sum = f32x4{__uint_as_float(old.x << 16), __uint_as_float(old.x & 0xffff0000u), __uint_as_float(old.y << 16),
                    __uint_as_float(old.y & 0xffff0000u)};
    }
    const size_t stride = size_t(M) * N;
    const float *p = part + size_t(m) * N + n;
    for (int s0 = 0; s0 < S; s0 += kReduceBatch) {
        f32x4 v[kReduceBatch];
#pragma unroll
        for (int i = 0; i < kReduceBatch; ++i)
            v[i] = *reinterpret_cast<const f32x4 *>(p + size_t(min(s0 + i, S - 1)) * stride);
#pragma unroll
        for (int i = 0; i < kReduceBatch; ++i)
            if (s0 + i < S) sum += v[i];
    }
    auto pack = [](float a0, float a1) {
        const __bf16 b0 = (__bf16)a0, b1 = (__bf16)a1;
        return uint32_t(__builtin_bit_cast(uint16_t, b0)) | (uint32_t(__builtin_bit_cast(uint16_t, b1)) << 16);
    };
    const uint2 out = make_uint2(pack(sum[0], sum[1]), pack(sum[2], sum[3]));
    *reinterpret_cast<uint2 *>(y + size_t(m) * N + n) = out;
    if (y_packed) *reinterpret_cast<uint2 *>(y_packed + packedRowIndex(m, n, N)) = out; // 4 elements, one 8 B piece
}

// About one workgroup per CU, at most kSplitMaxTiles k tiles per split (one
// LDS row of X). (Splitting further for small M, so that a workgroup's whole
// W range is in flight at once, measured slower: more partials to reduce.)
int splitsFor(int M, int N, int K) {
    (void)M;
    const int tiles = N / kSplitTileRows, KT = K / 32;
    const int for_cus = (computeUnitsOf() + tiles / 2) / tiles;
    const int for_lds = (KT + kSplitMaxTiles - 1) / kSplitMaxTiles;
    return std::max(1, std::min(KT, std::max(for_cus, for_lds)));
}

template <int MB> void launchSplitK(const SplitKArgs &a, hipStream_t st) {
    const size_t lds = size_t(16) * MB * 64 * sizeof(u32x4);
    hipLaunchKernelGGL((splitKGemmKernel<MB>), dim3((a.N / kSplitTileRows) * a.S), dim3(256), lds, st, a);
}
// Packed-X GEMM: workgroup (mt, nt) owns the 32 x 32 tile of Y at rows
// 32 mt, columns 32 nt; wave w owns k tiles [12 w, 12 w + 12). Each wave
// issues all 24 W tiles and 24 X tiles of its range (1 KiB each, 192
// registers) and the old Y before its first MFMA: at M = 128 the time is
// the workgroup's 192 KiB of operands reaching the CU, which a deeper
// schedule cannot shorten. The four k partials meet in LDS; each wave adds
// one 16 x 16 tile's in wave order (plus the old Y) and rounds once. An m
// block past the last one re-reads the last (its rows are computed and
// dropped).
constexpr int kPxTile = 2;   // 16-row blocks per tile side
constexpr int kPxSteps = 12; // k tiles per wave (K = 4 x 12 x 32)

template <bool ACC>
__global__ void __launch_bounds__(256) packedXGemmKernel(uint16_t *y, const u32x4 *xp, const u32x4 *wp, int M,
                                                         int N, uint16_t *y_packed) {
    static_assert(kPxTile * kPxTile == 4, "one 16 x 16 tile per wave in the epilogue");
    __shared__ f32x4 red[4][kPxTile][kPxTile][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    constexpr int KT = 4 * kPxSteps;
    const int ntiles = N / (16 * kPxTile);
    const int mt = int(blockIdx.x) / ntiles, nt = int(blockIdx.x) % ntiles;
    const int kb0 = wave * kPxSteps;
    const int last_mb = (M - 1) >> 4;
    u32x4 w[kPxSteps][kPxTile], xv[kPxSteps][kPxTile];
#pragma unroll
    for (int j = 0; j < kPxSteps; ++j) {
#pragma unroll
        for (int t = 0; t < kPxTile; ++t)
            w[j][t] = __builtin_nontemporal_load(wp + (size_t(nt * kPxTile + t) * KT + kb0 + j) * 64 + lane);
#pragma unroll
        for (int i = 0; i < kPxTile; ++i) {
            const int mb = min(mt * kPxTile + i, last_mb);
            xv[j][i] = xp[(size_t(mb) * KT + kb0 + j) * 64 + lane];
        }
    }
    // Wave w finishes tile (t, i) = (w / 2, w % 2): lane holds C^T rows
    // n0 + 0..3 of column m. Its old Y goes out behind the operands.
    const int ft = wave >> 1, fi = wave & 1;
    const int m = 16 * (mt * kPxTile + fi) + (lane & 15);
    const int n0 = 16 * (nt * kPxTile + ft) + 4 * (lane >> 4);
    uint2 old_y = make_uint2(0, 0);
    if (ACC) old_y = *reinterpret_cast<const uint2 *>(y + size_t(min(m, M - 1)) * N + n0);
    f32x4 acc[kPxTile][kPxTile];
#pragma unroll
    for (int t = 0; t < kPxTile; ++t)
#pragma unroll
        for (int i = 0; i < kPxTile; ++i) acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kPxSteps; ++j)
#pragma unroll
        for (int t = 0; t < kPxTile; ++t)
#pragma unroll
            for (int i = 0; i < kPxTile; ++i) acc[t][i] = mfma(w[j][t], xv[j][i], acc[t][i]);
#pragma unroll
    for (int t = 0; t < kPxTile; ++t)
#pragma unroll
        for (int i = 0; i < kPxTile; ++i) red[wave][t][i][lane] = acc[t][i];
    __syncthreads();
    if (m >= M) return;
    f32x4 v = ACC ? f32x4{__uint_as_float(old_y.x << 16), __uint_as_float(old_y.x & 0xffff0000u),
                          __uint_as_float(old_y.y << 16), __uint_as_float(old_y.y & 0xffff0000u)}
                  : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) v += red[q][ft][fi][lane]; // the k partials in wave order
    const __bf16 e0 = (__bf16)v[0], e1 = (__bf16)v[1], e2 = (__bf16)v[2], e3 = (__bf16)v[3];
    const uint32_t w0 = uint32_t(__builtin_bit_cast(uint16_t, e0)) | (uint32_t(__builtin_bit_cast(uint16_t, e1)) << 16);
    const uint32_t w1 = uint32_t(__builtin_bit_cast(uint16_t, e2)) | (uint32_t(__builtin_bit_cast(uint16_t, e3)) << 16);
    *reinterpret_cast<uint2 *>(y + size_t(m) * N + n0) = make_uint2(w0, w1);
    if (y_packed) *reinterpret_cast<uint2 *>(y_packed + packedRowIndex(m, n0, N)) = make_uint2(w0, w1);
}

// QKV projection + qkvRopeAppend's epilogue. Workgroup (mt, g) owns rows
// 32 mt .. + 31 and, of head g / 4, the 16-column blocks t and t + 4 (t =
// g % 4): dims d and d + 64 of the head sit in the same lane, so the
// rotation needs no exchange. The operands and the k sweep are those of
// packedXGemmKernel; each wave also sums the squares of the x values it
// loads, per row, for the row's 1/rms; the four waves share the finish.
struct QkvRopeArgs {
    uint16_t *q, *k_pool, *v_pool;
    const uint16_t *bias;
    const int32_t *table, *ctx;
    int nh, nkvh, max_pages, num_blocks, hs;
    float eps, theta;
    int *err;
};

__device__ __forceinline__ uint32_t packBf16(float a, float b) {
    const __bf16 x = (__bf16)a, y = (__bf16)b;
    return uint32_t(__builtin_bit_cast(uint16_t, x)) | (uint32_t(__builtin_bit_cast(uint16_t, y)) << 16);
}

__global__ void __launch_bounds__(256) qkvRopeGemmKernel(const u32x4 *xp, const u32x4 *wp, int M, QkvRopeArgs e) {
    __shared__ f32x4 red[4][2][kPxTile][64];
    __shared__ float ssl[4][16 * kPxTile];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    constexpr int KT = 4 * kPxSteps;
    const int groups = (e.nh + 2 * e.nkvh) * 4;
    const int mt = int(blockIdx.x) / groups, g = int(blockIdx.x) % groups;
    const int head = g >> 2, t4 = g & 3;
    const int kb0 = wave * kPxSteps;
    const int last_mb = (M - 1) >> 4;
    // Wave w finishes m block w % 2 of the tile, elements 2 (w / 2) and
    // 2 (w / 2) + 1 of the lane's four: dims dd, dd + 1 and dd + 64, dd + 65.
    // Its row's position (the sequence's length) and the bias are loaded
    // before the operands, so the angles are worked out while those are in
    // flight; the block-table entry, which needs the position, goes out
    // behind them.
    const int fi = wave & 1, ch = wave >> 1;
    const int m_own = 16 * (mt * kPxTile + fi) + (lane & 15);
    const int pos = e.ctx[min(m_own, M - 1)];
    const int dd = 16 * t4 + 4 * (lane >> 4) + 2 * ch;
    const int c0 = head * kHeadDim + dd;
    const uint32_t bw0 = *reinterpret_cast<const uint32_t *>(e.bias + c0);
    const uint32_t bw1 = *reinterpret_cast<const uint32_t *>(e.bias + c0 + 64);
    u32x4 w[kPxSteps][2], xv[kPxSteps][kPxTile];
#pragma unroll
    for (int j = 0; j < kPxSteps; ++j) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
            w[j][u] = __builtin_nontemporal_load(wp + (size_t(8 * head + t4 + 4 * u) * KT + kb0 + j) * 64 + lane);
#pragma unroll
        for (int i = 0; i < kPxTile; ++i) {
            const int mb = min(mt * kPxTile + i, last_mb);
            xv[j][i] = xp[(size_t(mb) * KT + kb0 + j) * 64 + lane];
        }
    }
    const bool rope = head < e.nh + e.nkvh;
    float sn[2], cs[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        sn[c] = 0.f;
        cs[c] = 1.f;
        if (rope) sincosf(ropePhi(pos, dd + c, kHeadDim, e.theta), &sn[c], &cs[c]);
    }
    const int page = pos >> 4, slot = pos & 15;
    const bool in_table = pos >= 0 && page < e.max_pages;
    const int blk = e.table[size_t(min(m_own, M - 1)) * e.max_pages + (in_table ? page : 0)];
    f32x4 acc[2][kPxTile];
    float ss[kPxTile];
#pragma unroll
    for (int i = 0; i < kPxTile; ++i) {
        ss[i] = 0.f;
        acc[0][i] = acc[1][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < kPxSteps; ++j)
#pragma unroll
        for (int i = 0; i < kPxTile; ++i) {
#pragma unroll
            for (int u = 0; u < 2; ++u) acc[u][i] = mfma(w[j][u], xv[j][i], acc[u][i]);
#pragma unroll
            for (int c = 0; c < 4; ++c) ss[i] = addSquares(ss[i], xv[j][i][c]);
        }
#pragma unroll
    for (int i = 0; i < kPxTile; ++i) ss[i] = sumOverGroups(ss[i]);
    if (lane < 16) {
#pragma unroll
        for (int i = 0; i < kPxTile; ++i) ssl[wave][16 * i + lane] = ss[i];
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int i = 0; i < kPxTile; ++i) red[wave][u][i][lane] = acc[u][i];
    __syncthreads();
    if (m_own >= M) return;
    const int rr = 16 * fi + (lane & 15);
    const float r = rsqrtf((ssl[0][rr] + ssl[1][rr] + ssl[2][rr] + ssl[3][rr]) / float(e.hs) + e.eps);
    float v0[2] = {0.f, 0.f}, v1[2] = {0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) { // the k partials in wave order
        const f32x4 p0 = red[q][0][fi][lane], p1 = red[q][1][fi][lane];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            v0[c] += p0[2 * ch + c];
            v1[c] += p1[2 * ch + c];
        }
    }
    const float b0[2] = {__uint_as_float(bw0 << 16), __uint_as_float(bw0 & 0xffff0000u)};
    const float b1[2] = {__uint_as_float(bw1 << 16), __uint_as_float(bw1 & 0xffff0000u)};
    float y0[2], y1[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const float a = r * v0[c] + b0[c], bb = r * v1[c] + b1[c];
        y0[c] = rope ? a * cs[c] - bb * sn[c] : a;
        y1[c] = rope ? bb * cs[c] + a * sn[c] : bb;
    }
    if (head < e.nh) {
        uint16_t *dst = e.q + (size_t(m_own) * e.nh + head) * kHeadDim + dd;
        *reinterpret_cast<uint32_t *>(dst) = packBf16(y0[0], y0[1]);
        *reinterpret_cast<uint32_t *>(dst + 64) = packBf16(y1[0], y1[1]);
        return;
    }
    // k or v head: the new token's page slot
    if (!in_table || blk < 0 || blk >= e.num_blocks) {
        if (head == e.nh && t4 == 0 && ch == 0 && (lane >> 4) == 0) atomicOr(e.err, in_table ? 1 : 2);
        return;
    }
    if (rope) {
        uint16_t *pg = e.k_pool + (size_t(blk) * e.nkvh + (head - e.nh)) * kPageElems;
        *reinterpret_cast<uint32_t *>(pg + kPageIndex(slot, dd)) = packBf16(y0[0], y0[1]);
        *reinterpret_cast<uint32_t *>(pg + kPageIndex(slot, dd + 64)) = packBf16(y1[0], y1[1]);
    } else {
        uint16_t *pg = e.v_pool + (size_t(blk) * e.nkvh + (head - e.nh - e.nkvh)) * kPageElems;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const __bf16 h0 = (__bf16)y0[c], h1 = (__bf16)y1[c];
            pg[vPageIndex(slot, dd + c)] = __builtin_bit_cast(uint16_t, h0);
            pg[vPageIndex(slot, dd + c + 64)] = __builtin_bit_cast(uint16_t, h1);
        }
    }
}

// Gate-up projection + row 1/rms + SwiGLU over packed x and a
// packWeightGateUp weight. Workgroup g owns NB 16-row blocks (8 act columns
// each) and all M rows; its 4 waves split K (12 k tiles each) and stream W
// and X tiles of one k step together through a kGuRing-deep register ring
// (loads return in issue order, so X issued behind all of W would wait for
// all of W). Every wave also sums the squares of the x values it loads, per
// row; the rows' sums meet in LDS with the partial tiles, and the wave that
// owns m blocks 2w, 2w + 1 adds the four k partials in wave order, scales by
// r, pairs each gate value with its up value (lane l and l ^ 32 hold the
// same columns) and stores act.
constexpr int kGuRing = 2; // (config-5 step: 2: 18.9 us, 3: 19.3, 4: 20.6, 6: spills)
constexpr int kGuRows = 8; // 16-row m blocks (M <= 128)

template <int NB>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
gateUpSwigluKernel(uint16_t *act, const u32x4 *xp, const u32x4 *wp, int M, int di, float eps, int act_packed) {
    constexpr int KT = 4 * kPxSteps, MB = kGuRows, R = kGuRing;
    __shared__ f32x4 red[3][NB][MB][64];
    __shared__ float ssl[4][16 * MB];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int blk0 = int(blockIdx.x) * NB;
    const int kb0 = wave * kPxSteps;
    const int last_mb = (M - 1) >> 4;
    const u32x4 *wl = wp + (size_t(blk0) * KT + kb0) * 64 + lane;
    const u32x4 *xl = xp + size_t(kb0) * 64 + lane;
    u32x4 rw[R][NB], rx[R][MB];
    // Every workgroup reads the same X tiles: each starts its k range at its
    // own step (the sum is the same; the order of the k partials is fixed per
    // workgroup), so those of one XCD do not ask for the same lines at once.
    const int krot = int(blockIdx.x) % kPxSteps;
    auto issue = [&](int st, int j0) {
        const int j = j0 + krot < kPxSteps ? j0 + krot : j0 + krot - kPxSteps;
#pragma unroll
        for (int t = 0; t < NB; ++t) rw[st][t] = __builtin_nontemporal_load(wl + (size_t(t) * KT + j) * 64);
#pragma unroll
        for (int i = 0; i < MB; ++i) rx[st][i] = xl[(size_t(min(i, last_mb)) * KT + j) * 64];
    };
#pragma unroll
    for (int j = 0; j < R; ++j) issue(j, j);
    f32x4 acc[NB][MB];
#pragma unroll
    for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int i = 0; i < MB; ++i) acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float ss[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) ss[i] = 0.f;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kPxSteps; ++j) {
        const int st = j % R;
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int t = 0; t < NB; ++t) acc[t][i] = mfma(rw[st][t], rx[st][i], acc[t][i]);
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) ss[i] = addSquares(ss[i], rx[st][i][e]);
        if (j + R < kPxSteps) issue(st, j + R);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Row m = 16 i + lane % 16: the lane's 8 k per step, then its 4 k groups.
#pragma unroll
    for (int i = 0; i < MB; ++i) ss[i] = sumOverGroups(ss[i]);
    if (lane < 16) {
#pragma unroll
        for (int i = 0; i < MB; ++i) ssl[wave][16 * i + lane] = ss[i];
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int owner = i / 2;
        if (owner == wave) continue;
        const int slot = wave < owner ? wave : wave - 1;
#pragma unroll
        for (int t = 0; t < NB; ++t) red[slot][t][i][lane] = acc[t][i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        if (i / 2 != wave) continue;
        const int m = 16 * i + (lane & 15);
        const float r = rsqrtf((ssl[0][m] + ssl[1][m] + ssl[2][m] + ssl[3][m]) / float(KT * 32) + eps);
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q = 0; q < 4; ++q) v += q == wave ? acc[t][i] : red[q < wave ? q : q - 1][t][i][lane];
            // Lane groups 0, 1 hold gate rows 4 g .. 4 g + 3 of the block, 2, 3
            // the up rows of the same columns; lane < 32 finishes elements
            // 0, 1, lane >= 32 elements 2, 3.
            const bool lo = lane < 32;
            const float p0 = partner32(lo ? v[2] : v[0]), p1 = partner32(lo ? v[3] : v[1]);
            const float g0 = r * (lo ? v[0] : p0), g1 = r * (lo ? v[1] : p1);
            const float u0 = r * (lo ? p0 : v[2]), u1 = r * (lo ? p1 : v[3]);
            const __bf16 b0 = (__bf16)siluTimes(g0, u0);
            const __bf16 b1 = (__bf16)siluTimes(g1, u1);
            const int col = 8 * (blk0 + t) + 4 * ((lane >> 4) & 1) + (lo ? 0 : 2);
            // act_packed: in operand order (the two columns share one 8-column chunk)
            if (m < M)
                *reinterpret_cast<uint32_t *>(act + (act_packed ? packedRowIndex(m, col, di) : size_t(m) * di + col)) =
                    uint32_t(__builtin_bit_cast(uint16_t, b0)) | (uint32_t(__builtin_bit_cast(uint16_t, b1)) << 16);
        }
    }
}

int gateUpBlocksPerGroup(int di) {
    const int blocks = 2 * di / 16;
    return blocks % 5 == 0 ? 5 : blocks % 4 == 0 ? 4 : 0;
}

// Split-K partials over packed X (long K): workgroup (g, s) owns W row
// blocks kSkBlocks g .. + kSkBlocks - 1 and k tiles [4 KSW s, 4 KSW (s + 1));
// its 4 waves split that range (KSW tiles each) and stream W and X of one k
// step together through a kSkRing-deep register ring, as gateUpSwiglu does.
// With X streamed instead of staged in LDS, a workgroup can cover a longer
// k range: fewer splits, so fewer fp32 partials to write and sum. The four
// k partials meet in LDS; the wave that owns m blocks 2w, 2w + 1 adds them in
// wave order and stores part[s][m][n] (m < M).
constexpr int kSkBlocks = 4; // (config-5 down: 4 x 10 splits 11.95 us; 6 x 14: 12.75; 3 x 7: 12.84)
constexpr int kSkRing = 2; // (config-5 step: 2: 11.95 us, 3: 12.04, 4: 12.36)

template <int KSW>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
splitKPackedKernel(float *part, const u32x4 *xp, const u32x4 *wp, int M, int N, int KT, int S) {
    constexpr int NB = kSkBlocks, MB = kGuRows, R = KSW < kSkRing ? KSW : kSkRing;
    __shared__ f32x4 red[3][NB][MB][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int g = int(blockIdx.x) / S, s = int(blockIdx.x) % S;
    const int kb0 = (4 * s + wave) * KSW;
    const int last_mb = (M - 1) >> 4;
    const u32x4 *wl = wp + (size_t(NB * g) * KT + kb0) * 64 + lane;
    const u32x4 *xl = xp + size_t(kb0) * 64 + lane;
    u32x4 rw[R][NB], rx[R][MB];
    // The workgroups of one split read the same X tiles: each starts at its
    // own step of the range (12.26 -> 12.03 us at the config-5 shape).
    const int krot = g % KSW;
    auto issue = [&](int st, int j0) {
        const int j = j0 + krot < KSW ? j0 + krot : j0 + krot - KSW;
#pragma unroll
        for (int t = 0; t < NB; ++t) rw[st][t] = __builtin_nontemporal_load(wl + (size_t(t) * KT + j) * 64);
#pragma unroll
        for (int i = 0; i < MB; ++i) rx[st][i] = xl[(size_t(min(i, last_mb)) * KT + j) * 64];
    };
#pragma unroll
    for (int j = 0; j < R; ++j) issue(j, j);
    f32x4 acc[NB][MB];
#pragma unroll
    for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int i = 0; i < MB; ++i) acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < KSW; ++j) {
        const int st = j % R;
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int t = 0; t < NB; ++t) acc[t][i] = mfma(rw[st][t], rx[st][i], acc[t][i]);
        if (j + R < KSW) issue(st, j + R);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int owner = i / 2;
        if (owner == wave) continue;
        const int slot = wave < owner ? wave : wave - 1;
#pragma unroll
        for (int t = 0; t < NB; ++t) red[slot][t][i][lane] = acc[t][i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        if (i / 2 != wave) continue;
        const int m = 16 * i + (lane & 15);
        if (m >= M) continue;
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int q = 0; q < 4; ++q) v += q == wave ? acc[t][i] : red[q < wave ? q : q - 1][t][i][lane];
            const int n0 = 16 * (NB * g + t) + 4 * (lane >> 4);
            *reinterpret_cast<f32x4 *>(part + (size_t(s) * M + m) * N + n0) = v;
        }
    }
}

// Splits S and k tiles per wave for splitKPackedKernel: the largest S with
// S * (row blocks / kSkBlocks) workgroups on the chip and an instantiated
// KT / (4 S); 0 if none.
int splitKPackedSplits(int N, int K, int *ksw) {
    const int KT = K / 32, groups = N / (16 * kSkBlocks);
    for (int S = 16; S >= 1; --S) {
        if (KT % (4 * S)) continue;
        const int k = KT / (4 * S);
        if ((k == 2 || k == 4 || k == 7 || k == 8) && groups * S <= computeUnitsOf()) {
            *ksw = k;
            return S;
        }
    }
    return 0;
}
} // namespace

bool splitKPackedSupported(int M, int N, int K) {
    int ksw = 0;
    return M >= 1 && M <= 16 * kGuRows && K % 32 == 0 && N % (16 * kSkBlocks) == 0 && K <= kSplitKMaxK &&
           splitKPackedSplits(N, K, &ksw) > 0;
}

size_t splitKPackedWorkspaceBytes(int M, int N, int K) {
    int ksw = 0;
    return size_t(splitKPackedSplits(N, K, &ksw)) * M * N * sizeof(float);
}

void splitKPackedGemm(uint16_t *y, const uint16_t *x_packed, const uint16_t *w_packed, int M, int N, int K,
                      bool accumulate, float *partials, void *stream, uint16_t *y_packed) {
    LLAISYS_CHECK(splitKPackedSupported(M, N, K),
                  "splitKPackedGemm: unsupported shape M=" << M << " N=" << N << " K=" << K);
    int ksw = 0;
    const int S = splitKPackedSplits(N, K, &ksw);
    const dim3 grid(unsigned(N / (16 * kSkBlocks) * S));
    auto st = static_cast<hipStream_t>(stream);
    const auto *xp = reinterpret_cast<const u32x4 *>(x_packed);
    const auto *wp = reinterpret_cast<const u32x4 *>(w_packed);
    switch (ksw) {
    case 2: hipLaunchKernelGGL(splitKPackedKernel<2>, grid, dim3(256), 0, st, partials, xp, wp, M, N, K / 32, S); break;
    case 4: hipLaunchKernelGGL(splitKPackedKernel<4>, grid, dim3(256), 0, st, partials, xp, wp, M, N, K / 32, S); break;
    case 7: hipLaunchKernelGGL(splitKPackedKernel<7>, grid, dim3(256), 0, st, partials, xp, wp, M, N, K / 32, S); break;
    default: hipLaunchKernelGGL(splitKPackedKernel<8>, grid, dim3(256), 0, st, partials, xp, wp, M, N, K / 32, S); break;
    }
    HIP_CHECK(hipGetLastError());
    const size_t threads = size_t(M) * (N / 4);
    hipLaunchKernelGGL(splitKReduceKernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, st, y, partials, M, N,
                       S, accumulate ? 1 : 0, y_packed);
    HIP_CHECK(hipGetLastError());
}

bool qkvRopeGemmSupported(int M, int nh, int nkvh, int K) {
    return nh > 0 && nkvh > 0 && packedXGemmSupported(M, (nh + 2 * nkvh) * kHeadDim, K);
}

void qkvRopeGemm(uint16_t *q, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *x_packed, const uint16_t *w_packed,
                 const uint16_t *bias, const int32_t *table, const int32_t *ctx, int M, int nh, int nkvh, int K,
                 int max_pages, int num_blocks, float eps, float theta, int *err, void *stream) {
    LLAISYS_CHECK(qkvRopeGemmSupported(M, nh, nkvh, K),
                  "qkvRopeGemm: unsupported shape M=" << M << " nh=" << nh << " nkvh=" << nkvh << " K=" << K);
    const QkvRopeArgs e{q, k_pool, v_pool, bias, table, ctx, nh, nkvh, max_pages, num_blocks, K, eps, theta, err};
    const int mtiles = (M + 16 * kPxTile - 1) / (16 * kPxTile);
    const dim3 grid(unsigned(mtiles * (nh + 2 * nkvh) * 4));
    hipLaunchKernelGGL(qkvRopeGemmKernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<const u32x4 *>(x_packed), reinterpret_cast<const u32x4 *>(w_packed), M, e);
    HIP_CHECK(hipGetLastError());
}

bool gateUpSwigluSupported(int M, int di, int K) {
    return M >= 1 && M <= 16 * kGuRows && K == 4 * kPxSteps * 32 && di > 0 && di % 8 == 0 &&
           gateUpBlocksPerGroup(di) > 0;
}

void gateUpSwiglu(uint16_t *act, const uint16_t *x_packed, const uint16_t *w_packed, int M, int di, int K, float eps,
                  void *stream, bool act_packed) {
    LLAISYS_CHECK(gateUpSwigluSupported(M, di, K), "gateUpSwiglu: unsupported shape M=" << M << " di=" << di
                                                                                        << " K=" << K);
    LLAISYS_CHECK(!act_packed || di % 32 == 0, "gateUpSwiglu: a packed output needs di % 32 == 0, got " << di);
    const int nb = gateUpBlocksPerGroup(di);
    const dim3 grid(unsigned(2 * di / 16 / nb));
    auto st = static_cast<hipStream_t>(stream);
    const auto *xp = reinterpret_cast<const u32x4 *>(x_packed);
    const auto *wp = reinterpret_cast<const u32x4 *>(w_packed);
    if (nb == 5)
        hipLaunchKernelGGL(gateUpSwigluKernel<5>, grid, dim3(256), 0, st, act, xp, wp, M, di, eps, act_packed ? 1 : 0);
    else
        hipLaunchKernelGGL(gateUpSwigluKernel<4>, grid, dim3(256), 0, st, act, xp, wp, M, di, eps, act_packed ? 1 : 0);
    HIP_CHECK(hipGetLastError());
}


bool packedXGemmSupported(int M, int N, int K) {
    return M >= 1 && M <= kDecodeGemmMaxM && K == 4 * kPxSteps * 32 && N >= 32 && N % (16 * kPxTile) == 0;
}

void packedXGemm(uint16_t *y, const uint16_t *x_packed, const uint16_t *w_packed, int M, int N, int K,
                 bool accumulate, void *stream, uint16_t *y_packed) {
    LLAISYS_CHECK(packedXGemmSupported(M, N, K),
                  "packedXGemm: unsupported shape M=" << M << " N=" << N << " K=" << K);
    const int mtiles = (M + 16 * kPxTile - 1) / (16 * kPxTile);
    const dim3 grid(unsigned(mtiles * (N / (16 * kPxTile))));
    auto st = static_cast<hipStream_t>(stream);
    const auto *xp = reinterpret_cast<const u32x4 *>(x_packed);
    const auto *wp = reinterpret_cast<const u32x4 *>(w_packed);
    if (accumulate)
        hipLaunchKernelGGL(packedXGemmKernel<true>, grid, dim3(256), 0, st, y, xp, wp, M, N, y_packed);
    else
        hipLaunchKernelGGL(packedXGemmKernel<false>, grid, dim3(256), 0, st, y, xp, wp, M, N, y_packed);
    HIP_CHECK(hipGetLastError());
}

bool decodeGemmSupported(int M, int N, int K) {
    return M >= 1 && M <= kDecodeGemmMaxM && N >= 16 && N % 16 == 0 && K == kDecodeGemmK;
}

size_t packedWeightElems(int N, int K) { return size_t(N) * K; }

void packWeight(uint16_t *packed, const uint16_t *w, const uint16_t *fold_g, int N, int K, void *stream) {
    LLAISYS_CHECK(N % 16 == 0 && K % 32 == 0, "packWeight: N % 16 and K % 32 must be 0 (N=" << N << ", K=" << K << ")");
    const size_t total = size_t(N / 16) * (K / 32) * 64;
    if (!total) return;
    hipLaunchKernelGGL(packKernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<u32x4 *>(packed), w, fold_g, N, K, 0);
    HIP_CHECK(hipGetLastError());
}

void packWeightGateUp(uint16_t *packed, const uint16_t *w, int di, int K, void *stream) {
    LLAISYS_CHECK(di % 8 == 0 && K % 32 == 0,
                  "packWeightGateUp: di % 8 and K % 32 must be 0 (di=" << di << ", K=" << K << ")");
    const size_t total = size_t(2 * di / 16) * (K / 32) * 64;
    if (!total) return;
    hipLaunchKernelGGL(packKernel, dim3(unsigned((total + 255) / 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       reinterpret_cast<u32x4 *>(packed), w, nullptr, 2 * di, K, di);
    HIP_CHECK(hipGetLastError());
}

void decodeGemm(uint16_t *y, const uint16_t *x, const uint16_t *packed, int M, int N, int K, bool accumulate,
                void *stream, uint64_t *argmax_keys) {
    LLAISYS_CHECK(decodeGemmSupported(M, N, K),
                  "decodeGemm: unsupported shape M=" << M << " N=" << N << " K=" << K);
    LLAISYS_CHECK(!argmax_keys || M <= 64 || N >= kSplitMaxN, "decodeGemm: argmax keys need one workgroup per row set");
    GemmArgs a{y, x, reinterpret_cast<const u32x4 *>(packed), M, N, K, N / 16, accumulate ? 1 : 0, 1, argmax_keys};
    launchByM(a, static_cast<hipStream_t>(stream));
    HIP_CHECK(hipGetLastError());
}

int decodeGemmKeyChunks(int N) { return std::max(1, std::min(N / 16, computeUnitsOf())); }

bool splitKGemmSupported(int M, int N, int K) {
    return M >= 1 && M <= kDecodeGemmMaxM && N >= kSplitTileRows && N % kSplitTileRows == 0 && K % 32 == 0 &&
           K > kDecodeGemmK && K <= kSplitKMaxK;
}

size_t splitKWorkspaceBytes(int M, int N, int K) {
    return splitKGemmSupported(M, N, K) ? size_t(splitsFor(M, N, K)) * M * N * sizeof(float) : 0;
}

void splitKGemm(uint16_t *y, const uint16_t *x, const uint16_t *packed, int M, int N, int K, bool accumulate,
                float *partials, void *stream, uint16_t *y_packed) {
    LLAISYS_CHECK(splitKGemmSupported(M, N, K), "splitKGemm: unsupported shape M=" << M << " N=" << N << " K=" << K);
    auto st = static_cast<hipStream_t>(stream);
    SplitKArgs a{x, reinterpret_cast<const u32x4 *>(packed), partials, M, N, K, K / 32, splitsFor(M, N, K)};
    switch ((M + 15) / 16) {
    case 1: launchSplitK<1>(a, st); break;
    case 2: launchSplitK<2>(a, st); break;
    case 3: launchSplitK<3>(a, st); break;
    case 4: launchSplitK<4>(a, st); break;
    case 5: launchSplitK<5>(a, st); break;
    case 6: launchSplitK<6>(a, st); break;
    case 7: launchSplitK<7>(a, st); break;
    default: launchSplitK<8>(a, st); break;
    }
    const size_t threads = size_t(M) * (N / 4);
    hipLaunchKernelGGL(splitKReduceKernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, st, y, partials, M, N,
                       a.S, accumulate ? 1 : 0, y_packed);
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
