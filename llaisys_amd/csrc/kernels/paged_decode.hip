// Batched paged decode attention for gfx950: stream-K flash-decoding.
//
// Work = every (sequence b, kv head h) unit's page pairs, laid end to end:
// unit u = b*nkvh + h owns npairs(b) = ceil(ceil(ctx_b/16)/2) consecutive
// pair indices. A grid of W single-wave workgroups (about one per CU) splits
// the N pairs evenly: wave w takes pairs [w*P, (w+1)*P), P = ceil(N/W) <= 64
// (the last waves take what is left), and
// streams them through a ring of NSTAGE page pairs in flight, crossing unit
// boundaries without draining the ring. Every wave does the same small prefix
// scan of ctx into LDS to find its slice, so no host-side knowledge of the
// lengths and no planning kernel is needed.
//
// A unit whose pairs all fall in one wave is finished by that wave
// (normalised output). Otherwise every wave holding part of it writes a
// record (unnormalised O, running max m, sum l), and the combine kernel,
// launched next on the same stream, merges each split unit's records with
// log-sum-exp weights. A unit spread over at most kUnitSlots waves keeps its
// records in slots of its own (slot k = the wave's place among the unit's
// waves) in a persistent buffer, each with a header holding the record count:
// the combine then finds them without knowing the lengths, in one memory
// round trip, and returns the headers to zero. A unit spread further uses
// per-wave records (slot 0:
// the wave's first unit, slot 1: its last) with slot 0's header set to -1, and
// the combine locates them through the length scan. The kernel boundary makes the records visible to the
// combine on every XCD. (Merging inside this kernel instead needs either
// agent-scope fences, which write back / invalidate a whole L2 per wave, or
// device-scope record traffic plus a serial merge at the tail; both measured
// slower than the second launch.)
//
// Per pair a wave reads 16 KiB of K/V plus the unit's query rows (1 KiB per
// 16 columns, from L2) and issues 24 MFMAs (mfma_common.hpp has the layout).
#include "mfma_common.hpp"
#include "step_common.hpp"

#include "../device/hip_check.hpp"

#include <hip/hip_bf16.h>

#include <algorithm>
#include <cstddef>
#include <cstdlib>
#include <mutex>
#include <vector>

namespace llaisys::kernels {

namespace {

using namespace mfma;

constexpr int kPairsPerWave = 64; // one pair per lane in the wave's block-id window
constexpr int kMergeBatch = 4;    // records whose loads are in flight together
constexpr int kUnitSlots = 8;     // per-unit record slots (units spread over more waves use per-wave records)

struct DecodeArgs {
    const uint16_t *q;
    void *out;
    const uint16_t *k_pool;
    const uint16_t *v_pool;
    const int32_t *table;
    const int32_t *ctx;
    const int32_t *cu_q; // null: query row b is sequence b; else row cu_q[b], and only
                         // sequences with exactly one query are handled here
    float *records;
    int *err;
    int *slot_hdr;   // null: every split unit uses the per-wave records
    float *slot_rec; // kUnitSlots records of G * (kHeadDim + 2) floats per unit
    uint16_t *out_packed; // non-null (bf16 out): rows go there in operand order (packedRowIndex) instead of to out
    int B, T, nh, nkvh, G, max_pages, num_blocks, W;
    float scale_log2;
};

// Dims 16 i + 4 grp .. + 3 (i < 8) of output column block col0 - 4 grp of
// query row `row`, times inv, rounded to bf16 into the packed row copy: one
// 8 B piece each (4 consecutive columns never cross an 8-column chunk).
__device__ __forceinline__ void storePackedPieces(uint16_t *dst, int row, int col0, int K, const f32x4 (&o)[8],
                                                  float inv) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const f32x4 v = o[i] * inv;
        const __bf16 e0 = (__bf16)v[0], e1 = (__bf16)v[1], e2 = (__bf16)v[2], e3 = (__bf16)v[3];
        const uint32_t w0 =
            uint32_t(__builtin_bit_cast(uint16_t, e0)) | (uint32_t(__builtin_bit_cast(uint16_t, e1)) << 16);
        const uint32_t w1 =
            uint32_t(__builtin_bit_cast(uint16_t, e2)) | (uint32_t(__builtin_bit_cast(uint16_t, e3)) << 16);
        *reinterpret_cast<uint2 *>(dst + packedRowIndex(row, col0 + 16 * i, K)) = make_uint2(w0, w1);
    }
}

// Exclusive prefix (over b) of nkvh * npairs(b) into S[0..B], lengths into C,
// query rows into Q. Invalid lengths (< 1 or beyond the block table) count as
// empty and raise kErrTooLong when `report`; so do sequences with more than one
// query when cu_q is given (they are the prefill kernel's), without an error.
// Returns the total pair count N. One wave; the caller synchronises before
// reading S/C/Q from other waves.
__device__ int scanPairs(const DecodeArgs &a, int *S, int *C, int *Q, bool report) {
    const int lane = threadIdx.x & 63;
    int carry = 0;
    for (int base = 0; base < a.B; base += 64) {
        const int bb = base + lane;
        int c = 0, row = bb;
        if (bb < a.B) {
            c = a.ctx[bb];
            bool mine = true;
            if (a.cu_q) {
                row = a.cu_q[bb];
                const int lq = a.cu_q[bb + 1] - row;
                mine = lq == 1;
                if (mine && (row < 0 || row >= a.T)) {
                    if (report) atomicOr(a.err, kErrTooLong);
                    mine = false;
                }
            }
            if (mine && (c < 1 || c > a.max_pages * 16)) {
                if (report) atomicOr(a.err, kErrTooLong);
                mine = false;
            }
            if (!mine) c = 0;
        }
        const int mine_pairs = ((((c + 15) >> 4) + 1) >> 1) * a.nkvh;
        const int incl = waveInclusiveSum(mine_pairs);
        if (bb < a.B) {
            S[bb] = carry + incl - mine_pairs;
            C[bb] = c;
            Q[bb] = row;
        }
        carry += __builtin_amdgcn_readlane(incl, 63);
    }
    if (lane == 0) S[a.B] = carry;
    return carry;
}

// Slices of P = ceil(N / W) pairs: wave w takes [w P, min((w + 1) P, N)), so
// only the last waves can be short or empty.
__device__ __forceinline__ int pairsPerWave(int N, int W) { return (N + W - 1) / W; }
__device__ __forceinline__ int waveStart(int w, int N, int P) { return min(w * P, N); }
// Wave holding pair g (0 <= g < N).
__device__ __forceinline__ int waveOf(int g, int W, int P) { return min(g / P, W - 1); }

// Record r (2 per wave) holds, for the G live columns, O as 128*G floats in
// [blk][col][dims 4*grp .. 4*grp+3] order, so a lane's 16 B access for one
// block lands in a contiguous G*64 B run, then (m, l) per column.
__device__ __forceinline__ float *recordAt(const DecodeArgs &a, int r) {
    return a.records + size_t(r) * a.G * (kHeadDim + 2);
}
__device__ __forceinline__ int recordO(int G, int blk, int col, int grp) { return (blk * G + col) * 16 + grp * 4; }
__device__ __forceinline__ int recordML(int G, int col) { return G * kHeadDim + 2 * col; }

template <int NSTAGE> struct Ring {
    PagePair pp[NSTAGE];
    u32x4 q[NSTAGE][4];
};

// Two stages fit 256 registers (two waves per SIMD); three need the whole
// register file (one wave per SIMD) to avoid spilling. PACKED (bf16): rows
// go to a.out_packed; a separate instance, since the branch in the finish
// cost the plain kernel 14 % (53.8 -> 61.3 us at config 3).
template <bool OUT_F32, int NSTAGE, bool PACKED = false>
__global__ void __launch_bounds__(64)
    __attribute__((amdgpu_waves_per_eu(NSTAGE == 2 ? 2 : 1, NSTAGE == 2 ? 2 : 1))) decodeKernel(DecodeArgs a) {
    extern __shared__ int lds[];
    int *S = lds;
    int *C = lds + a.B + 1;
    int *Q = C + a.B;
    const int lane = threadIdx.x;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int w = blockIdx.x;
    const int G = a.G;

    const int N = scanPairs(a, S, C, Q, w == 0);
    __syncthreads();
    const int P = pairsPerWave(N, a.W);
    const int s = waveStart(w, N, P);
    const int e = waveStart(w + 1, N, P);
    const int cnt = e - s;
    if (cnt <= 0) return;
    if (cnt > kPairsPerWave) { // the host sizes W so this cannot happen
        if (lane == 0) atomicOr(a.err, kErrTooLong);
        return;
    }

    // Block-id window: lane i describes pair s + i. Block ids are range-checked
    // where used (issue): checking here would wait on the loads.
    int lb, lh, lj, bidA, bidB;
    {
        const int g = s + min(lane, cnt - 1);
        int lo = 0, hi = a.B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (S[mid] <= g)
                lo = mid;
            else
                hi = mid - 1;
        }
        lb = lo;
        const int np = (C[lb] + 15) >> 4;
        const int npr = (np + 1) >> 1;
        const int rem = g - S[lb];
        lh = rem / npr;
        lj = rem - lh * npr;
        const int pa = 2 * lj;
        const int pb = min(pa + 1, np - 1);
        const int32_t *row = a.table + size_t(lb) * a.max_pages;
        bidA = row[pa];
        bidB = row[pb];
    }

    // Record slot of this wave in its split units (set after the first issues).
    int slot_k[2] = {0, 0}, slot_n[2] = {0, 0};
    const u32x4 *kp = reinterpret_cast<const u32x4 *>(a.k_pool) + lane;
    const u32x4 *vp = reinterpret_cast<const u32x4 *>(a.v_pool) + lane;
    const int ncol = min(n, G - 1); // columns past G read a valid row and are masked later

    Ring<NSTAGE> ring;
    bool bad_block = false;
    // Pair k of the window into ring slot st; past the end it re-reads the
    // last pair (an L2 hit), so loads are never conditional and the compiler
    // can count them and wait only for the slot about to be consumed.
    auto issue = [&](int st, int k) {
        const int kk = min(k, cnt - 1);
        int bA = __builtin_amdgcn_readlane(bidA, kk);
        int bB = __builtin_amdgcn_readlane(bidB, kk);
        const bool bad = unsigned(bA) >= unsigned(a.num_blocks) || unsigned(bB) >= unsigned(a.num_blocks);
        bad_block |= bad;
        bA = bad ? 0 : bA;
        bB = bad ? 0 : bB;
        const int b = __builtin_amdgcn_readlane(lb, kk);
        const int h = __builtin_amdgcn_readlane(lh, kk);
        loadPair(ring.pp[st], kp, vp, (size_t(bA) * a.nkvh + h) * 256, (size_t(bB) * a.nkvh + h) * 256);
        const uint16_t *qrow = a.q + (size_t(Q[b]) * a.nh + h * G + ncol) * kHeadDim + grp * 8;
#pragma unroll
        for (int t = 0; t < 4; ++t) ring.q[st][t] = *reinterpret_cast<const u32x4 *>(qrow + 32 * t);
    };

    Acc acc;
    acc.reset();
    int cur_b = -1, cur_h = 0;

    auto finish = [&]() {
        float lt = acc.l + __shfl_xor(acc.l, 16);
        lt += __shfl_xor(lt, 32);
        const int np = (C[cur_b] + 15) >> 4;
        const int npr = (np + 1) >> 1;
        const int first = S[cur_b] + cur_h * npr;
        if (first >= s && first + npr <= e) {
            if (n < G) {
                const float inv = 1.f / lt;
                if constexpr (PACKED && !OUT_F32) {
                    storePackedPieces(a.out_packed, Q[cur_b], (cur_h * G + n) * kHeadDim + 4 * grp, a.nh * kHeadDim,
                                      acc.o, inv);
                    return;
                }
                const size_t row = (size_t(Q[cur_b]) * a.nh + cur_h * G + n) * kHeadDim;
#pragma unroll
                for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, row, i, grp, acc.o[i] * inv);
            }
            return;
        }
        // The unit's records: slot k (this wave's place among the unit's
        // waves) of the unit's own slots with a header holding the record
        // count, or, past kUnitSlots waves, this wave's per-wave record with
        // slot 0's header marking the unit as overflowed (-1).
        const int unit = cur_b * a.nkvh + cur_h;
        const int nrec = first < s ? slot_n[0] : slot_n[1];
        float *rec;
        if (nrec <= kUnitSlots) {
            const int k = first < s ? slot_k[0] : slot_k[1];
            rec = a.slot_rec + size_t(unit * kUnitSlots + k) * G * (kHeadDim + 2);
            if (lane == 0) a.slot_hdr[unit * kUnitSlots + k] = nrec;
        } else {
            rec = recordAt(a, 2 * w + (first <= s ? 0 : 1));
            if (a.slot_hdr && first >= s && lane == 0) a.slot_hdr[unit * kUnitSlots] = -1;
        }
        if (n < G) {
#pragma unroll
            for (int i = 0; i < 8; ++i) *reinterpret_cast<f32x4 *>(rec + recordO(G, i, n, grp)) = acc.o[i];
            if (grp == 0) *reinterpret_cast<float2 *>(rec + recordML(G, n)) = make_float2(acc.m, lt);
        }
    };

#pragma unroll
    for (int st = 0; st < NSTAGE; ++st) issue(st, st);
    // The only units of this slice that can be split: the one holding its
    // first pair (if it began in an earlier wave) and the one holding its last
    // (if it continues in a later one). Their record counts and this wave's
    // place among their waves are worked out once, while the first pairs
    // load: index 0 for the unit that began earlier, 1 for the one that began
    // in this slice.
    {
        const int bf = __builtin_amdgcn_readlane(lb, 0), hf = __builtin_amdgcn_readlane(lh, 0);
        const int bl = __builtin_amdgcn_readlane(lb, cnt - 1), hl = __builtin_amdgcn_readlane(lh, cnt - 1);
        const int nf = ((((C[bf] + 15) >> 4) + 1) >> 1), nl = ((((C[bl] + 15) >> 4) + 1) >> 1);
        const int ff = S[bf] + hf * nf, fl = S[bl] + hl * nl;
        auto wv = [&](int g) { return waveOf(g, a.W, P); };
        const int w0f = wv(ff), w0l = fl < s ? w0f : w;
        slot_k[0] = w - w0f;
        slot_n[0] = wv(ff + nf - 1) - w0f + 1;
        slot_k[1] = w - w0l;
        slot_n[1] = wv(fl + nl - 1) - w0l + 1;
        const bool slots = a.slot_hdr != nullptr;
#pragma unroll
        for (int i = 0; i < 2; ++i) slot_n[i] = __builtin_amdgcn_readfirstlane(slots ? slot_n[i] : kUnitSlots + 1);
#pragma unroll
        for (int i = 0; i < 2; ++i) slot_k[i] = __builtin_amdgcn_readfirstlane(slot_k[i]);
    }

    for (int k0 = 0; k0 < cnt; k0 += NSTAGE) {
#pragma unroll
        for (int st = 0; st < NSTAGE; ++st) {
            const int k = k0 + st;
            if (k < cnt) {
                const int b = __builtin_amdgcn_readlane(lb, k);
                const int h = __builtin_amdgcn_readlane(lh, k);
                const int j = __builtin_amdgcn_readlane(lj, k);
                if (b != cur_b || h != cur_h) {
                    if (cur_b >= 0) finish();
                    acc.reset();
                    cur_b = b;
                    cur_h = h;
                }
                const int c = C[b];
                const bool hasB = 2 * j + 1 < ((c + 15) >> 4);
                u32x4 qop[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) qop[t] = n < G ? ring.q[st][t] : u32x4{0, 0, 0, 0};
                consumePair<OUT_F32>(acc, ring.pp[st], qop, 32 * j, c - 1, c, hasB, grp, a.scale_log2);
            }
            issue(st, k + NSTAGE);
        }
    }
    finish();
    if (bad_block && lane == 0) atomicOr(a.err, kErrBadBlock);
}

// Merge the records of every unit that spans more than one wave.
// 256 threads = 4 waves per unit. With record slots, wave v loads slots 2v
// and 2v+1 with their headers (and every wave slot 0's header) in one go and
// merges the valid ones. Without them (or for an overflowed unit) wave 0
// scans the lengths into LDS, lane k works out which per-wave record k of the
// unit lives in (the integer divisions run lane-parallel), and wave v takes
// records v, v+4, ... in batches with all loads of a batch in flight. Merging
// is online (O = sum_r 2^(m_r - M) O_r, l likewise); the four partial states
// meet in LDS and wave 0 writes the output.
constexpr int kCombineWaves = 4;

template <bool OUT_F32, bool PACKED = false>
__global__ void __launch_bounds__(64 * kCombineWaves) decodeCombineKernel(DecodeArgs a) {
    extern __shared__ int lds[];
    int *S = lds;
    int *C = lds + a.B + 1;
    int *Q = C + a.B;
    __shared__ float part_o[kCombineWaves - 1][8][64][4];
    __shared__ float part_ml[kCombineWaves - 1][2][64];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int G = a.G;
    const int u = blockIdx.x;
    const int b = u / a.nkvh;
    const int h = u - b * a.nkvh;
    const int col = min(n, G - 1);
    float M = -INFINITY, L = 0.f;
    f32x4 o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    int row;
    int clear_mask = 0; // this wave's slots whose headers go back to zero (after the barrier below)
    bool per_wave = a.slot_hdr == nullptr;
    if (!per_wave) {
        // The unit's slots: wave v takes slots 2v and 2v+1. Headers, records
        // and the output row are all requested before any of them is used, so
        // the merge waits for one memory round trip.
        int *hdr = a.slot_hdr + u * kUnitSlots;
        const int h0 = hdr[0];
        int hk[2];
        float2 ml[2];
        f32x4 orr[2][8];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int k = 2 * wave + t;
            hk[t] = hdr[k];
            const float *rec = a.slot_rec + size_t(u * kUnitSlots + k) * G * (kHeadDim + 2);
            ml[t] = *reinterpret_cast<const float2 *>(rec + recordML(G, col));
#pragma unroll
            for (int i = 0; i < 8; ++i) orr[t][i] = *reinterpret_cast<const f32x4 *>(rec + recordO(G, i, col, grp));
        }
        row = a.cu_q ? a.cu_q[b] : b;
        if (h0 == 0) return; // unit whole in one wave (or not a decode row): nothing to merge
        if (h0 > 0) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                if (hk[t] <= 0 || ml[t].x == -INFINITY) continue;
                const float Mn = fmaxf(M, ml[t].x);
                const float sa = exp2Fast(M - Mn);
                const float sb = exp2Fast(ml[t].x - Mn);
                L = L * sa + ml[t].y * sb;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[i] = o[i] * sa + orr[t][i] * sb;
                M = Mn;
            }
            clear_mask = (hk[0] != 0 ? 1 : 0) | (hk[1] != 0 ? 2 : 0);
        } else {
            per_wave = true; // overflowed: per-wave records
            clear_mask = wave == 0 ? 1 : 0;
        }
    }
    if (per_wave) {
        if (wave == 0) scanPairs(a, S, C, Q, false);
        __syncthreads();
        const int N = S[a.B];
        const int np = (C[b] + 15) >> 4;
        const int npr = (np + 1) >> 1;
        if (npr == 0) return;
        const int first = S[b] + h * npr;
        const int P = pairsPerWave(N, a.W);
        const int w0 = waveOf(first, a.W, P);
        const int w1 = waveOf(first + npr - 1, a.W, P);
        if (w0 == w1) return;
        row = Q[b];
        for (int base = w0; base <= w1; base += 64) {
            // Lane k: record of wave base+k, or -1 if that wave's range is empty
            // (possible when N < W).
            const int wk = base + lane;
            int rec_k = -1;
            if (wk <= w1) {
                const int st = waveStart(wk, N, P);
                if (waveStart(wk + 1, N, P) > st) rec_k = 2 * wk + ((wk == w0 && st < first) ? 1 : 0);
            }
            const int cnt = min(64, w1 - base + 1);
            for (int k0 = wave * kMergeBatch; k0 < cnt; k0 += kCombineWaves * kMergeBatch) {
                float mr[kMergeBatch], lr[kMergeBatch];
                f32x4 orr[kMergeBatch][8];
#pragma unroll
                for (int t = 0; t < kMergeBatch; ++t) {
                    const int r = __builtin_amdgcn_readlane(rec_k, min(k0 + t, cnt - 1));
                    const float *rec = recordAt(a, r < 0 ? 0 : r);
                    const float2 ml = *reinterpret_cast<const float2 *>(rec + recordML(G, col));
                    mr[t] = ml.x;
                    lr[t] = ml.y;
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        orr[t][i] = *reinterpret_cast<const f32x4 *>(rec + recordO(G, i, col, grp));
                    if (r < 0 || k0 + t >= cnt) mr[t] = -INFINITY; // weight 0
                }
#pragma unroll
                for (int t = 0; t < kMergeBatch; ++t) {
                    if (mr[t] == -INFINITY) continue;
                    const float Mn = fmaxf(M, mr[t]);
                    const float sa = exp2Fast(M - Mn);
                    const float sb = exp2Fast(mr[t] - Mn);
                    L = L * sa + lr[t] * sb;
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = o[i] * sa + orr[t][i] * sb;
                    M = Mn;
                }
            }
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) part_o[wave - 1][i][lane][c] = o[i][c];
        part_ml[wave - 1][0][lane] = M;
        part_ml[wave - 1][1][lane] = L;
    }
    __syncthreads();
    // Every wave has read the unit's headers by now: leave them at zero for
    // the next call.
    if (clear_mask && lane == 0) {
        int *hdr = a.slot_hdr + u * kUnitSlots + 2 * wave;
        if (clear_mask & 1) hdr[0] = 0;
        if (clear_mask & 2) hdr[1] = 0;
    }
    if (wave > 0 || n >= G) return;
#pragma unroll
    for (int v = 0; v < kCombineWaves - 1; ++v) {
        const float mv = part_ml[v][0][lane];
        if (mv == -INFINITY) continue;
        const float Mn = fmaxf(M, mv);
        const float sa = exp2Fast(M - Mn);
        const float sb = exp2Fast(mv - Mn);
        L = L * sa + part_ml[v][1][lane] * sb;
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int c = 0; c < 4; ++c) o[i][c] = o[i][c] * sa + part_o[v][i][lane][c] * sb;
        M = Mn;
    }
    const float inv = 1.f / L;
    if constexpr (PACKED && !OUT_F32) {
        storePackedPieces(a.out_packed, row, (h * G + n) * kHeadDim + 4 * grp, a.nh * kHeadDim, o, inv);
        return;
    }
    const size_t orow = (size_t(row) * a.nh + h * G + n) * kHeadDim;
#pragma unroll
    for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, orow, i, grp, o[i] * inv);
}


// Decode attention with one workgroup per (sequence, kv head) unit: its
// kUnitWaves waves take the unit's page pairs in turn, stream them through a
// register ring into the same MFMA step as the stream-K kernel, and merge
// their (O, m, l) in LDS; wave 0 writes the normalised output. No records and
// no second launch, no length scan: each workgroup reads its own length.
// Balanced only when the units have similar lengths, which the caller
// decides (a decode batch of similar contexts); query row b is sequence b.
//
// With ROPE the kernel also does the step's QKV epilogue for its unit (the
// work of qkvRopeAppend for one decode token): each wave forms the G query
// heads in its own MFMA operand registers from the projection row (scaled by
// the row's 1/rms when the RMSNorm is folded into the weights, plus bias,
// rotated by position ctx - 1). The wave that holds the unit's last pair
// forms the new k and v after its loop, patches them into that pair's
// registers, consumes it and only then stores them into their page slot for
// later steps. The waves start their first pages before the epilogue's
// arithmetic.
//
// Two waves per unit (one workgroup per CU at 128 sequences x 2 kv heads, two
// pairs in flight per wave): 45.5 us per layer in the config-5 step, against
// 48.6 us with 4 waves, 47.0 with 1, 46.5 with 2 waves and 3 pairs in flight,
// 46.1 without the 256-register cap (8 waves had measured slower than 4
// earlier).
constexpr int kUnitWaves = 2;
constexpr int kRopeMaxGroup = 16; // query heads per kv head in the fused epilogue: one MFMA column each

// The new token (slot tok of the last page) written into a loaded page pair's
// registers from wave 0's LDS copy (kf, vf: bf16 by dim): its page is A when
// the pair's first page is the last one (then B repeats A and is masked),
// else B. K: lane L holds token L % 16's chunks [d / 8 = L / 16 + 4 s]; V:
// lanes with L / 16 == tok / 4 hold element (d / 16 % 2) * 4 + tok % 4 of
// dims d = 32 s + 16 p + L % 16 in word 2 p + (tok % 4) / 2 (chosen by
// select: a runtime index into a vector register would go through scratch).
__device__ __forceinline__ void patchNewToken(PagePair &pp, const uint16_t *kf, const uint16_t *vf, int tok,
                                              bool in_a, int lane) {
    if ((lane & 15) == tok) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const u32x4 kn = *reinterpret_cast<const u32x4 *>(kf + 8 * ((lane >> 4) + 4 * s));
            if (in_a) pp.ka[s] = kn;
            pp.kb[s] = kn;
        }
    }
    if ((lane >> 4) == (tok >> 2)) {
        const int wd0 = (tok & 3) >> 1, sh = 16 * (tok & 1);
        const uint32_t keep = ~(0xffffu << sh);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                const bool hit = (wd & 1) == wd0;
                const uint32_t val = uint32_t(vf[32 * s + 16 * (wd >> 1) + (lane & 15)]) << sh;
                pp.va[s][wd] = hit && in_a ? (pp.va[s][wd] & keep) | val : pp.va[s][wd];
                pp.vb[s][wd] = hit ? (pp.vb[s][wd] & keep) | val : pp.vb[s][wd];
            }
    }
}

struct RopeArgs {
    const uint16_t *qkv;  // [B, (nh + 2 nkvh) * 128] projection rows, before bias
    const uint16_t *bias; // [(nh + 2 nkvh) * 128]
    const uint16_t *x;    // [B, hs] residual rows whose RMSNorm is folded in; null: none
    uint16_t *k_pool, *v_pool;
    int hs;
    float eps, theta;
    uint16_t *o_packed; // non-null: the output rows go there in operand order (with or without ROPE)
};

template <bool OUT_F32, int NSTAGE, bool ROPE>
__global__ void __launch_bounds__(64 * kUnitWaves)
    __attribute__((amdgpu_waves_per_eu(NSTAGE == 2 ? 2 : 1, NSTAGE == 2 ? 2 : 1)))
        decodeUnitKernel(DecodeArgs a, RopeArgs r) {
    __shared__ f32x4 part_o[kUnitWaves - 1][8][64];
    __shared__ float part_ml[kUnitWaves - 1][2][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int G = a.G;
    const int u = blockIdx.x;
    const int b = u / a.nkvh;
    const int h = u - b * a.nkvh;
    // Fused epilogue (ROPE) inputs, none of which depends on the length: the
    // projection row's query head h G + n (4 x 16 B of the lane's dims) and
    // its bias; the new token's k dims (lane, lane + 64), v dims (2 lane,
    // 2 lane + 1) and their biases; the row's x for its 1/rms (the
    // projection row stands in when no norm is folded: read, not used).
    const uint16_t *prow = ROPE ? r.qkv + size_t(b) * (a.nh + 2 * a.nkvh) * kHeadDim : nullptr;
    u32x4 qw[4], qb[4];
    uint32_t kw0 = 0, kw1 = 0, kb0 = 0, kb1 = 0, vw = 0, vb = 0;
    RowChunks xr;
    const int xd = r.x ? r.hs : 8;
    auto loadEpilogueInputs = [&]() {
        const int qcol = (h * G + min(n, G - 1)) * kHeadDim + grp * 8;
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            qw[t4] = *reinterpret_cast<const u32x4 *>(prow + qcol + 32 * t4);
            qb[t4] = *reinterpret_cast<const u32x4 *>(r.bias + qcol + 32 * t4);
        }
        const int kcol = (a.nh + h) * kHeadDim, vcol = (a.nh + a.nkvh + h) * kHeadDim;
        kw0 = prow[kcol + lane];
        kw1 = prow[kcol + lane + 64];
        kb0 = r.bias[kcol + lane];
        kb1 = r.bias[kcol + lane + 64];
        vw = *reinterpret_cast<const uint32_t *>(prow + vcol + 2 * lane);
        vb = *reinterpret_cast<const uint32_t *>(r.bias + vcol + 2 * lane);
        xr.load(r.x ? r.x + size_t(b) * r.hs : prow, xd);
    };
    // The waves take the unit's page pairs in turn: wave w owns pairs
    // w, w + kUnitWaves, ... (its k-th pair is unit pair w + kUnitWaves k).
    // So a wave's first block-table window does not depend on the length,
    // and its loads go out beside the length's: the first pages wait for
    // one memory round trip before them instead of two.
    const int32_t *row = a.table + size_t(b) * a.max_pages;
    // Window state: lane i holds the block ids of the wave's pair base + i
    // (windows of up to 64 pairs), read clamped to the table row: entries
    // past the sequence's pages are read but never used (the issue below
    // selects page A for a missing page B, and clamps to the wave's count).
    int base = 0, cnt = 0, bidA = 0, bidB = 0;
    auto loadWindow = [&]() {
        const int pa = 2 * (wave + kUnitWaves * (base + lane));
        bidA = row[min(pa, a.max_pages - 1)];
        bidB = row[min(pa + 1, a.max_pages - 1)];
    };
    if (!ROPE) loadWindow();
    int c = a.ctx[b];
    if (c < 1 || c > a.max_pages * 16) { // invalid length: zero output, error flag
        if (threadIdx.x == 0) atomicOr(a.err, kErrTooLong);
        c = 0;
    }
    c = __builtin_amdgcn_readfirstlane(c);
    const int np = (c + 15) >> 4;
    const int npr = (np + 1) >> 1;
    const int nw = npr > wave ? (npr - wave + kUnitWaves - 1) / kUnitWaves : 0; // this wave's pairs
    cnt = min(kPairsPerWave, nw);
    Acc acc;
    acc.reset();
    bool bad_block = false;
    const u32x4 *kp = reinterpret_cast<const u32x4 *>(a.k_pool) + lane;
    const u32x4 *vp = reinterpret_cast<const u32x4 *>(a.v_pool) + lane;

    PagePair ring[NSTAGE];
    // Pair k of the window into ring slot st (past the window's end its last
    // pair again, an L2 hit, so loads are never conditional).
    auto issue = [&](int st, int k) {
        const int kk = max(min(k, cnt - 1), 0);
        const int j = wave + kUnitWaves * (base + kk); // unit pair
        int bA = __builtin_amdgcn_readlane(bidA, kk);
        int bB = 2 * j + 1 < np ? __builtin_amdgcn_readlane(bidB, kk) : bA;
        const bool bad = unsigned(bA) >= unsigned(a.num_blocks) || unsigned(bB) >= unsigned(a.num_blocks);
        bad_block |= bad && cnt > 0; // a wave with no pairs loads a stand-in
        bA = bad ? 0 : bA;
        bB = bad ? 0 : bB;
        loadPair(ring[st], kp, vp, (size_t(bA) * a.nkvh + h) * 256, (size_t(bB) * a.nkvh + h) * 256);
    };

    u32x4 qop[4];
    // Fused epilogue (ROPE): the wave that holds the unit's last pair forms
    // the new token's k and v after its loop (kflat, vflat: bf16 by dim, in
    // LDS), patches them into that pair and stores them to the pool. Stores
    // count in the same in-order counter as loads, so a store issued before
    // the loop would hold up the waits on every page issued after it.
    __shared__ __align__(16) uint16_t kflat[ROPE ? kHeadDim : 8], vflat[ROPE ? kHeadDim : 8];
    const bool last_wave = ROPE && nw > 0 && (npr - 1) % kUnitWaves == wave;
    const int tok = (c - 1) & 15;
    bool issued = false; // the first window's first stages already in flight
    float rs = 1.f;      // the row's 1/rms (ROPE)
    int blk = 0;         // the new token's block id (ROPE)
    __shared__ float2 trig[ROPE ? kUnitWaves : 1][64];
    if constexpr (ROPE) {
        // Loads return in issue order, so the block-table window and the new
        // token's block id go out first: the wait for them before the first
        // pages' addresses then covers nothing else. The epilogue's inputs
        // follow, then the first pages, with no branch in between (loads
        // clamped to valid addresses, results selected afterwards), so the
        // epilogue's waits count only the loads before the pages.
        const int pos = c - 1;
        loadWindow();
        const bool qlive = c > 0 && n < G;
        // The new token's page (the index goes through a vector register, so
        // the block id stays per lane: moved to a scalar right after its load
        // it would make the wave wait for every load issued before it).
        int slot_page = max(pos, 0) >> 4;
        asm volatile("" : "+v"(slot_page));
        blk = row[slot_page];
        loadEpilogueInputs();
#pragma unroll
        for (int st = 0; st < NSTAGE; ++st) issue(st, st);
        issued = true;
        // (sin, cos) of the 64 rotation angles of position pos: lane (n, grp)
        // works out j = grp * 8 + 32 (n / 8) + n % 8 (the lane's own dims
        // below d/2 are grp * 8 + 32 t + e, t < 2), shared through LDS.
        {
            const int j = grp * 8 + 32 * (n >> 3) + (n & 7);
            float sn, cs;
            sincosf(ropePhi(pos, j, kHeadDim, r.theta), &sn, &cs);
            trig[wave][lane] = make_float2(sn, cs);
        }
        const float ss = xr.sumSquares(r.x ? r.x + size_t(b) * r.hs : prow, xd);
        rs = r.x ? rsqrtf(ss / float(r.hs) + r.eps) : 1.f;
        __builtin_amdgcn_wave_barrier();
        // Query: rotate (j, j + 64) for the lane's 16 j; word w of chunk t4
        // holds dims grp * 8 + 32 t4 + 2 w, + 1, chunk t4 + 2 their partners.
#pragma unroll
        for (int t4 = 0; t4 < 2; ++t4)
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                uint32_t lo_out = 0, hi_out = 0;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float2 sc = trig[wave][grp * 16 + t4 * 8 + 2 * wd + e];
                    const int sh = e ? 0 : 16;
                    const float x0 = rs * __uint_as_float((qw[t4][wd] << sh) & 0xffff0000u) +
                                     __uint_as_float((qb[t4][wd] << sh) & 0xffff0000u);
                    const float x1 = rs * __uint_as_float((qw[t4 + 2][wd] << sh) & 0xffff0000u) +
                                     __uint_as_float((qb[t4 + 2][wd] << sh) & 0xffff0000u);
                    const uint32_t r0 = __builtin_bit_cast(uint16_t, __float2bfloat16(x0 * sc.y - x1 * sc.x));
                    const uint32_t r1 = __builtin_bit_cast(uint16_t, __float2bfloat16(x1 * sc.y + x0 * sc.x));
                    lo_out |= r0 << (16 * e);
                    hi_out |= r1 << (16 * e);
                }
                qop[t4][wd] = lo_out;
                qop[t4 + 2][wd] = hi_out;
            }
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) qop[t4] = qlive ? qop[t4] : u32x4{0, 0, 0, 0};
    } else {
        const uint16_t *qrow = a.q + (size_t(b) * a.nh + h * G + min(n, G - 1)) * kHeadDim + grp * 8;
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            qop[t4] = *reinterpret_cast<const u32x4 *>(qrow + 32 * t4);
            qop[t4] = n < G ? qop[t4] : u32x4{0, 0, 0, 0};
        }
    }
    for (; base < nw; base += kPairsPerWave) {
        cnt = min(kPairsPerWave, nw - base);
        if (base != 0) loadWindow();
        if (!issued) {
#pragma unroll
            for (int st = 0; st < NSTAGE; ++st) issue(st, st);
        }
        issued = false;
        // The fused epilogue's last wave leaves the unit's last pair to the
        // tail below (the patch stays out of the loop's registers).
        const int cnt_c = cnt - (last_wave && base + cnt == nw ? 1 : 0);
        for (int k0 = 0; k0 < cnt; k0 += NSTAGE) {
#pragma unroll
            for (int st = 0; st < NSTAGE; ++st) {
                const int k = k0 + st;
                if (k < cnt_c) {
                    const int j = wave + kUnitWaves * (base + k);
                    consumePair<OUT_F32>(acc, ring[st], qop, 32 * j, c - 1, c, 2 * j + 1 < np, grp, a.scale_log2);
                }
                issue(st, k + NSTAGE);
            }
        }
    }
    if constexpr (ROPE) {
        // Past the window's end every ring slot re-reads its last pair, so
        // slot 0 holds the unit's last pair: form the new token's k and v,
        // patch them in, consume, then store them into the page slot.
        if (last_wave) {
            // k: lane j rotates (j, j + 64) with the angle lane
            // (j / 8 % 4) * 16 + (j / 32) * 8 + j % 8 worked out; v: 2 dims.
            const float2 sc = trig[wave][((lane >> 3) & 3) * 16 + (lane >> 5) * 8 + (lane & 7)];
            const float x0 = rs * __uint_as_float(kw0 << 16) + __uint_as_float(kb0 << 16);
            const float x1 = rs * __uint_as_float(kw1 << 16) + __uint_as_float(kb1 << 16);
            const uint16_t k0 = __builtin_bit_cast(uint16_t, __float2bfloat16(x0 * sc.y - x1 * sc.x));
            const uint16_t k1 = __builtin_bit_cast(uint16_t, __float2bfloat16(x1 * sc.y + x0 * sc.x));
            const uint16_t v0 = __builtin_bit_cast(
                uint16_t, __float2bfloat16(rs * __uint_as_float(vw << 16) + __uint_as_float(vb << 16)));
            const uint16_t v1 = __builtin_bit_cast(
                uint16_t, __float2bfloat16(rs * __uint_as_float(vw & 0xffff0000u) + __uint_as_float(vb & 0xffff0000u)));
            kflat[lane] = k0;
            kflat[lane + 64] = k1;
            vflat[2 * lane] = v0;
            vflat[2 * lane + 1] = v1;
            __builtin_amdgcn_wave_barrier();
            const int j = npr - 1;
            patchNewToken(ring[0], kflat, vflat, tok, 2 * j == np - 1, lane);
            consumePair<OUT_F32>(acc, ring[0], qop, 32 * j, c - 1, c, 2 * j + 1 < np, grp, a.scale_log2);
            // Stores into the page slot for later steps: lanes 0-15 the k
            // chunks [d / 8][tok] (16 B each), every lane its 2 v dims.
            if (unsigned(blk) >= unsigned(a.num_blocks)) {
                if (lane == 0) atomicOr(a.err, kErrBadBlock);
            } else {
                const size_t page = (size_t(blk) * a.nkvh + h) * kPageElems;
                if (lane < 16)
                    *reinterpret_cast<u32x4 *>(r.k_pool + page + kPageIndex(tok, 8 * lane)) =
                        *reinterpret_cast<const u32x4 *>(&kflat[8 * lane]);
                r.v_pool[page + vPageIndex(tok, 2 * lane)] = v0;
                r.v_pool[page + vPageIndex(tok, 2 * lane + 1)] = v1;
            }
        }
    }
    if (bad_block && lane == 0) atomicOr(a.err, kErrBadBlock);
    float lt = acc.l + __shfl_xor(acc.l, 16);
    lt += __shfl_xor(lt, 32);
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) part_o[wave - 1][i][lane] = acc.o[i];
        part_ml[wave - 1][0][lane] = acc.m;
        part_ml[wave - 1][1][lane] = lt;
    }
    __syncthreads();
    if (wave > 0 || n >= G) return;
    float M = acc.m, L = lt;
#pragma unroll
    for (int v = 0; v < kUnitWaves - 1; ++v) {
        const float mv = part_ml[v][0][lane];
        if (mv == -INFINITY) continue;
        const float Mn = fmaxf(M, mv);
        const float sa = exp2Fast(M - Mn);
        const float sb = exp2Fast(mv - Mn);
        L = L * sa + part_ml[v][1][lane] * sb;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc.o[i] = acc.o[i] * sa + part_o[v][i][lane] * sb;
        M = Mn;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f; // no keys (invalid length): zeros
    if (!OUT_F32 && r.o_packed) {
        // Dims 16 i + 4 grp .. + 3 of head h G + n: one 8 B piece of the
        // packed row (4 consecutive columns never cross an 8-column chunk).
        const int col0 = (h * G + n) * kHeadDim + 4 * grp;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const f32x4 v = acc.o[i] * inv;
            const __bf16 e0 = (__bf16)v[0], e1 = (__bf16)v[1], e2 = (__bf16)v[2], e3 = (__bf16)v[3];
            const uint32_t w0 =
                uint32_t(__builtin_bit_cast(uint16_t, e0)) | (uint32_t(__builtin_bit_cast(uint16_t, e1)) << 16);
            const uint32_t w1 =
                uint32_t(__builtin_bit_cast(uint16_t, e2)) | (uint32_t(__builtin_bit_cast(uint16_t, e3)) << 16);
            *reinterpret_cast<uint2 *>(r.o_packed + packedRowIndex(b, col0 + 16 * i, a.nh * kHeadDim)) =
                make_uint2(w0, w1);
        }
        return;
    }
    const size_t orow = (size_t(b) * a.nh + h * G + n) * kHeadDim;
#pragma unroll
    for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, orow, i, grp, acc.o[i] * inv);
}

int envInt(const char *name, int fallback) {
    const char *v = std::getenv(name);
    return (v && *v) ? std::atoi(v) : fallback;
}

int computeUnits() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    if (size_t(dev) >= cache.size()) cache.resize(dev + 1, 0);
    if (!cache[dev]) HIP_CHECK(hipDeviceGetAttribute(&cache[dev], hipDeviceAttributeMultiprocessorCount, dev));
    return cache[dev];
}

} // namespace

// Device workspace of pagedDecodeNoAlloc (llaisysPagedAttentionNoAlloc):
// split records of the decode kernel, in a fixed array each GPU holds for the
// life of the process instead of runtime allocations. In host code `scratch`
// names a host-side stand-in; kernels get the device address that
// hipGetSymbolAddress returns, looked up once per device by noAllocInit().
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};
} // namespace

void noAllocInit() {
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    LLAISYS_CHECK(dev >= 0 && dev < kMaxDevices, "device id " << dev << " beyond " << kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev]) return;
    void *ptr = nullptr;
    HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    LLAISYS_CHECK(ptr != nullptr, "hipGetSymbolAddress returned no address for the decode scratch");
    computeUnits(); // cached per device here, so the entry point's plan only reads it
    g_scratch_ptr[dev] = ptr;
}

size_t noAllocScratchBytes() { return kNoAllocScratchBytes; }

void pagedDecodeNoAlloc(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                        const int32_t *block_table, const int32_t *ctx_len, int B, int nh, int nkvh, int max_pages,
                        int num_blocks, float scale, int *err, void *stream) {
    if (B == 0) return;
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    void *ptr = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        ptr = dev >= 0 && dev < kMaxDevices ? g_scratch_ptr[dev] : nullptr;
    }
    LLAISYS_CHECK(ptr, "paged_attention_no_alloc: device " << dev << " is not set up (noAllocInit)");
    const int G = nh / nkvh;
    const size_t esz = out_f32 ? 4 : 2;
    // Sequences in chunks whose length prefix fits the kernel's LDS; the
    // chunks run one after another on the stream and reuse the records.
    for (int b0 = 0; b0 < B; b0 += kDecodeMaxBatch) {
        const int Bc = std::min(kDecodeMaxBatch, B - b0);
        DecodePlan plan = planDecode(Bc, nkvh, G, max_pages);
        plan.slot_headers = 0; // per-wave records only: nothing to keep zeroed between calls
        plan.slot_record_bytes = 0;
        LLAISYS_CHECK(plan.record_bytes <= kNoAllocScratchBytes,
                      "paged_attention_no_alloc: " << Bc << " sequences x " << nkvh << " kv heads x " << max_pages
                          << " pages need " << plan.record_bytes << " bytes of split records, more than the "
                          << kNoAllocScratchBytes << "-byte scratch; use llaisysPagedAttention");
        pagedDecode(static_cast<std::byte *>(out) + size_t(b0) * nh * kHeadDim * esz, out_f32,
                    q + size_t(b0) * nh * kHeadDim, k_pool, v_pool, block_table + size_t(b0) * max_pages,
                    ctx_len + b0, nullptr, Bc, Bc, nh, nkvh, max_pages, num_blocks, scale, plan,
                    static_cast<float *>(ptr), err, nullptr, nullptr, stream);
    }
}

DecodePlan planDecode(int B, int nkvh, int group, int max_pages) {
    DecodePlan p{};
    const long long max_pairs = (long long)B * nkvh * ((max_pages + 1) / 2);
    // 1.75 waves per CU: measured best for the model's 128 x ~2100-token
    // batches (3.54 ms per step against 3.56-3.60 at 1.5 and 3.56 at 2 waves
    // per CU; 1 wave per CU was 3 % slower than 1.5), slightly ahead for the
    // mixed batch and neutral for the config-3 batch (53.15 us at 1.5 or 1.75).
    const int fill = std::max(1, envInt("LLAISYS_DECODE_WAVES", computeUnits() * 7 / 4));
    p.waves = int(std::max<long long>(fill, (max_pairs + kPairsPerWave - 1) / kPairsPerWave));
    p.record_bytes = size_t(2) * p.waves * group * (kHeadDim + 2) * sizeof(float);
    p.lds_bytes = size_t(3 * B + 1) * sizeof(int);
    p.stages = envInt("LLAISYS_DECODE_STAGES", 2) >= 3 ? 3 : 2;
    // Per-unit record slots, unless disabled or implausibly large.
    const size_t slots = size_t(B) * nkvh * kUnitSlots;
    const size_t rec_bytes = slots * group * (kHeadDim + 2) * sizeof(float);
    const bool use = envInt("LLAISYS_DECODE_SLOTS", 1) != 0 && rec_bytes <= (size_t(1) << 30);
    p.slot_headers = use ? slots : 0;
    p.slot_record_bytes = use ? rec_bytes : 0;
    return p;
}

void pagedDecode(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                 const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_q, int B, int T, int nh,
                 int nkvh, int max_pages,
                 int num_blocks, float scale, const DecodePlan &plan, float *records, int *err,
                 int *slot_headers, void *slot_records, void *stream, uint16_t *out_packed) {
    if (B == 0) return;
    DecodeArgs a;
    a.q = q;
    a.out = out;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.table = block_table;
    a.ctx = ctx_len;
    a.cu_q = cu_q;
    a.records = records;
    a.err = err;
    LLAISYS_CHECK(!out_packed || (!out_f32 && (nh * kHeadDim) % 32 == 0),
                  "pagedDecode: a packed output needs bf16 and nh * 128 % 32 == 0");
    a.out_packed = out_packed;
    const bool slots = plan.slot_headers && slot_headers && slot_records;
    a.slot_hdr = slots ? slot_headers : nullptr;
    a.slot_rec = slots ? static_cast<float *>(slot_records) : nullptr;
    a.B = B;
    a.T = T;
    a.nh = nh;
    a.nkvh = nkvh;
    a.G = nh / nkvh;
    a.max_pages = max_pages;
    a.num_blocks = num_blocks;
    a.W = plan.waves;
    a.scale_log2 = scale * 1.4426950408889634f;
    auto s = static_cast<hipStream_t>(stream);
    const unsigned lds = unsigned(plan.lds_bytes);
    const dim3 grid(plan.waves), block(64), comb(B * nkvh), comb_block(64 * kCombineWaves);
    if (out_f32) {
        if (plan.stages == 3)
            hipLaunchKernelGGL((decodeKernel<true, 3>), grid, block, lds, s, a);
        else
            hipLaunchKernelGGL((decodeKernel<true, 2>), grid, block, lds, s, a);
        hipLaunchKernelGGL((decodeCombineKernel<true>), comb, comb_block, lds, s, a);
    } else {
        if (out_packed) {
            if (plan.stages == 3)
                hipLaunchKernelGGL((decodeKernel<false, 3, true>), grid, block, lds, s, a);
            else
                hipLaunchKernelGGL((decodeKernel<false, 2, true>), grid, block, lds, s, a);
            hipLaunchKernelGGL((decodeCombineKernel<false, true>), comb, comb_block, lds, s, a);
        } else {
            if (plan.stages == 3)
                hipLaunchKernelGGL((decodeKernel<false, 3>), grid, block, lds, s, a);
            else
                hipLaunchKernelGGL((decodeKernel<false, 2>), grid, block, lds, s, a);
            hipLaunchKernelGGL((decodeCombineKernel<false>), comb, comb_block, lds, s, a);
        }
    }
    HIP_CHECK(hipGetLastError());
}

namespace {
void launchDecodeUnits(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                       const int32_t *block_table, const int32_t *ctx_len, int B, int nh, int nkvh, int max_pages,
                       int num_blocks, float scale, int *err, const RopeArgs &r, bool rope, void *stream) {
    if (B == 0) return;
    DecodeArgs a{};
    a.q = q;
    a.out = out;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.table = block_table;
    a.ctx = ctx_len;
    a.err = err;
    a.B = B;
    a.T = B;
    a.nh = nh;
    a.nkvh = nkvh;
    a.G = nh / nkvh;
    a.max_pages = max_pages;
    a.num_blocks = num_blocks;
    a.scale_log2 = scale * 1.4426950408889634f;
    // Two page pairs in flight per wave (see kUnitWaves for the measurements).
    auto s = static_cast<hipStream_t>(stream);
    const dim3 grid(unsigned(B) * unsigned(nkvh)), block(64 * kUnitWaves);
    if (rope) {
        if (out_f32)
            hipLaunchKernelGGL((decodeUnitKernel<true, 2, true>), grid, block, 0, s, a, r);
        else
            hipLaunchKernelGGL((decodeUnitKernel<false, 2, true>), grid, block, 0, s, a, r);
    } else {
        if (out_f32)
            hipLaunchKernelGGL((decodeUnitKernel<true, 2, false>), grid, block, 0, s, a, r);
        else
            hipLaunchKernelGGL((decodeUnitKernel<false, 2, false>), grid, block, 0, s, a, r);
    }
    HIP_CHECK(hipGetLastError());
}
} // namespace

void pagedDecodeUnits(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                      const int32_t *block_table, const int32_t *ctx_len, int B, int nh, int nkvh, int max_pages,
                      int num_blocks, float scale, int *err, void *stream, uint16_t *out_packed) {
    LLAISYS_CHECK(!out_packed || (!out_f32 && (nh * kHeadDim) % 32 == 0),
                  "pagedDecodeUnits: a packed output is bf16 with nh * 128 % 32 == 0");
    RopeArgs r{};
    r.o_packed = out_packed;
    launchDecodeUnits(out, out_f32, q, k_pool, v_pool, block_table, ctx_len, B, nh, nkvh, max_pages, num_blocks,
                      scale, err, r, false, stream);
}

bool decodeUnitsRopeSupported(int nh, int nkvh, int d) {
    return d == kHeadDim && nkvh > 0 && nh % nkvh == 0 && nh / nkvh <= kRopeMaxGroup;
}

void pagedDecodeUnitsRope(void *out, bool out_f32, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *qkv,
                          const uint16_t *bias, const uint16_t *x, int hs, float eps, float theta,
                          const int32_t *block_table, const int32_t *ctx_len, int B, int nh, int nkvh, int max_pages,
                          int num_blocks, float scale, int *err, void *stream, uint16_t *out_packed) {
    LLAISYS_CHECK(decodeUnitsRopeSupported(nh, nkvh, kHeadDim),
                  "pagedDecodeUnitsRope: " << nh << " query heads over " << nkvh << " kv heads exceed "
                                           << kRopeMaxGroup << " per kv head");
    LLAISYS_CHECK(!x || (hs > 0 && hs % 8 == 0), "pagedDecodeUnitsRope: hidden size must be a positive multiple of 8");
    LLAISYS_CHECK(!out_packed || (!out_f32 && (nh * kHeadDim) % 32 == 0),
                  "pagedDecodeUnitsRope: a packed output is bf16 with nh * 128 % 32 == 0");
    const RopeArgs r{qkv, bias, x, k_pool, v_pool, hs, eps, theta, out_packed};
    launchDecodeUnits(out, out_f32, nullptr, k_pool, v_pool, block_table, ctx_len, B, nh, nkvh, max_pages,
                      num_blocks, scale, err, r, true, stream);
}

} // namespace llaisys::kernels
