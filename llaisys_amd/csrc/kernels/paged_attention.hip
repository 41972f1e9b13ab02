// Chunked-prefill attention over paged KV for gfx950 (the multi-query
// sequences of a mixed batch; single-query sequences go to the decode kernel).
//
// Work unit = (query group, kv head). A query tile is 16 "columns"; column n
// of tile t is the (query row, query head) pair number t*16+n of its
// sequence, pairs ordered query-major: pair = qi*G + g, G = nh/nkvh query
// heads per kv head. A group is kTiles adjacent tiles carried by one wave.
// A workgroup is kWaves waves on kWaves adjacent groups of one sequence and
// kv head ("block"): each K/V page pair is read from L2 once per workgroup
// into LDS (double buffered, one barrier per pair) and feeds kWaves x kTiles
// x 24 MFMAs, and the waves hold no private K/V ring.
// Query qi of a sequence with Lq new tokens sits at position ctx - Lq + qi
// and sees keys at positions <= that (bottom-right causal alignment). A
// block's visible pages (up to its last query) are cut into splits of
// `pages_per_split` pages; one workgroup runs one (block, split): the next
// pair is loaded into registers while the current one is consumed from LDS
// (loads never conditional: past the end they re-read the last pair), into
// the MFMA step of mfma_common.hpp. A unit with one split writes its normalised
// output; with more, each split writes a record (O, m, l) and the combine
// kernel launched next merges them (the kernel boundary orders the records;
// no fences, no waiting between waves).
//
// Two launch forms run the same (block, split) code. By default a persistent
// kernel (prefillQueueKernel, one workgroup per CU) takes the items from a
// device counter, longest first, and for mixed batches of up to 256
// sequences also the single-query sequences (decodeItem), so no decode
// kernel runs beside it. Batches whose item tables do not fit its LDS use one
// workgroup per grid slot (prefillKernel), slot ids split-major over blocks
// padded to a multiple of 8.
#include "mfma_common.hpp"

#include "../device/hip_check.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <vector>

namespace llaisys::kernels {

namespace {

using namespace mfma;

constexpr int kXcds = 8;
constexpr int kTiles = 2;                                    // query tiles per wave
constexpr int kWaves = 8;                                    // waves (groups) per workgroup
constexpr int kStagePairs = 2;                               // page pairs per LDS stage (one barrier each)
constexpr int kRecordFloats = kTiles * 16 * (kHeadDim + 2); // O for the group's columns, then (m, l)

struct Args {
    const uint16_t *q;
    void *out;
    const uint16_t *k_pool;
    const uint16_t *v_pool;
    const int32_t *table;
    const int32_t *ctx;
    const int32_t *cu_q;
    float *records;
    int *err;
    int *queue; // prefillQueueKernel: {next item, workgroups done}, zero between launches
    int with_decode; // pagedPrefill runs prefillQueueKernel<, true>: the single-query sequences too
    int B, T, nh, nkvh, G, max_pages, num_blocks, pps, max_splits, units, block_units, block_units_padded;
    float scale_log2;
};

__device__ __forceinline__ int groupsOf(const Args &a, int bb) {
    const int lq = a.cu_q[bb + 1] - a.cu_q[bb];
    return lq >= 2 ? (((lq * a.G + 15) >> 4) + kTiles - 1) / kTiles : 0;
}

// Item `index` of the list where each sequence with Lq >= 2 contributes its
// groups (blocks == false) or its blocks of kWaves groups (blocks == true):
// its sequence b, index within the sequence, and the number of groups of the
// sequences before b. Returns false past the last item. One wave.
__device__ bool locate(const Args &a, int index, bool blocks, int &b, int &local, int &group_base) {
    const int lane = threadIdx.x & 63;
    int remaining = index, groups_before = 0;
    for (int base = 0; base < a.B; base += 64) {
        const int bb = base + lane;
        const int ng = bb < a.B ? groupsOf(a, bb) : 0;
        const int ni = blocks ? (ng + kWaves - 1) / kWaves : ng;
        const int incl = waveInclusiveSum(ni), gincl = waveInclusiveSum(ng);
        const int total = __builtin_amdgcn_readlane(incl, 63);
        if (remaining < total) {
            const unsigned long long hit = __ballot(incl > remaining);
            const int first = __builtin_amdgcn_readfirstlane(__ffsll(hit) - 1);
            b = base + first;
            local = remaining - (__builtin_amdgcn_readlane(incl, first) - __builtin_amdgcn_readlane(ni, first));
            group_base = groups_before + __builtin_amdgcn_readlane(gincl, first) - __builtin_amdgcn_readlane(ng, first);
            return true;
        }
        remaining -= total;
        groups_before += __builtin_amdgcn_readlane(gincl, 63);
    }
    return false;
}

// Per-unit geometry shared by the attention and combine kernels. The visible
// pages are those of the last query of the group's block, the same for every
// group of a workgroup (their splits line up).
struct TileGeom {
    int b, group, q0, Lq, ctx, npages, nsplit;
};

__device__ bool blockGeom(const Args &a, int b, int block, TileGeom &t, bool report) {
    t.b = b;
    t.q0 = a.cu_q[b];
    t.Lq = a.cu_q[b + 1] - t.q0;
    t.ctx = a.ctx[b];
    if (t.q0 < 0 || t.q0 + t.Lq > a.T || t.ctx > a.max_pages * 16 || t.Lq > t.ctx) {
        if (report && (threadIdx.x & 63) == 0) atomicOr(a.err, kErrTooLong);
        return false;
    }
    const int qi_max = min(t.Lq - 1, ((block + 1) * kWaves * kTiles * 16 - 1) / a.G);
    const int kv_len = t.ctx - t.Lq + qi_max + 1; // keys some column of the block sees
    t.npages = (kv_len + 15) >> 4;
    t.nsplit = (t.npages + a.pps - 1) / a.pps;
    return true;
}

// Partial O of a split record, element `idx` of the record's O block. For
// bf16 outputs it is kept as bf16 (RNE): its 2^-9 relative rounding matches
// the output's own, and it halves the record bytes that the attention kernel
// writes and the combine reads. fp32 outputs keep fp32 records. The (m, l)
// pairs stay fp32 after the O block either way.
template <bool OUT_F32> __device__ __forceinline__ void storeRecordO(float *rec, int idx, f32x4 v) {
    if constexpr (OUT_F32) {
        *reinterpret_cast<f32x4 *>(rec + idx) = v;
    } else {
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        const bf16x4 h = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
        *reinterpret_cast<bf16x4 *>(reinterpret_cast<uint16_t *>(rec) + idx) = h;
    }
}
template <bool OUT_F32> __device__ __forceinline__ f32x4 loadRecordO(const float *rec, int idx) {
    if constexpr (OUT_F32) {
        return *reinterpret_cast<const f32x4 *>(rec + idx);
    } else {
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        const bf16x4 h = *reinterpret_cast<const bf16x4 *>(reinterpret_cast<const uint16_t *>(rec) + idx);
        return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
    }
}

typedef u32x4 StageBuf[2][kStagePairs * 16 * 64]; // page pairs: K a, K b, V a, V b quarters

// One (block, split) of a unit: kv head h of sequence b's query block `block`
// (groups block * kWaves .. + kWaves - 1 of its groups_b; group_base groups
// before the sequence), pages [split * pps, ...) of its t.npages. Called by
// every wave of the workgroup with the same arguments (it has barriers).
template <bool OUT_F32>
__device__ __forceinline__ void prefillItem(const Args &a, StageBuf &kvs, int b, int block, int group_base, int h,
                                            int split, int groups_b, const TileGeom &t) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: scalar branches on it
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int G = a.G;
    const int p0 = split * a.pps;
    if (p0 >= t.npages) return;
    const int p1 = min(t.npages, p0 + a.pps);
    const int group = block * kWaves + wave;        // this wave's group in the sequence
    const bool active = group < groups_b;

    // Columns of the wave's tiles.
    int qi[kTiles], g[kTiles], pos[kTiles];
    bool col_ok[kTiles];
#pragma unroll
    for (int k = 0; k < kTiles; ++k) {
        const int pair = (group * kTiles + k) * 16 + n;
        qi[k] = pair / G;
        g[k] = pair - qi[k] * G;
        col_ok[k] = active && qi[k] < t.Lq;
        pos[k] = col_ok[k] ? t.ctx - t.Lq + qi[k] : -1;
    }

    // Smallest causal limit among the wave's real columns (wave-uniform).
    int min_pos = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < kTiles; ++k) min_pos = min(min_pos, col_ok[k] ? pos[k] : 0x7fffffff);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) min_pos = min(min_pos, __shfl_xor(min_pos, off));
    min_pos = __builtin_amdgcn_readfirstlane(min_pos);

    // Block ids of the split's pages: page p0 + i in lane i % 64 of bid[i / 64].
    int bid[2] = {0, 0};
#pragma unroll
    for (int w = 0; w < 2; ++w)
        if (lane + 64 * w < p1 - p0) bid[w] = a.table[size_t(t.b) * a.max_pages + p0 + 64 * w + lane];
    auto blockOf = [&](int page) {
        const int i = page - p0;
        return i < 64 ? __builtin_amdgcn_readlane(bid[0], i) : __builtin_amdgcn_readlane(bid[1], i - 64);
    };

    u32x4 qop[kTiles][4];
#pragma unroll
    for (int k = 0; k < kTiles; ++k) {
        const uint16_t *qrow =
            a.q + (size_t(t.q0 + (col_ok[k] ? qi[k] : 0)) * a.nh + h * G + (col_ok[k] ? g[k] : 0)) * kHeadDim + grp * 8;
#pragma unroll
        for (int s = 0; s < 4; ++s) qop[k][s] = *reinterpret_cast<const u32x4 *>(qrow + 32 * s);
#pragma unroll
        for (int s = 0; s < 4; ++s) qop[k][s] = col_ok[k] ? qop[k][s] : u32x4{0, 0, 0, 0};
    }

    const u32x4 *kp = reinterpret_cast<const u32x4 *>(a.k_pool) + lane;
    const u32x4 *vp = reinterpret_cast<const u32x4 *>(a.v_pool) + lane;
    bool bad_block = false;
    const int last_pair = p0 + ((p1 - 1 - p0) & ~1);
    // The pair is 16 one-KiB quarters: slot q = page part (q / 4: K a, K b,
    // V a, V b) and quarter (q % 4). Wave w stages slots w, w + kWaves, ...
    // Clamped: past the end it re-reads the last pair, so loads are never
    // conditional.
    static_assert(16 % kWaves == 0, "the 16 quarters of a pair split evenly over the waves");
    constexpr int kPer = 16 / kWaves;
    u32x4 st[kStagePairs][kPer];
    auto stageLoad = [&](int pp) { // the kStagePairs pairs from page pp
#pragma unroll
        for (int sp = 0; sp < kStagePairs; ++sp) {
            const int q0 = min(pp + 2 * sp, last_pair);
            int ba = blockOf(q0);
            int bb = (q0 + 1 < p1) ? blockOf(q0 + 1) : ba;
            const bool bad = unsigned(ba) >= unsigned(a.num_blocks) || unsigned(bb) >= unsigned(a.num_blocks);
            bad_block |= bad;
            ba = bad ? 0 : ba;
            bb = bad ? 0 : bb;
            const size_t oa = (size_t(ba) * a.nkvh + h) * 256, ob = (size_t(bb) * a.nkvh + h) * 256;
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                const int q = wave + kWaves * j, part = q >> 2, quarter = q & 3;
                const u32x4 *base = (part & 2) ? vp : kp;
                st[sp][j] = __builtin_nontemporal_load(base + ((part & 1) ? ob : oa) + quarter * 64);
            }
        }
    };
    // K quarters go to LDS as loaded. V quarters go in P.V operand order:
    // slot (8 + 2 s + h) of a pair holds, per lane, half h (dwords 2h, 2h+1)
    // of V page A's quarter s in its low 8 bytes and of page B's in its high 8.
    auto stageStore = [&](int buf) {
#pragma unroll
        for (int sp = 0; sp < kStagePairs; ++sp)
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                const int q = wave + kWaves * j, part = q >> 2, quarter = q & 3;
                u32x4 *pair = kvs[buf] + sp * 16 * 64;
                if (part < 2) {
                    pair[q * 64 + lane] = st[sp][j];
                } else {
                    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                    u32x2 *half = reinterpret_cast<u32x2 *>(pair + (8 + 2 * quarter) * 64 + lane) + (part & 1);
                    half[0] = u32x2{st[sp][j][0], st[sp][j][1]};
                    half[64 * 2] = u32x2{st[sp][j][2], st[sp][j][3]}; // next slot, same lane
                }
            }
    };

    Acc acc[kTiles];
#pragma unroll
    for (int k = 0; k < kTiles; ++k) acc[k].reset();
    constexpr int kStagePages = 2 * kStagePairs;
    stageLoad(p0);
    stageStore(0);
    __syncthreads();
    stageLoad(p0 + kStagePages);
    for (int i = 0, ps = p0; ps < p1; ++i, ps += kStagePages) {
        // stage i + 1 into the other buffer (read by everyone before the last
        // barrier), stage i + 2 into registers, then consume stage i from LDS.
        stageStore((i + 1) & 1);
        stageLoad(ps + 2 * kStagePages);
        if (active) {
            // Per softmax group of kSoft pairs: scores of each pair for every
            // tile (K of one pair live at a time), one softmax update per tile
            // over the group's keys, then P.V pair by pair (V of one pair live
            // at a time). fp32 outputs carry P as hi + lo, which leaves
            // registers for one pair per group only.
            constexpr int kSoft = OUT_F32 ? 1 : kStagePairs;
            const u32x4 *stage = kvs[i & 1];
#pragma unroll
            for (int sg = 0; sg < kStagePairs; sg += kSoft) {
                if (ps + 2 * sg >= p1) break;
                float sv[kTiles][kSoft][8];
#pragma unroll
                for (int j = 0; j < kSoft; ++j) {
                    const int pp = ps + 2 * (sg + j);
                    const u32x4 *src = stage + (sg + j) * 16 * 64;
                    const bool hasA = pp < p1, hasB = pp + 1 < p1;
                    // Every key of the pair visible to every column of the
                    // wave (no causal cut, no stale slots): no per-key mask.
                    const bool full = hasB && pp * 16 + 31 <= min_pos && pp * 16 + 32 <= t.ctx;
                    u32x4 ka[4], kb[4];
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        ka[s] = src[(0 * 4 + s) * 64 + lane];
                        kb[s] = src[(1 * 4 + s) * 64 + lane];
                    }
                    int lim[kTiles];
#pragma unroll
                    for (int k = 0; k < kTiles; ++k) lim[k] = hasA ? pos[k] : -1;
                    float svj[kTiles][8];
                    pairScoresN<kTiles>(svj, ka, kb, qop, pp * 16, lim, hasB, grp, full);
#pragma unroll
                    for (int k = 0; k < kTiles; ++k)
#pragma unroll
                        for (int e = 0; e < 8; ++e) sv[k][j][e] = svj[k][e];
                }
                PairP P[kTiles][kSoft];
#pragma unroll
                for (int k = 0; k < kTiles; ++k) softmaxUpdate<OUT_F32, kSoft>(acc[k], sv[k], P[k], a.scale_log2);
#pragma unroll
                for (int j = 0; j < kSoft; ++j) {
                    const int pp = ps + 2 * (sg + j);
                    if (pp >= p1) break;
                    const u32x4 *src = stage + (sg + j) * 16 * 64;
                    const bool hasB = pp + 1 < p1;
                    u32x4 v0[4], v1[4];
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        v0[s] = src[(8 + 2 * s) * 64 + lane];
                        v1[s] = src[(9 + 2 * s) * 64 + lane];
                    }
                    maskStaleVPacked(v0, v1, pp * 16, t.ctx, hasB, grp);
#pragma unroll
                    for (int k = 0; k < kTiles; ++k) accumulatePVPacked<OUT_F32>(acc[k], v0, v1, P[k][j]);
                }
            }
        }
        __syncthreads();
    }
    if (bad_block && lane == 0) atomicOr(a.err, kErrBadBlock);
    if (!active) return;
    const int unit = (group_base + group) * a.nkvh + h;
    float *rec = a.records + (size_t(unit) * a.max_splits + split) * kRecordFloats;
#pragma unroll
    for (int k = 0; k < kTiles; ++k) {
        float lt = acc[k].l + __shfl_xor(acc[k].l, 16);
        lt += __shfl_xor(lt, 32);
        if (!col_ok[k]) continue;
        if (t.nsplit == 1) {
            const size_t row = (size_t(t.q0 + qi[k]) * a.nh + h * G + g[k]) * kHeadDim;
            const float inv = 1.f / lt;
#pragma unroll
            for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, row, i, grp, acc[k].o[i] * inv);
            continue;
        }
        const int c = k * 16 + n; // column within the group
#pragma unroll
        for (int i = 0; i < 8; ++i) storeRecordO<OUT_F32>(rec, (i * kTiles * 16 + c) * 16 + grp * 4, acc[k].o[i]);
        if (grp == 0)
            *reinterpret_cast<float2 *>(rec + kTiles * 16 * kHeadDim + 2 * c) = make_float2(acc[k].m, lt);
    }
}

template <bool OUT_F32>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) prefillKernel(Args a) {
    __shared__ StageBuf kvs;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int split = blockIdx.x / a.block_units_padded;
    const int wunit = blockIdx.x - split * a.block_units_padded;
    if (wunit >= a.block_units) return;
    const int h = wunit % a.nkvh;
    int b, block, group_base;
    if (!locate(a, wunit / a.nkvh, true, b, block, group_base)) return;
    b = __builtin_amdgcn_readfirstlane(b);
    block = __builtin_amdgcn_readfirstlane(block);
    group_base = __builtin_amdgcn_readfirstlane(group_base);
    TileGeom t;
    if (!blockGeom(a, b, block, t, split == 0 && wave == 0)) return;
    // The geometry is wave-uniform: scalar registers, scalar branches.
    t.q0 = __builtin_amdgcn_readfirstlane(t.q0);
    t.Lq = __builtin_amdgcn_readfirstlane(t.Lq);
    t.ctx = __builtin_amdgcn_readfirstlane(t.ctx);
    t.npages = __builtin_amdgcn_readfirstlane(t.npages);
    prefillItem<OUT_F32>(a, kvs, b, block, group_base, h, split, __builtin_amdgcn_readfirstlane(groupsOf(a, b)), t);
}

// One single-query sequence's kv head h (query row `row`, c keys) in the
// persistent kernel: the workgroup's kWaves waves split its page pairs
// evenly, stream them through a two-stage register ring into the decode MFMA
// step, and merge their (O, m, l) through LDS (the stage buffers, idle
// during this item); wave 0 writes the row. The decode kernel's math with
// kWaves partial states instead of per-wave records.
constexpr int kDecWindow = 64; // pairs per block-id window (one per lane)
template <bool OUT_F32>
__device__ __forceinline__ void decodeItem(const Args &a, StageBuf &kvs, int b, int h, int row, int c) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int G = a.G;
    const int np = (c + 15) >> 4;
    const int npr = (np + 1) >> 1;
    const int p0 = wave * npr / kWaves, p1 = (wave + 1) * npr / kWaves;
    Acc acc;
    acc.reset();
    bool bad_block = false;
    if (p1 > p0) {
        u32x4 qop[4];
        const uint16_t *qrow = a.q + (size_t(row) * a.nh + h * G + min(n, G - 1)) * kHeadDim + grp * 8;
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            qop[t4] = *reinterpret_cast<const u32x4 *>(qrow + 32 * t4);
            qop[t4] = n < G ? qop[t4] : u32x4{0, 0, 0, 0};
        }
        const u32x4 *kp = reinterpret_cast<const u32x4 *>(a.k_pool) + lane;
        const u32x4 *vp = reinterpret_cast<const u32x4 *>(a.v_pool) + lane;
        const int32_t *trow = a.table + size_t(b) * a.max_pages;
        for (int base = p0; base < p1; base += kDecWindow) {
            const int cnt = min(kDecWindow, p1 - base);
            int bidA, bidB;
            {
                const int pa = 2 * (base + min(lane, cnt - 1));
                bidA = trow[pa];
                bidB = trow[min(pa + 1, np - 1)];
            }
            PagePair ring[2];
            auto issue = [&](int st, int k) {
                const int kk = min(k, cnt - 1);
                int bA = __builtin_amdgcn_readlane(bidA, kk);
                int bB = __builtin_amdgcn_readlane(bidB, kk);
                const bool bad = unsigned(bA) >= unsigned(a.num_blocks) || unsigned(bB) >= unsigned(a.num_blocks);
                bad_block |= bad;
                bA = bad ? 0 : bA;
                bB = bad ? 0 : bB;
                loadPair(ring[st], kp, vp, (size_t(bA) * a.nkvh + h) * 256, (size_t(bB) * a.nkvh + h) * 256);
            };
            issue(0, 0);
            issue(1, 1);
            for (int k0 = 0; k0 < cnt; k0 += 2) {
#pragma unroll
                for (int st = 0; st < 2; ++st) {
                    const int k = k0 + st;
                    if (k < cnt) {
                        const int j = base + k;
                        consumePair<OUT_F32>(acc, ring[st], qop, 32 * j, c - 1, c, 2 * j + 1 < np, grp, a.scale_log2);
                    }
                    issue(st, k + 2);
                }
            }
        }
    }
    if (bad_block && lane == 0) atomicOr(a.err, kErrBadBlock);
    float lt = acc.l + __shfl_xor(acc.l, 16);
    lt += __shfl_xor(lt, 32);
    f32x4 *part_o = reinterpret_cast<f32x4 *>(&kvs[0][0]);                 // [kWaves - 1][8][64]
    float *part_ml = reinterpret_cast<float *>(part_o + (kWaves - 1) * 8 * 64); // [kWaves - 1][2][64]
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) part_o[((wave - 1) * 8 + i) * 64 + lane] = acc.o[i];
        part_ml[((wave - 1) * 2 + 0) * 64 + lane] = acc.m;
        part_ml[((wave - 1) * 2 + 1) * 64 + lane] = lt;
    }
    __syncthreads();
    if (wave == 0 && n < G) {
        float M = acc.m, L = lt;
        for (int v = 0; v < kWaves - 1; ++v) {
            const float mv = part_ml[(v * 2 + 0) * 64 + lane];
            if (mv == -INFINITY) continue;
            const float Mn = fmaxf(M, mv);
            const float sa = exp2Fast(M - Mn);
            const float sb = exp2Fast(mv - Mn);
            L = L * sa + part_ml[(v * 2 + 1) * 64 + lane] * sb;
#pragma unroll
            for (int i = 0; i < 8; ++i) acc.o[i] = acc.o[i] * sa + part_o[(v * 8 + i) * 64 + lane] * sb;
            M = Mn;
        }
        const float inv = 1.f / L;
        const size_t orow = (size_t(row) * a.nh + h * G + n) * kHeadDim;
#pragma unroll
        for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, orow, i, grp, acc.o[i] * inv);
    }
}

// Exclusive prefix sums of va[0..n) and vb[0..n) in place (n <= 64 * 64), in
// one pass by the whole workgroup; the totals go to *total_a and *total_b.
// tmp: 130 ints of LDS. Barriers inside.
__device__ void blockExclusiveScan2(int *va, int *vb, int n, int *tmp, int *total_a, int *total_b) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nch = (n + 63) >> 6;
    for (int ch = wave; ch < 2 * nch; ch += kWaves) {
        const int which = ch >= nch ? 1 : 0, c = ch - which * nch;
        int *v = which ? vb : va;
        const int i = c * 64 + lane;
        const int x = i < n ? v[i] : 0;
        const int incl = waveInclusiveSum(x);
        if (i < n) v[i] = incl - x;
        if (lane == 63) tmp[65 * which + c] = incl;
    }
    __syncthreads();
    if (wave < 2) {
        int *t = tmp + 65 * wave;
        const int x = lane < nch ? t[lane] : 0;
        const int incl = waveInclusiveSum(x);
        if (lane < nch) t[lane] = incl - x;
        if (lane == 63) t[64] = incl;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 64 * kWaves) {
        va[i] += tmp[i >> 6];
        vb[i] += tmp[65 + (i >> 6)];
    }
    *total_a = tmp[64];
    *total_b = tmp[65 + 64];
    __syncthreads();
}

// Largest i in [0, n) with v[i] <= x, for non-decreasing v with v[0] <= x.
__device__ __forceinline__ int lastAtMost(const int *v, int n, int x) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (v[mid] <= x)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// Persistent prefill: one workgroup per CU works through the (unit, split)
// items of the batch instead of one workgroup per grid slot. A grid sized for
// the host's upper bound of units (it cannot see the lengths) is mostly
// empty workgroups, each spending a length lookup before it exits, and they
// delay the dispatch of real ones; per-item lookups cost dependent global
// round trips. Here every workgroup reads cu_q and ctx once and builds the
// item tables in LDS (per sequence: unit and group prefix sums; per unit: its
// split count and prefix of full splits; the units whose last split is
// partial), then takes items (its first by its own index, the rest from a
// device counter): all full (pps-page)
// splits first in unit order, then the partial last splits, so the longest
// items start earliest. The last workgroup to finish returns the counter and
// the done count to zero for the next launch. Items are the old kernel's
// (block, split) workgroups, run by the same code with the same records.
// WITH_DECODE: the batch's single-query sequences are items too, one per kv
// head (decodeItem), placed between the full and the partial splits, longest
// context first; their HBM-bound streams then run beside the splits' MFMA
// work, and no decode kernel or decode combine runs for them. (Ordering the
// whole tail by an estimated time instead measured no better with decode
// items and 4 us worse for prefill-only batches.)
constexpr int kQueueMaxSeqs = 1024;
constexpr int kQueueSortSeqs = 256; // decode items ranked by length up to this batch size
constexpr int kQueueMaxUnits = 4000; // the unit scans (U + 1 entries) fit blockExclusiveScan2

__host__ __device__ constexpr size_t queueTableInts(int B, int units) {
    return size_t(6) * (B + 1) + size_t(4) * (units + 1);
}

template <bool OUT_F32, bool WITH_DECODE>
__global__ void __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
    prefillQueueKernel(Args a) {
    __shared__ StageBuf kvs;
    __shared__ int scan_tmp[2 * 65];
    __shared__ int s_item[2];
    extern __shared__ int tables[];
    const int B = a.B, tid = threadIdx.x, nthreads = 64 * kWaves;
    int *cu = tables, *ctx = cu + (B + 1), *ubase = ctx + (B + 1), *gbase = ubase + (B + 1);
    int *nspl = gbase + (B + 1), *fpre = nspl + (a.block_units + 1), *ppos = fpre + (a.block_units + 1);
    int *punit = ppos + (a.block_units + 1), *dkey = punit + (a.block_units + 1), *dseq = dkey + (B + 1);
    for (int i = tid; i <= B; i += nthreads) {
        cu[i] = a.cu_q[i];
        ctx[i] = i < B ? a.ctx[i] : 0;
    }
    __syncthreads();
    // Per sequence: units (blocks x kv heads) and groups, as groupsOf counts
    // them (sequences with bad geometry keep their slots but get no items).
    for (int b = tid; b <= B; b += nthreads) {
        int ng = 0;
        if (b < B) {
            const int lq = cu[b + 1] - cu[b];
            ng = lq >= 2 ? (((lq * a.G + 15) >> 4) + kTiles - 1) / kTiles : 0;
        }
        gbase[b] = ng;
        ubase[b] = (ng + kWaves - 1) / kWaves * a.nkvh;
        // Single-query sequences (with_decode) with a valid query row and
        // length are decode items (nkvh each; else error bit 2, no items):
        // key = their length, -1 for the rest.
        int key = -1;
        if (WITH_DECODE && b < B && cu[b + 1] - cu[b] == 1) {
            const int row = cu[b], c = ctx[b];
            if (row < 0 || row >= a.T || c < 1 || c > a.max_pages * 16) {
                if (blockIdx.x == 0) atomicOr(a.err, kErrTooLong);
            } else {
                key = c;
            }
        }
        if (b < B) dkey[b] = key;
    }
    __syncthreads();
    int U = 0, n_groups = 0;
    blockExclusiveScan2(gbase, ubase, B + 1, scan_tmp, &n_groups, &U);
    U = min(U, a.block_units);
    // Decode sequences longest first: dseq[rank] = b, the rank of b being
    // the number of valid sequences with a longer context, or as long and
    // listed earlier (deterministic, so every workgroup builds the same order;
    // O(B^2), so the host gives this kernel the decode items only for batches
    // of at most kQueueSortSeqs sequences). Every wave holds all the keys,
    // 64 per register; wave w ranks sequences w, w + kWaves, ..., a ballot
    // per register counting those ahead (a loop over the batch in LDS per
    // thread was 2 us of LDS latency at B = 64).
    int n_dec_seqs = 0;
    if constexpr (WITH_DECODE) {
        constexpr int kRegs = kQueueSortSeqs / 64;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
        int ko[kRegs];
#pragma unroll
        for (int r = 0; r < kRegs; ++r) {
            const int o = 64 * r + lane;
            ko[r] = o < B ? dkey[o] : -1;
            n_dec_seqs += __popcll(__ballot(ko[r] >= 0));
        }
        for (int b = wave; b < B; b += kWaves) {
            int kb = ko[0];
#pragma unroll
            for (int r = 1; r < kRegs; ++r)
                if ((b >> 6) == r) kb = ko[r];
            kb = __builtin_amdgcn_readlane(kb, b & 63);
            if (kb < 0) continue;
            int rank = 0;
#pragma unroll
            for (int r = 0; r < kRegs; ++r)
                if (64 * r < B) rank += __popcll(__ballot(ko[r] > kb || (ko[r] == kb && 64 * r + lane < b)));
            if (lane == 0) dseq[rank] = b;
        }
        __syncthreads();
    }
    const int n_dec = n_dec_seqs * a.nkvh;
    // Per unit: splits, full splits, partial flag.
    for (int u = tid; u <= U; u += nthreads) {
        int ns = 0, full = 0;
        if (u < U) {
            const int b = lastAtMost(ubase, B, u);
            const int j = (u - ubase[b]) / a.nkvh;
            const int q0 = cu[b], lq = cu[b + 1] - q0, c = ctx[b];
            if (q0 < 0 || q0 + lq > a.T || c > a.max_pages * 16 || lq > c) {
                if (blockIdx.x == 0 && u == ubase[b]) atomicOr(a.err, kErrTooLong);
            } else {
                const int qi_max = min(lq - 1, ((j + 1) * kWaves * kTiles * 16 - 1) / a.G);
                const int np = (c - lq + qi_max + 1 + 15) >> 4;
                ns = (np + a.pps - 1) / a.pps;
                full = np - (ns - 1) * a.pps == a.pps ? ns : ns - 1;
            }
        }
        nspl[u] = ns;
        fpre[u] = full;
        ppos[u] = ns > full ? 1 : 0;
    }
    __syncthreads();
    int n_full = 0, n_part = 0;
    blockExclusiveScan2(fpre, ppos, U + 1, scan_tmp, &n_full, &n_part);
    for (int u = tid; u < U; u += nthreads)
        if (nspl[u] > fpre[u + 1] - fpre[u]) punit[ppos[u]] = u;
    __syncthreads();
    const int n_items = n_full + n_part + n_dec;
    // Workgroup g's first item is item g; later ones come from the counter,
    // past the grid.
    for (int it = 0;; ++it) {
        if (it > 0 && tid == 0) s_item[it & 1] = int(gridDim.x) + atomicAdd(a.queue, 1);
        __syncthreads();
        const int item = it == 0 ? int(blockIdx.x) : __builtin_amdgcn_readfirstlane(s_item[it & 1]);
        if (item >= n_items) break;
        // Order: the full prefill splits, the single-query sequences' kv heads
        // (longest first), then the partial last splits.
        const bool dec_item = WITH_DECODE && item >= n_full && item < n_full + n_dec;
        if (!dec_item) {
            int u, split;
            if (item < n_full) {
                u = lastAtMost(fpre, U, item);
                split = item - fpre[u];
            } else {
                u = punit[item - n_full - n_dec];
                split = nspl[u] - 1;
            }
            u = __builtin_amdgcn_readfirstlane(u);
            split = __builtin_amdgcn_readfirstlane(split);
            const int b = __builtin_amdgcn_readfirstlane(lastAtMost(ubase, B, u));
            const int local = u - ubase[b];
            const int block = local / a.nkvh, h = local - block * a.nkvh;
            TileGeom t;
            t.b = b;
            t.q0 = __builtin_amdgcn_readfirstlane(cu[b]);
            t.Lq = __builtin_amdgcn_readfirstlane(cu[b + 1]) - t.q0;
            t.ctx = __builtin_amdgcn_readfirstlane(ctx[b]);
            const int qi_max = min(t.Lq - 1, ((block + 1) * kWaves * kTiles * 16 - 1) / a.G);
            t.npages = (t.ctx - t.Lq + qi_max + 1 + 15) >> 4;
            t.nsplit = __builtin_amdgcn_readfirstlane(nspl[u]);
            const int group_base = __builtin_amdgcn_readfirstlane(gbase[b]);
            const int groups_b = __builtin_amdgcn_readfirstlane(gbase[b + 1]) - group_base;
            prefillItem<OUT_F32>(a, kvs, b, block, group_base, h, split, groups_b, t);
        } else if constexpr (WITH_DECODE) {
            const int d = item - n_full;
            const int b = __builtin_amdgcn_readfirstlane(dseq[d / a.nkvh]);
            const int h = d - (d / a.nkvh) * a.nkvh;
            decodeItem<OUT_F32>(a, kvs, b, h, __builtin_amdgcn_readfirstlane(cu[b]),
                                __builtin_amdgcn_readfirstlane(ctx[b]));
        }
    }
    if (tid == 0 && atomicAdd(a.queue + 1, 1) == int(gridDim.x) - 1) {
        atomicExch(a.queue, 0);
        atomicExch(a.queue + 1, 0);
    }
}

// Merge the split records of each unit with more than one split.
constexpr int kMergeBatch = 4;

template <bool OUT_F32> __global__ void __launch_bounds__(64) prefillCombineKernel(Args a) {
    const int lane = threadIdx.x;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int unit = blockIdx.x / kTiles;
    const int k = blockIdx.x - unit * kTiles; // tile of the group this wave merges
    if (unit >= a.units) return;
    const int h = unit % a.nkvh;
    int b, group, group_base;
    if (!locate(a, unit / a.nkvh, false, b, group, group_base)) return;
    TileGeom t;
    if (!blockGeom(a, b, group / kWaves, t, false) || t.nsplit <= 1) return;
    const int G = a.G;
    const int pair = (group * kTiles + k) * 16 + n;
    const int qi = pair / G;
    const int g = pair - qi * G;
    const bool col_ok = qi < t.Lq;
    const int c = k * 16 + n;
    const float *recs = a.records + size_t(unit) * a.max_splits * kRecordFloats;
    float M = -INFINITY, L = 0.f;
    f32x4 o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < t.nsplit; k0 += kMergeBatch) {
        float mr[kMergeBatch], lr[kMergeBatch];
        f32x4 orr[kMergeBatch][8];
#pragma unroll
        for (int s = 0; s < kMergeBatch; ++s) {
            const float *rec = recs + size_t(min(k0 + s, t.nsplit - 1)) * kRecordFloats;
            const float2 ml = *reinterpret_cast<const float2 *>(rec + kTiles * 16 * kHeadDim + 2 * c);
            mr[s] = k0 + s < t.nsplit ? ml.x : -INFINITY;
            lr[s] = ml.y;
#pragma unroll
            for (int i = 0; i < 8; ++i) orr[s][i] = loadRecordO<OUT_F32>(rec, (i * kTiles * 16 + c) * 16 + grp * 4);
        }
#pragma unroll
        for (int s = 0; s < kMergeBatch; ++s) {
            // A split can lie wholly past a column's causal limit: m = -inf, weight 0.
            if (mr[s] == -INFINITY) continue;
            const float Mn = fmaxf(M, mr[s]);
            const float sa = exp2Fast(M - Mn);
            const float sb = exp2Fast(mr[s] - Mn);
            L = L * sa + lr[s] * sb;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = o[i] * sa + orr[s][i] * sb;
            M = Mn;
        }
    }
    if (!col_ok) return;
    const float inv = 1.f / L;
    const size_t row = (size_t(t.q0 + qi) * a.nh + h * G + g) * kHeadDim;
#pragma unroll
    for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, row, i, grp, o[i] * inv);
}

int envInt(const char *name, int fallback) {
    const char *v = std::getenv(name);
    if (!v || !*v) return fallback;
    return std::atoi(v);
}

// LDS left for the persistent kernel's item tables beside its 64 KiB of
// stages (160 KiB per CU on gfx950, one workgroup per CU).
constexpr size_t kQueueTableBytes = size_t(80) << 10;

int cuCount() {
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

PagedAttentionPlan planPrefill(int B, int T, int nkvh, int group, int max_pages) {
    PagedAttentionPlan p{};
    const int groups = ((T * group + 15) / 16 + kTiles - 1) / kTiles + B; // upper bound over the batch
    p.units = groups * nkvh;
    p.units_padded = p.units;
    p.block_units = (groups / kWaves + B) * nkvh;
    p.block_units_padded = (p.block_units + kXcds - 1) / kXcds * kXcds;
    // Pages per split: even (pairs of pages), at most 128 (two block ids per lane).
    int pps = envInt("LLAISYS_PAGES_PER_SPLIT", 64);
    pps = std::max(2, std::min(128, pps & ~1));
    p.pages_per_split = pps;
    p.max_splits = std::max(1, (max_pages + pps - 1) / pps);
    p.partial_bytes = size_t(p.units) * p.max_splits * kRecordFloats * sizeof(float);
    return p;
}

bool prefillQueueUsable(int B, const PagedAttentionPlan &plan, const int *queue) {
    return queue && envInt("LLAISYS_PREFILL_QUEUE", 1) != 0 && B <= kQueueMaxSeqs &&
           plan.block_units <= kQueueMaxUnits &&
           queueTableInts(B, plan.block_units) * sizeof(int) <= kQueueTableBytes;
}

bool prefillTakesDecode(int B, int T, const PagedAttentionPlan &plan, const int *queue) {
    // A batch of single queries only (T == B) keeps the stream-K decode
    // kernel, which balances sequences of very different lengths; so does a
    // batch of more than kQueueSortSeqs sequences (the item order would cost
    // more than it saves).
    return T != B && B <= kQueueSortSeqs && prefillQueueUsable(B, plan, queue) &&
           envInt("LLAISYS_PREFILL_TAKES_DECODE", 1) != 0;
}

void pagedPrefill(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                  const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_q, int B, int T, int nh,
                  int nkvh, int max_pages, int num_blocks, float scale, const PagedAttentionPlan &plan,
                  float *records, int *err, int *queue, void *stream) {
    if (B == 0 || T == 0) return;
    Args a;
    a.q = q;
    a.out = out;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.table = block_table;
    a.ctx = ctx_len;
    a.cu_q = cu_q;
    a.records = records;
    a.err = err;
    a.queue = queue;
    a.with_decode = 0;
    a.B = B;
    a.T = T;
    a.nh = nh;
    a.nkvh = nkvh;
    a.G = nh / nkvh;
    a.max_pages = max_pages;
    a.num_blocks = num_blocks;
    a.pps = plan.pages_per_split;
    a.max_splits = plan.max_splits;
    a.units = plan.units;
    a.block_units = plan.block_units;
    a.block_units_padded = plan.block_units_padded;
    a.scale_log2 = scale * 1.4426950408889634f;
    const dim3 grid(plan.block_units_padded * plan.max_splits), block(64 * kWaves), cblock(64);
    auto s = static_cast<hipStream_t>(stream);
    // The persistent kernel whenever its item tables fit in LDS beside the
    // stages (and a counter buffer is given); otherwise one workgroup per
    // grid slot.
    const size_t table_bytes = queueTableInts(B, plan.block_units) * sizeof(int);
    const bool queued = prefillQueueUsable(B, plan, queue);
    a.with_decode = queued && prefillTakesDecode(B, T, plan, queue);
    const dim3 qgrid(unsigned(std::min<long long>(cuCount(), (long long)plan.block_units * plan.max_splits)));
    if (out_f32) {
        if (queued && a.with_decode)
            hipLaunchKernelGGL((prefillQueueKernel<true, true>), qgrid, block, unsigned(table_bytes), s, a);
        else if (queued)
            hipLaunchKernelGGL((prefillQueueKernel<true, false>), qgrid, block, unsigned(table_bytes), s, a);
        else
            hipLaunchKernelGGL((prefillKernel<true>), grid, block, 0, s, a);
        if (plan.max_splits > 1) hipLaunchKernelGGL((prefillCombineKernel<true>), dim3(plan.units * kTiles), cblock, 0, s, a);
    } else {
        if (queued && a.with_decode)
            hipLaunchKernelGGL((prefillQueueKernel<false, true>), qgrid, block, unsigned(table_bytes), s, a);
        else if (queued)
            hipLaunchKernelGGL((prefillQueueKernel<false, false>), qgrid, block, unsigned(table_bytes), s, a);
        else
            hipLaunchKernelGGL((prefillKernel<false>), grid, block, 0, s, a);
        if (plan.max_splits > 1) hipLaunchKernelGGL((prefillCombineKernel<false>), dim3(plan.units * kTiles), cblock, 0, s, a);
    }
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
