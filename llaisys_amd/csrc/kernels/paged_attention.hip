// Chunked-prefill attention over paged KV for gfx950 (the multi-query
// sequences of a mixed batch; single-query sequences go to the decode kernel).
//
// Work unit = (query group, kv head). A query tile is 16 "columns"; column n
// of tile t is the (query row, query head) pair number t*16+n of its
// sequence, pairs ordered query-major: pair = qi*G + g, G = nh/nkvh query
// heads per kv head. A group is kTiles adjacent tiles: one wave carries all of
// them, so each K/V page pair it loads feeds kTiles x 24 MFMAs (the kernel is
// otherwise bound by re-streaming the same pages from L2 per tile).
// Query qi of a sequence with Lq new tokens sits at position ctx - Lq + qi
// and sees keys at positions <= that (bottom-right causal alignment). A
// unit's visible pages are cut into splits of `pages_per_split` pages; one
// wave (one 64-lane workgroup) runs one (unit, split), streaming page pairs
// through a two-stage register ring (loads never conditional) into the MFMA
// step of mfma_common.hpp. A unit with one split writes its normalised
// output; with more, each split writes a record (O, m, l) and the combine
// kernel launched next merges them (the kernel boundary orders the records;
// no fences, no waiting between waves).
//
// Workgroup ids are split-major over units padded to a multiple of 8, so all
// splits of a unit run on one XCD and share its L2 for the unit's K/V pages.
#include "mfma_common.hpp"

#include "../device/hip_check.hpp"

#include <algorithm>
#include <cstdlib>

namespace llaisys::kernels {

namespace {

using namespace mfma;

constexpr int kXcds = 8;
constexpr int kTiles = 2;                                    // query tiles per wave
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
    int B, T, nh, nkvh, G, max_pages, num_blocks, pps, max_splits, units, units_padded;
    float scale_log2;
};

// Sequence and group of unit-row `group_global`: groups are numbered sequence
// by sequence, ceil(ceil(Lq*G/16)/kTiles) for each sequence with Lq >= 2
// queries. Returns false past the last group. One wave.
__device__ bool locateGroup(const Args &a, int group_global, int &b, int &group) {
    const int lane = threadIdx.x & 63;
    int remaining = group_global;
    for (int base = 0; base < a.B; base += 64) {
        const int bb = base + lane;
        int nt = 0;
        if (bb < a.B) {
            const int lq = a.cu_q[bb + 1] - a.cu_q[bb];
            nt = lq >= 2 ? (((lq * a.G + 15) >> 4) + kTiles - 1) / kTiles : 0;
        }
        int incl = nt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(incl, off);
            if (lane >= off) incl += y;
        }
        const int total = __shfl(incl, 63);
        if (remaining < total) {
            const unsigned long long hit = __ballot(incl > remaining);
            const int first = __ffsll(hit) - 1;
            b = base + first;
            group = remaining - (__shfl(incl, first) - __shfl(nt, first));
            return true;
        }
        remaining -= total;
    }
    return false;
}

// Per-unit geometry shared by the attention and combine kernels.
struct TileGeom {
    int b, group, q0, Lq, ctx, npages, nsplit;
};

__device__ bool tileGeom(const Args &a, int group_global, TileGeom &t, bool report) {
    if (!locateGroup(a, group_global, t.b, t.group)) return false;
    t.q0 = a.cu_q[t.b];
    t.Lq = a.cu_q[t.b + 1] - t.q0;
    t.ctx = a.ctx[t.b];
    if (t.q0 < 0 || t.q0 + t.Lq > a.T || t.ctx > a.max_pages * 16 || t.Lq > t.ctx) {
        if (report && (threadIdx.x & 63) == 0) atomicOr(a.err, kErrTooLong);
        return false;
    }
    const int qi_max = min(t.Lq - 1, ((t.group + 1) * kTiles * 16 - 1) / a.G);
    const int kv_len = t.ctx - t.Lq + qi_max + 1; // keys some column of the group sees
    t.npages = (kv_len + 15) >> 4;
    t.nsplit = (t.npages + a.pps - 1) / a.pps;
    return true;
}

template <bool OUT_F32> __global__ void __launch_bounds__(64) prefillKernel(Args a) {
    const int lane = threadIdx.x;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int split = blockIdx.x / a.units_padded;
    const int unit = blockIdx.x - split * a.units_padded;
    if (unit >= a.units) return;
    const int h = unit % a.nkvh;
    TileGeom t;
    if (!tileGeom(a, unit / a.nkvh, t, split == 0)) return;
    const int G = a.G;
    const int p0 = split * a.pps;
    if (p0 >= t.npages) return;
    const int p1 = min(t.npages, p0 + a.pps);

    // Columns of the group's tiles.
    int qi[kTiles], g[kTiles], pos[kTiles];
    bool col_ok[kTiles];
#pragma unroll
    for (int k = 0; k < kTiles; ++k) {
        const int pair = (t.group * kTiles + k) * 16 + n;
        qi[k] = pair / G;
        g[k] = pair - qi[k] * G;
        col_ok[k] = qi[k] < t.Lq;
        pos[k] = col_ok[k] ? t.ctx - t.Lq + qi[k] : -1;
    }

    int bid = 0;
    if (lane < p1 - p0) bid = a.table[size_t(t.b) * a.max_pages + p0 + lane];

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
    // Loads for the pair starting at page pp (clamped: past the end it
    // re-reads the last pair, so loads are never conditional).
    auto issue = [&](PagePair &r, int pp) {
        pp = min(pp, last_pair);
        int ba = __builtin_amdgcn_readlane(bid, pp - p0);
        int bb = (pp + 1 < p1) ? __builtin_amdgcn_readlane(bid, pp + 1 - p0) : ba;
        const bool bad = unsigned(ba) >= unsigned(a.num_blocks) || unsigned(bb) >= unsigned(a.num_blocks);
        bad_block |= bad;
        ba = bad ? 0 : ba;
        bb = bad ? 0 : bb;
        loadPair(r, kp, vp, (size_t(ba) * a.nkvh + h) * 256, (size_t(bb) * a.nkvh + h) * 256);
    };

    Acc acc[kTiles];
#pragma unroll
    for (int k = 0; k < kTiles; ++k) acc[k].reset();
    auto consume = [&](PagePair &r, int pp) {
#pragma unroll
        for (int k = 0; k < kTiles; ++k) consumePair<OUT_F32>(acc[k], r, qop[k], pp * 16, pos[k], t.ctx, pp + 1 < p1, grp, a.scale_log2);
    };
    PagePair ra, rb;
    issue(ra, p0);
    issue(rb, p0 + 2);
    for (int pp = p0; pp < p1; pp += 4) {
        consume(ra, pp);
        issue(ra, pp + 4);
        if (pp + 2 < p1) consume(rb, pp + 2);
        issue(rb, pp + 6);
    }
    if (bad_block && lane == 0) atomicOr(a.err, kErrBadBlock);
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
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<f32x4 *>(rec + (i * kTiles * 16 + c) * 16 + grp * 4) = acc[k].o[i];
        if (grp == 0)
            *reinterpret_cast<float2 *>(rec + kTiles * 16 * kHeadDim + 2 * c) = make_float2(acc[k].m, lt);
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
    TileGeom t;
    if (!tileGeom(a, unit / a.nkvh, t, false) || t.nsplit <= 1) return;
    const int G = a.G;
    const int pair = (t.group * kTiles + k) * 16 + n;
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
            for (int i = 0; i < 8; ++i)
                orr[s][i] = *reinterpret_cast<const f32x4 *>(rec + (i * kTiles * 16 + c) * 16 + grp * 4);
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

} // namespace

PagedAttentionPlan planPrefill(int B, int T, int nkvh, int group, int max_pages) {
    PagedAttentionPlan p{};
    const int groups = ((T * group + 15) / 16 + kTiles - 1) / kTiles + B;
    p.units = groups * nkvh;
    p.units_padded = (p.units + kXcds - 1) / kXcds * kXcds;
    // Pages per split: even (pairs of pages), at most 64 (one block id per lane).
    int pps = envInt("LLAISYS_PAGES_PER_SPLIT", 64);
    pps = std::max(2, std::min(64, pps & ~1));
    p.pages_per_split = pps;
    p.max_splits = std::max(1, (max_pages + pps - 1) / pps);
    p.partial_bytes = size_t(p.units_padded) * p.max_splits * kRecordFloats * sizeof(float);
    return p;
}

void pagedPrefill(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                  const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_q, int B, int T, int nh,
                  int nkvh, int max_pages, int num_blocks, float scale, const PagedAttentionPlan &plan,
                  float *records, int *err, void *stream) {
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
    a.units_padded = plan.units_padded;
    a.scale_log2 = scale * 1.4426950408889634f;
    const dim3 grid(plan.units_padded * plan.max_splits), block(64);
    auto s = static_cast<hipStream_t>(stream);
    if (out_f32) {
        hipLaunchKernelGGL((prefillKernel<true>), grid, block, 0, s, a);
        if (plan.max_splits > 1) hipLaunchKernelGGL((prefillCombineKernel<true>), dim3(plan.units * kTiles), block, 0, s, a);
    } else {
        hipLaunchKernelGGL((prefillKernel<false>), grid, block, 0, s, a);
        if (plan.max_splits > 1) hipLaunchKernelGGL((prefillCombineKernel<false>), dim3(plan.units * kTiles), block, 0, s, a);
    }
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
