// Paged flash-decoding / chunked-prefill attention for gfx950 (MI355X).
//
// Work unit = (query tile, kv head). A query tile is 16 "columns"; column n is
// the (query row, query head) pair number tile*16+n of its sequence, pairs
// ordered query-major: pair = qi*G + g, G = nh/nkvh query heads per kv head.
// A decode sequence (one query) is one tile whose first G columns are live.
// Each unit's visible pages are cut into splits of `pages_per_split` pages;
// one wave (one 64-lane workgroup) runs one (unit, split).
//
// Per pair of pages (32 keys) a wave issues, all from registers:
//   S^T[16 keys x 16 cols]  = K_page[16 x 128] . Q^T[128 x 16]
//       4 x v_mfma_f32_16x16x32_bf16 per page; the K page format makes each
//       A operand one coalesced 1 KiB load (64 lanes x 16 B);
//   online softmax in base 2 on the 8 scores each lane holds (its column,
//       keys 4*(lane/16)+i of both pages); max across the 4 lane groups by
//       two lane shuffles; fp32 throughout;
//   O^T[128 x 16 cols] += V^T[128 x 32 keys] . P^T[32 keys x 16 cols]
//       8 dim blocks x 2 MFMAs: P is split as P = hi + lo (two bf16 parts,
//       ~16 significant bits), so the product is fp32-accurate to ~1e-5 while
//       V (bf16 data) is exact. The V page format makes each A operand half of
//       one coalesced 1 KiB load.
// The lane layouts line up so nothing crosses lanes except the max: the S^T
// accumulator a lane holds is the P^T operand it needs, and O^T's column is the
// lane's own column, so rescaling by exp2(m_old - m_new) is lane-local.
//
// Split-KV combine: a unit with one split writes the normalised output. With
// more, each wave writes (O, m, l) for its split, then bumps the unit's
// arrival counter; the wave that arrives last merges all splits with
// log-sum-exp weights, writes the output and resets the counter to zero. No
// wave ever waits on another, so no ordering between waves is assumed.
//
// Workgroup ids are split-major over units padded to a multiple of 8, so every
// split of a unit runs on the same XCD (id % 8) and the combine reads its
// partials from that XCD's L2.
#include "launch.hpp"

#include "../device/hip_check.hpp"

#include <algorithm>
#include <cstdlib>

namespace llaisys::kernels {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kErrBadBlock = 1;
constexpr int kErrTooLong = 2;
constexpr int kXcds = 8;
constexpr int kPartialFloats = 16 * kHeadDim + 32; // O for 16 columns, then (m, l) per column

struct Args {
    const uint16_t *q;
    void *out;
    const uint16_t *k_pool;
    const uint16_t *v_pool;
    const int32_t *table;
    const int32_t *ctx;
    const int32_t *cu_q;
    float *partial;
    int *counters;
    int *err;
    int B, T, nh, nkvh, G, max_pages, num_blocks, pps, max_splits, units, units_padded;
    float scale_log2;
};

__device__ __forceinline__ bf16x8 asBf16(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2Fast(float x) { return __builtin_amdgcn_exp2f(x); }

struct PageRegs {
    u32x4 ka[4], kb[4], va[4], vb[4];
};

// Keeps the halves of each 32-bit word whose key is valid.
__device__ __forceinline__ uint32_t keepPair(bool lo, bool hi) {
    return (lo ? 0x0000ffffu : 0u) | (hi ? 0xffff0000u : 0u);
}

template <bool OUT_F32>
__device__ __forceinline__ void storeOut(void *out, size_t base, int blk, int grp, f32x4 v) {
    const size_t idx = base + blk * 16 + grp * 4;
    if constexpr (OUT_F32) {
        *reinterpret_cast<f32x4 *>(static_cast<float *>(out) + idx) = v;
    } else {
        const __bf16 e0 = (__bf16)v[0], e1 = (__bf16)v[1], e2 = (__bf16)v[2], e3 = (__bf16)v[3];
        const uint32_t w0 = uint32_t(__builtin_bit_cast(uint16_t, e0)) | (uint32_t(__builtin_bit_cast(uint16_t, e1)) << 16);
        const uint32_t w1 = uint32_t(__builtin_bit_cast(uint16_t, e2)) | (uint32_t(__builtin_bit_cast(uint16_t, e3)) << 16);
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(out) + idx) = make_uint2(w0, w1);
    }
}

template <bool OUT_F32, bool VARLEN>
__global__ void __launch_bounds__(64) pagedAttentionKernel(Args a) {
    const int lane = threadIdx.x;
    const int n = lane & 15;
    const int grp = lane >> 4;
    const int split = blockIdx.x / a.units_padded;
    const int unit = blockIdx.x - split * a.units_padded;
    if (unit >= a.units) return;
    const int h = unit % a.nkvh;
    const int tile_global = unit / a.nkvh;
    const int G = a.G;

    // ---- locate (sequence, tile)
    int b, tile, q0, Lq;
    if constexpr (!VARLEN) {
        b = tile_global;
        tile = 0;
        q0 = b;
        Lq = 1;
    } else {
        b = -1;
        tile = 0;
        int remaining = tile_global;
        for (int base = 0; base < a.B; base += 64) {
            const int bb = base + lane;
            int nt = 0;
            if (bb < a.B) nt = ((a.cu_q[bb + 1] - a.cu_q[bb]) * G + 15) >> 4;
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
                tile = remaining - (__shfl(incl, first) - __shfl(nt, first));
                break;
            }
            remaining -= total;
        }
        if (b < 0) return;
        q0 = a.cu_q[b];
        Lq = a.cu_q[b + 1] - q0;
        if (q0 < 0 || Lq < 0 || q0 + Lq > a.T) { // query rows outside q/out: refuse the sequence
            if (lane == 0) atomicOr(a.err, kErrTooLong);
            return;
        }
    }
    const int ctx = a.ctx[b];
    if (ctx > a.max_pages * 16 || Lq > ctx || ctx <= 0) {
        if (lane == 0) atomicOr(a.err, kErrTooLong);
        return;
    }

    // ---- columns of this tile
    const int pair = tile * 16 + n;
    const int qi = pair / G;
    const int g = pair - qi * G;
    const bool col_ok = qi < Lq;
    const int pos = col_ok ? ctx - Lq + qi : -1; // last key this column sees
    const int qi_max = min(Lq - 1, (tile * 16 + 15) / G);
    const int kv_len = ctx - Lq + qi_max + 1;
    const int npages = (kv_len + 15) >> 4;
    const int nsplit = (npages + a.pps - 1) / a.pps;
    const int p0 = split * a.pps;
    if (p0 >= npages) return;
    const int p1 = min(npages, p0 + a.pps);

    int bid = 0;
    if (lane < p1 - p0) {
        bid = a.table[size_t(b) * a.max_pages + p0 + lane];
        if (bid < 0 || bid >= a.num_blocks) {
            atomicOr(a.err, kErrBadBlock);
            bid = 0;
        }
    }

    u32x4 qop[4];
    {
        const uint16_t *qrow = a.q + (size_t(q0 + (col_ok ? qi : 0)) * a.nh + h * G + g) * kHeadDim + grp * 8;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            qop[s] = col_ok ? *reinterpret_cast<const u32x4 *>(qrow + 32 * s) : u32x4{0, 0, 0, 0};
        }
    }

    const u32x4 *kp = reinterpret_cast<const u32x4 *>(a.k_pool) + lane;
    const u32x4 *vp = reinterpret_cast<const u32x4 *>(a.v_pool) + lane;
    auto load = [&](int pp, PageRegs &r) {
        const int ba = __builtin_amdgcn_readlane(bid, pp - p0);
        const int bb = (pp + 1 < p1) ? __builtin_amdgcn_readlane(bid, pp + 1 - p0) : ba;
        const size_t oa = (size_t(ba) * a.nkvh + h) * 256;
        const size_t ob = (size_t(bb) * a.nkvh + h) * 256;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            r.ka[s] = __builtin_nontemporal_load(kp + oa + s * 64);
            r.kb[s] = __builtin_nontemporal_load(kp + ob + s * 64);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            r.va[s] = __builtin_nontemporal_load(vp + oa + s * 64);
            r.vb[s] = __builtin_nontemporal_load(vp + ob + s * 64);
        }
    };

    f32x4 o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY;
    float lsum = 0.f;

    // One page pair: scores, online softmax, P.V. Loads for it were issued earlier.
    auto consume = [&](PageRegs &r, int pp) {
        const bool hasB = pp + 1 < p1;
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            sa = mfma(asBf16(r.ka[s]), asBf16(qop[s]), sa);
            sb = mfma(asBf16(r.kb[s]), asBf16(qop[s]), sb);
        }
        const int kbase = pp * 16 + grp * 4;
        float sv[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv[i] = (kbase + i <= pos) ? sa[i] * a.scale_log2 : -INFINITY;
            sv[4 + i] = (hasB && kbase + 16 + i <= pos) ? sb[i] * a.scale_log2 : -INFINITY;
        }
        float mloc = sv[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mloc = fmaxf(mloc, sv[i]);
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        const float m_new = fmaxf(m, mloc);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = exp2Fast(m - m_use);
        float p[8];
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            p[i] = exp2Fast(sv[i] - m_use);
            psum += p[i];
        }
        lsum = lsum * alpha + psum;
        m = m_new;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] *= alpha;

        bf16x8 phi, plo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const __bf16 hi = (__bf16)p[i];
            phi[i] = hi;
            plo[i] = (__bf16)(p[i] - (float)hi);
        }

        // Keys at or past ctx may hold stale bytes (even NaN patterns): zero
        // their V so 0 * V stays 0. Only the last pair of a sequence has any.
        if (pp * 16 + 32 > ctx || !hasB) {
            const uint32_t ma01 = keepPair(kbase < ctx, kbase + 1 < ctx);
            const uint32_t ma23 = keepPair(kbase + 2 < ctx, kbase + 3 < ctx);
            const uint32_t mb01 = hasB ? keepPair(kbase + 16 < ctx, kbase + 17 < ctx) : 0u;
            const uint32_t mb23 = hasB ? keepPair(kbase + 18 < ctx, kbase + 19 < ctx) : 0u;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                r.va[s] &= u32x4{ma01, ma23, ma01, ma23};
                r.vb[s] &= u32x4{mb01, mb23, mb01, mb23};
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bf16x8 v0 = asBf16(u32x4{r.va[s][0], r.va[s][1], r.vb[s][0], r.vb[s][1]});
            const bf16x8 v1 = asBf16(u32x4{r.va[s][2], r.va[s][3], r.vb[s][2], r.vb[s][3]});
            o[2 * s] = mfma(v0, phi, o[2 * s]);
            o[2 * s] = mfma(v0, plo, o[2 * s]);
            o[2 * s + 1] = mfma(v1, phi, o[2 * s + 1]);
            o[2 * s + 1] = mfma(v1, plo, o[2 * s + 1]);
        }
    };

    // Two register sets in a ring, loads always issued (past the end they
    // re-read the last pair, an L2 hit) so the compiler can count the loads
    // in flight and wait only for the set about to be consumed.
    const int last_pair = p0 + ((p1 - 1 - p0) & ~1);
    PageRegs ra, rb;
    load(p0, ra);
    load(min(p0 + 2, last_pair), rb);
    for (int pp = p0; pp < p1; pp += 4) {
        consume(ra, pp);
        load(min(pp + 4, last_pair), ra);
        if (pp + 2 < p1) consume(rb, pp + 2);
        load(min(pp + 6, last_pair), rb);
    }
    lsum += __shfl_xor(lsum, 16);
    lsum += __shfl_xor(lsum, 32);

    const size_t out_base = (size_t(q0 + (col_ok ? qi : 0)) * a.nh + h * G + g) * kHeadDim;
    if (nsplit == 1) {
        if (col_ok) {
            const float inv = 1.f / lsum;
#pragma unroll
            for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, out_base, i, grp, o[i] * inv);
        }
        return;
    }

    float *part = a.partial + (size_t(unit) * a.max_splits) * kPartialFloats;
    if (col_ok) {
        float *mine = part + size_t(split) * kPartialFloats;
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<f32x4 *>(mine + n * kHeadDim + i * 16 + grp * 4) = o[i];
        if (grp == 0) {
            mine[16 * kHeadDim + 2 * n] = m;
            mine[16 * kHeadDim + 2 * n + 1] = lsum;
        }
    }
    __threadfence();
    int prev = 0;
    if (lane == 0) prev = atomicAdd(a.counters + unit, 1);
    prev = __shfl(prev, 0);
    if (prev != nsplit - 1) return;
    __threadfence();
    if (col_ok) {
        float M = -INFINITY;
        for (int s = 0; s < nsplit; ++s) M = fmaxf(M, part[size_t(s) * kPartialFloats + 16 * kHeadDim + 2 * n]);
        float L = 0.f;
        f32x4 acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < nsplit; ++s) {
            const float *ps = part + size_t(s) * kPartialFloats;
            const float w = exp2Fast(ps[16 * kHeadDim + 2 * n] - M);
            L += w * ps[16 * kHeadDim + 2 * n + 1];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                acc[i] += w * *reinterpret_cast<const f32x4 *>(ps + n * kHeadDim + i * 16 + grp * 4);
        }
        const float inv = 1.f / L;
#pragma unroll
        for (int i = 0; i < 8; ++i) storeOut<OUT_F32>(a.out, out_base, i, grp, acc[i] * inv);
    }
    if (lane == 0) __hip_atomic_store(a.counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int envInt(const char *name, int fallback) {
    const char *v = std::getenv(name);
    if (!v || !*v) return fallback;
    return std::atoi(v);
}

} // namespace

PagedAttentionPlan planPagedAttention(int B, int T, int nkvh, int group, int max_pages, bool varlen) {
    PagedAttentionPlan p{};
    const int tiles = varlen ? (T * group + 15) / 16 + B : B;
    p.units = tiles * nkvh;
    p.units_padded = (p.units + kXcds - 1) / kXcds * kXcds;
    // Pages per split: even (pairs of pages), at most 64 (one block id per lane).
    int pps = envInt("LLAISYS_PAGES_PER_SPLIT", varlen ? 32 : 16);
    pps = std::max(2, std::min(64, pps & ~1));
    p.pages_per_split = pps;
    p.max_splits = std::max(1, (max_pages + pps - 1) / pps);
    p.partial_bytes = size_t(p.units_padded) * p.max_splits * kPartialFloats * sizeof(float);
    return p;
}

void pagedAttention(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                    const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_q, int B, int T, int nh,
                    int nkvh, int max_pages, int num_blocks, float scale, const PagedAttentionPlan &plan,
                    float *partial, int *counters, int *err, void *stream) {
    if (B == 0 || T == 0) return;
    Args a;
    a.q = q;
    a.out = out;
    a.k_pool = k_pool;
    a.v_pool = v_pool;
    a.table = block_table;
    a.ctx = ctx_len;
    a.cu_q = cu_q;
    a.partial = partial;
    a.counters = counters;
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
    const dim3 grid(plan.units_padded * plan.max_splits);
    auto s = static_cast<hipStream_t>(stream);
    const bool varlen = cu_q != nullptr;
    if (out_f32) {
        if (varlen)
            hipLaunchKernelGGL((pagedAttentionKernel<true, true>), grid, dim3(64), 0, s, a);
        else
            hipLaunchKernelGGL((pagedAttentionKernel<true, false>), grid, dim3(64), 0, s, a);
    } else {
        if (varlen)
            hipLaunchKernelGGL((pagedAttentionKernel<false, true>), grid, dim3(64), 0, s, a);
        else
            hipLaunchKernelGGL((pagedAttentionKernel<false, false>), grid, dim3(64), 0, s, a);
    }
    HIP_CHECK(hipGetLastError());
}

} // namespace llaisys::kernels
