// Shared pieces of the gfx950 paged-attention kernels: vector types, the
// bf16 MFMA, and the page-pair step (scores, online softmax, P.V).
//
// Lane layout (64 lanes, n = lane % 16 "column", grp = lane / 16):
//   S^T[16 keys x 16 cols] = K_page[16 x 128] . Q^T[128 x 16]
//       4 x v_mfma_f32_16x16x32_bf16 per page; A operand (K) is one
//       coalesced 1 KiB load per 32 dims thanks to the K page format;
//       the accumulator gives each lane keys 4*grp+i of its column.
//   O^T[128 x 16 cols] += V^T[128 x 32 keys] . P^T[32 keys x 16 cols]
//       the 32 keys are 2 pages; key slot 8*grp+e is page A key 4*grp+e
//       (e<4) or page B key 4*grp+e-4, which is exactly what the S^T
//       accumulators of the two pages hold and what one 16 B load of the V
//       page format holds per 16-dim block pair. For fp32 output P = hi + lo
//       (two bf16, two MFMAs), so the product is accurate to ~2^-17 relative,
//       V being exact bf16; for bf16 output P is rounded once to bf16 (its
//       2^-9 error is below the output's own rounding), one MFMA.
// Nothing crosses lanes except the running max (2 shuffles).
#pragma once

#include "lanes.hpp"
#include "launch.hpp"

#include <hip/hip_runtime.h>

namespace llaisys::kernels::mfma {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kErrBadBlock = 1;
constexpr int kErrTooLong = 2;

__device__ __forceinline__ bf16x8 asBf16(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2Fast(float x) { return __builtin_amdgcn_exp2f(x); }

// maxOverGroups (lanes.hpp): max over the lanes n, n+16, n+32, n+48 (the
// four key groups of a column).
using kernels::maxOverGroups;

// Inclusive prefix sum over the 64 lanes of a wave with DPP: row shifts by
// 1, 2, 4, 8 sum within each row of 16 lanes (lanes without a source add 0),
// then row_bcast:15 adds row 0's total to row 1 and row 2's to row 3, and
// row_bcast:31 adds the total of rows 0-1 to rows 2-3. All VALU; a shuffle
// scan would take six LDS round trips.
__device__ __forceinline__ int waveInclusiveSum(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false); // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false); // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false); // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false); // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false); // row_bcast:15 -> rows 1, 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false); // row_bcast:31 -> rows 2, 3
    return x;
}

// Keeps the 16-bit halves of a word whose key is valid.
__device__ __forceinline__ uint32_t keepPair(bool lo, bool hi) {
    return (lo ? 0x0000ffffu : 0u) | (hi ? 0xffff0000u : 0u);
}

// Registers of one page pair (K and V of pages A and B).
struct PagePair {
    u32x4 ka[4], kb[4], va[4], vb[4];
};

// Issue the 16 loads of a page pair: page bases in u32x4 units, lane offset applied.
__device__ __forceinline__ void loadPair(PagePair &r, const u32x4 *kp, const u32x4 *vp, size_t oa, size_t ob) {
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
}

// Running attention state of one lane (its column, its 32 output dims).
struct Acc {
    f32x4 o[8];
    float m;
    float l;
    __device__ __forceinline__ void reset() {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        m = -INFINITY;
        l = 0.f;
    }
};

// P of one page pair for one lane's column, as bf16 (hi, and lo when SPLIT_P).
struct PairP {
    bf16x8 hi, lo;
};

// Raw scores of one page pair (K pages a, b) against the lane's column of
// each of NT query tiles, with keys a column may not see set to -inf.
// first_key = key position of page A's token 0; pos[k] = last key tile k's
// column may see (-1: none); hasB = page B exists. full = every key of the
// pair is visible to every column of the wave (wave-uniform): no per-key mask.
// A 16x16x32 MFMA's result reaches a dependent MFMA ~48 cycles after issue
// and MFMAs issue 16 cycles apart, so the NT tiles' page-A and page-B
// accumulator chains are interleaved (4 chains in flight with two tiles).
// (With one tile, splitting each page's 4 k steps over two chains, summed at
// the end, measured no faster in the memory-bound decode kernel.)
template <int NT>
__device__ __forceinline__ void pairScoresN(float (&sv)[NT][8], const u32x4 (&ka)[4], const u32x4 (&kb)[4],
                                            const u32x4 (&qop)[NT][4], int first_key, const int (&pos)[NT], bool hasB,
                                            int grp, bool full = false) {
    f32x4 sa[NT], sb[NT];
#pragma unroll
    for (int k = 0; k < NT; ++k) sa[k] = sb[k] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int k = 0; k < NT; ++k) {
            sa[k] = mfma(asBf16(ka[s]), asBf16(qop[k][s]), sa[k]);
            sb[k] = mfma(asBf16(kb[s]), asBf16(qop[k][s]), sb[k]);
        }
#pragma unroll
    for (int k = 0; k < NT; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sv[k][i] = sa[k][i];
            sv[k][4 + i] = sb[k][i];
        }
    // A branch of its own: folded into the selects, the wave-uniform `full`
    // would still leave every compare and select on the path.
    if (!full) {
        const int kbase = first_key + grp * 4;
#pragma unroll
        for (int k = 0; k < NT; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sv[k][i] = kbase + i <= pos[k] ? sv[k][i] : -INFINITY;
                sv[k][4 + i] = (hasB && kbase + 16 + i <= pos[k]) ? sv[k][4 + i] : -INFINITY;
            }
    }
}

// Online softmax over the raw scores of NP page pairs: update acc (running
// max in log2 units, sum, rescaled O) and return each pair's P. Scores enter
// as exp2(s * scale_log2 - m): the max is taken on raw scores (the scale is
// positive) and the scaling folds into one fma per key.
template <bool SPLIT_P, int NP>
__device__ __forceinline__ void softmaxUpdate(Acc &acc, const float (&sv)[NP][8], PairP (&P)[NP], float scale_log2) {
    float mloc = sv[0][0];
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) mloc = fmaxf(mloc, sv[j][i]);
    mloc = maxOverGroups(mloc);
    // Lazy rescale: a column keeps its running max until a score exceeds it
    // by more than 2^kLazyLog2 (P then stays below that bound). Only when some
    // column of the wave crosses it do all columns move to their true max and
    // rescale O and l; the normalised result is the same either way.
    constexpr float kLazyLog2 = 8.f;
    const float m_true = fmaxf(acc.m, mloc * scale_log2);
    if (__builtin_amdgcn_ballot_w64(m_true > acc.m + kLazyLog2) != 0) {
        const float alpha = exp2Fast(acc.m - ((m_true == -INFINITY) ? 0.f : m_true));
        acc.l *= alpha;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc.o[i] *= alpha;
        acc.m = m_true;
    }
    const float m_use = (acc.m == -INFINITY) ? 0.f : acc.m;
    float psum = 0.f;
#pragma unroll
    for (int j = 0; j < NP; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float p = exp2Fast(__builtin_fmaf(sv[j][i], scale_log2, -m_use));
            psum += p;
            const __bf16 hi = (__bf16)p;
            P[j].hi[i] = hi;
            if constexpr (SPLIT_P) P[j].lo[i] = (__bf16)(p - (float)hi);
        }
    acc.l += psum;
}

// Scores, online softmax update and P of one page pair (see pairScores).
template <bool SPLIT_P>
__device__ __forceinline__ PairP scorePair(Acc &acc, const u32x4 (&ka)[4], const u32x4 (&kb)[4], const u32x4 (&qop)[4],
                                          int first_key, int pos, bool hasB, int grp, float scale_log2) {
    float sv[1][8];
    const u32x4(&q1)[1][4] = *reinterpret_cast<const u32x4(*)[1][4]>(&qop);
    const int p1[1] = {pos};
    pairScoresN<1>(sv, ka, kb, q1, first_key, p1, hasB, grp);
    PairP P[1];
    softmaxUpdate<SPLIT_P, 1>(acc, sv, P, scale_log2);
    return P[0];
}

// Keys at or past ctx may hold stale bytes (even NaN patterns): zero their V
// so 0 * V stays 0. Only a sequence's last pair has any.
__device__ __forceinline__ void maskStaleV(u32x4 (&va)[4], u32x4 (&vb)[4], int first_key, int ctx, bool hasB, int grp) {
    if (first_key + 32 > ctx || !hasB) {
        const int kbase = first_key + grp * 4;
        const uint32_t ma01 = keepPair(kbase < ctx, kbase + 1 < ctx);
        const uint32_t ma23 = keepPair(kbase + 2 < ctx, kbase + 3 < ctx);
        const uint32_t mb01 = hasB ? keepPair(kbase + 16 < ctx, kbase + 17 < ctx) : 0u;
        const uint32_t mb23 = hasB ? keepPair(kbase + 18 < ctx, kbase + 19 < ctx) : 0u;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            va[s] &= u32x4{ma01, ma23, ma01, ma23};
            vb[s] &= u32x4{mb01, mb23, mb01, mb23};
        }
    }
}

// O^T += V^T . P^T for one page pair (V pages a, b already masked).
template <bool SPLIT_P>
__device__ __forceinline__ void accumulatePV(Acc &acc, const u32x4 (&va)[4], const u32x4 (&vb)[4], const PairP &P) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const bf16x8 v0 = asBf16(u32x4{va[s][0], va[s][1], vb[s][0], vb[s][1]});
        const bf16x8 v1 = asBf16(u32x4{va[s][2], va[s][3], vb[s][2], vb[s][3]});
        acc.o[2 * s] = mfma(v0, P.hi, acc.o[2 * s]);
        acc.o[2 * s + 1] = mfma(v1, P.hi, acc.o[2 * s + 1]);
        if constexpr (SPLIT_P) {
            acc.o[2 * s] = mfma(v0, P.lo, acc.o[2 * s]);
            acc.o[2 * s + 1] = mfma(v1, P.lo, acc.o[2 * s + 1]);
        }
    }
}

// The same two steps with V already in operand order: v0[s] = {A.x, A.y, B.x,
// B.y} and v1[s] = {A.z, A.w, B.z, B.w} of quarter s (the prefill kernel's LDS
// stages hold V this way, so no register moves assemble the operands).
__device__ __forceinline__ void maskStaleVPacked(u32x4 (&v0)[4], u32x4 (&v1)[4], int first_key, int ctx, bool hasB,
                                                 int grp) {
    if (first_key + 32 > ctx || !hasB) {
        const int kbase = first_key + grp * 4;
        const uint32_t ma01 = keepPair(kbase < ctx, kbase + 1 < ctx);
        const uint32_t ma23 = keepPair(kbase + 2 < ctx, kbase + 3 < ctx);
        const uint32_t mb01 = hasB ? keepPair(kbase + 16 < ctx, kbase + 17 < ctx) : 0u;
        const uint32_t mb23 = hasB ? keepPair(kbase + 18 < ctx, kbase + 19 < ctx) : 0u;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            v0[s] &= u32x4{ma01, ma23, mb01, mb23};
            v1[s] &= u32x4{ma01, ma23, mb01, mb23};
        }
    }
}

template <bool SPLIT_P>
__device__ __forceinline__ void accumulatePVPacked(Acc &acc, const u32x4 (&v0)[4], const u32x4 (&v1)[4],
                                                   const PairP &P) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        acc.o[2 * s] = mfma(asBf16(v0[s]), P.hi, acc.o[2 * s]);
        acc.o[2 * s + 1] = mfma(asBf16(v1[s]), P.hi, acc.o[2 * s + 1]);
        if constexpr (SPLIT_P) {
            acc.o[2 * s] = mfma(asBf16(v0[s]), P.lo, acc.o[2 * s]);
            acc.o[2 * s + 1] = mfma(asBf16(v1[s]), P.lo, acc.o[2 * s + 1]);
        }
    }
}

// Consume one page pair: scores, online softmax and P.V (see scorePair for
// the arguments; ctx = keys in cache, whose later slots get zeroed V).
// SPLIT_P: P enters P.V as hi + lo bf16 parts (fp32-accurate) or as one bf16.
template <bool SPLIT_P>
__device__ __forceinline__ void consumePair(Acc &acc, PagePair &r, const u32x4 (&qop)[4], int first_key, int pos,
                                           int ctx, bool hasB, int grp, float scale_log2) {
    const PairP P = scorePair<SPLIT_P>(acc, r.ka, r.kb, qop, first_key, pos, hasB, grp, scale_log2);
    maskStaleV(r.va, r.vb, first_key, ctx, hasB, grp);
    accumulatePV<SPLIT_P>(acc, r.va, r.vb, P);
}

// Output dims of lane (n, grp) for block i: 16*i + 4*grp + {0..3}.
template <bool OUT_F32>
__device__ __forceinline__ void storeOut(void *out, size_t row_base, int blk, int grp, f32x4 v) {
    const size_t idx = row_base + blk * 16 + grp * 4;
    if constexpr (OUT_F32) {
        *reinterpret_cast<f32x4 *>(static_cast<float *>(out) + idx) = v;
    } else {
        const __bf16 e0 = (__bf16)v[0], e1 = (__bf16)v[1], e2 = (__bf16)v[2], e3 = (__bf16)v[3];
        const uint32_t w0 =
            uint32_t(__builtin_bit_cast(uint16_t, e0)) | (uint32_t(__builtin_bit_cast(uint16_t, e1)) << 16);
        const uint32_t w1 =
            uint32_t(__builtin_bit_cast(uint16_t, e2)) | (uint32_t(__builtin_bit_cast(uint16_t, e3)) << 16);
        *reinterpret_cast<uint2 *>(static_cast<uint16_t *>(out) + idx) = make_uint2(w0, w1);
    }
}

} // namespace llaisys::kernels::mfma
