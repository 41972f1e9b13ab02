/*
 * CPU ORACLE for the LLAISYS KV-cache attention path — TEST INFRASTRUCTURE.
 *
 * This library is the checker: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it. The product (llaisys_amd /
 * libllaisys.so) never links or calls it.
 *
 * It restates the reference's specification in plain C:
 *   - self_attention: README.md:244-266 and the executable formula in
 *     test/ops/self_attention.py:11-28 (bottom-right causal mask
 *     tril(diagonal=S-L) at :17-18; GQA by repeat_interleave at :22-23, so
 *     query head h reads kv head h / (nh/nkvh); softmax(QK^T * scale) V at
 *     :25-28). Inputs are fp32 (bf16/f16 inputs are widened exactly by the
 *     caller); accumulation and output are fp32.
 *   - paged KV (no reference code exists; README.md:316, :412, :424 motivate
 *     it): a pool of 16-token pages addressed through per-sequence block
 *     tables; append writes token r of sequence b at position
 *     ctx[b] + (r - cu[b]); gather copies positions [0, len) back out.
 *     These work on the LOGICAL pool layout [num_blocks][nkvh][16][128]; the
 *     device page format is a fixed permutation inside each page
 *     (orc_pack_pages / orc_unpack_pages).
 *   - paged attention = gather + self_attention per sequence, query i of a
 *     sequence with Lq queries sitting at position ctx - Lq + i.
 *
 * Parity pins (tests/test_oracle.py): torch scaled_dot_product_attention in
 * float64, closed forms (S=1, scale=0 prefix means, constant-per-head values
 * for the GQA map), the reference test's shapes/tolerances, committed golden
 * fixtures, and the append/gather invariants on small pools.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define PAGE 16
#define HD 128

/* ---------------- self_attention (test/ops/self_attention.py:11-28) ------- */

/* One (query i, head h) row. scores: scratch of S floats. */
static void attend_row(float *out, const float *q, const float *k, const float *v, int S_vis, int nkvh, int d,
                       int dv, int kh, float scale, float *scores) {
    float mx = -INFINITY;
    for (int j = 0; j < S_vis; ++j) {
        const float *kr = k + ((size_t)j * nkvh + kh) * d;
        float s = 0.f;
        for (int e = 0; e < d; ++e) s += q[e] * kr[e];
        s *= scale;
        scores[j] = s;
        if (s > mx) mx = s;
    }
    float sum = 0.f;
    for (int j = 0; j < S_vis; ++j) {
        scores[j] = expf(scores[j] - mx);
        sum += scores[j];
    }
    for (int e = 0; e < dv; ++e) out[e] = 0.f;
    for (int j = 0; j < S_vis; ++j) {
        const float p = scores[j] / sum;
        const float *vr = v + ((size_t)j * nkvh + kh) * dv;
        for (int e = 0; e < dv; ++e) out[e] += p * vr[e];
    }
}

/* out [L,nh,dv], q [L,nh,d], k [S,nkvh,d], v [S,nkvh,dv], all fp32. */
void orc_self_attention(float *out, const float *q, const float *k, const float *v, int L, int S, int nh, int nkvh,
                        int d, int dv, float scale, int nthreads) {
    const int G = nh / nkvh;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
    {
        float *scores = (float *)malloc(sizeof(float) * (size_t)(S > 0 ? S : 1));
#pragma omp for schedule(static)
        for (long r = 0; r < (long)L * nh; ++r) {
            const int i = (int)(r / nh), h = (int)(r % nh);
            /* key j visible iff j <= i + (S - L)  (tril(diagonal=S-L)) */
            const int S_vis = i + (S - L) + 1;
            attend_row(out + (size_t)r * dv, q + (size_t)r * d, k, v, S_vis, nkvh, d, dv, h / G, scale, scores);
        }
        free(scores);
    }
}

/* ---------------- paged KV, logical layout [nb][nkvh][16][128] ------------ */

static int owning_sequence(const int32_t *cu, int B, int r) {
    int b = 0;
    while (b + 1 < B && cu[b + 1] <= r) ++b;
    return b;
}

/* Returns 0 on success, 1 if a position had no mapped page / bad block id. */
int orc_paged_append(uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new, const uint16_t *v_new,
                     const int32_t *table, int max_pages, const int32_t *ctx, const int32_t *cu_new, int B, int T,
                     int nkvh, int num_blocks) {
    int bad = 0;
    for (int r = 0; r < T; ++r) {
        const int b = cu_new ? owning_sequence(cu_new, B, r) : r;
        const int pos = ctx[b] + (cu_new ? r - cu_new[b] : 0);
        const int page = pos / PAGE, t = pos % PAGE;
        if (page >= max_pages) { bad = 1; continue; }
        const int blk = table[(size_t)b * max_pages + page];
        if (blk < 0 || blk >= num_blocks) { bad = 1; continue; }
        for (int h = 0; h < nkvh; ++h) {
            const size_t dst = (((size_t)blk * nkvh + h) * PAGE + t) * HD;
            const size_t src = ((size_t)r * nkvh + h) * HD;
            memcpy(k_pool + dst, k_new + src, HD * sizeof(uint16_t));
            memcpy(v_pool + dst, v_new + src, HD * sizeof(uint16_t));
        }
    }
    return bad;
}

int orc_paged_gather(uint16_t *k_out, uint16_t *v_out, const uint16_t *k_pool, const uint16_t *v_pool,
                     const int32_t *table, int max_pages, const int32_t *cu, int B, int nkvh, int num_blocks) {
    int bad = 0;
    for (int b = 0; b < B; ++b) {
        for (int pos = 0; pos < cu[b + 1] - cu[b]; ++pos) {
            const int page = pos / PAGE, t = pos % PAGE;
            if (page >= max_pages) { bad = 1; continue; }
            const int blk = table[(size_t)b * max_pages + page];
            if (blk < 0 || blk >= num_blocks) { bad = 1; continue; }
            for (int h = 0; h < nkvh; ++h) {
                const size_t src = (((size_t)blk * nkvh + h) * PAGE + t) * HD;
                const size_t dst = ((size_t)(cu[b] + pos) * nkvh + h) * HD;
                memcpy(k_out + dst, k_pool + src, HD * sizeof(uint16_t));
                memcpy(v_out + dst, v_pool + src, HD * sizeof(uint16_t));
            }
        }
    }
    return bad;
}

/* ---------------- device page format (a permutation inside each page) ---- */

static size_t k_index(int t, int d) { return (size_t)(d / 8) * 128 + (size_t)t * 8 + (size_t)(d % 8); }
static size_t v_index(int t, int d) {
    return (size_t)(d / 32) * 512 + (size_t)(t / 4) * 128 + (size_t)(d % 16) * 8 + (size_t)((d / 16) % 2) * 4 +
           (size_t)(t % 4);
}

/* logical [npages][16][128] -> device format, is_v selects the V permutation. */
void orc_pack_pages(uint16_t *dev, const uint16_t *logical, long npages, int is_v) {
    for (long p = 0; p < npages; ++p)
        for (int t = 0; t < PAGE; ++t)
            for (int d = 0; d < HD; ++d)
                dev[p * PAGE * HD + (is_v ? v_index(t, d) : k_index(t, d))] = logical[(p * PAGE + t) * HD + d];
}

void orc_unpack_pages(uint16_t *logical, const uint16_t *dev, long npages, int is_v) {
    for (long p = 0; p < npages; ++p)
        for (int t = 0; t < PAGE; ++t)
            for (int d = 0; d < HD; ++d)
                logical[(p * PAGE + t) * HD + d] = dev[p * PAGE * HD + (is_v ? v_index(t, d) : k_index(t, d))];
}

/* ---------------- paged attention = gather + self_attention -------------- */

static float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/*
 * out [T,nh,128] fp32; q [T,nh,128] fp32 (widened bf16); pools logical bf16.
 * cu_q NULL means one query per sequence (T == B, decode).
 */
int orc_paged_attention(float *out, const float *q, const uint16_t *k_pool, const uint16_t *v_pool,
                        const int32_t *table, int max_pages, const int32_t *ctx, const int32_t *cu_q, int B, int nh,
                        int nkvh, int num_blocks, float scale, int nthreads) {
    int bad = 0;
    /* Sequences are independent: one thread per sequence at a time. */
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1) reduction(| : bad)
    for (int b = 0; b < B; ++b) {
        const int len = ctx[b];
        const int q0 = cu_q ? cu_q[b] : b;
        const int Lq = cu_q ? cu_q[b + 1] - cu_q[b] : 1;
        if (Lq == 0) continue;
        if (len <= 0 || (len + PAGE - 1) / PAGE > max_pages || Lq > len) {
            bad = 1;
            continue;
        }
        float *kc = (float *)malloc(sizeof(float) * (size_t)len * nkvh * HD);
        float *vc = (float *)malloc(sizeof(float) * (size_t)len * nkvh * HD);
        for (int pos = 0; pos < len; ++pos) {
            const int blk = table[(size_t)b * max_pages + pos / PAGE];
            const int ok = blk >= 0 && blk < num_blocks;
            if (!ok) bad = 1;
            for (int h = 0; h < nkvh; ++h)
                for (int e = 0; e < HD; ++e) {
                    const size_t src = ok ? (((size_t)blk * nkvh + h) * PAGE + pos % PAGE) * HD + e : 0;
                    kc[((size_t)pos * nkvh + h) * HD + e] = ok ? bf16_to_f32(k_pool[src]) : 0.f;
                    vc[((size_t)pos * nkvh + h) * HD + e] = ok ? bf16_to_f32(v_pool[src]) : 0.f;
                }
        }
        orc_self_attention(out + (size_t)q0 * nh * HD, q + (size_t)q0 * nh * HD, kc, vc, Lq, len, nh, nkvh, HD, HD,
                           scale, 1);
        free(kc);
        free(vc);
    }
    return bad;
}

/* Threads OpenMP would use, for reporting the CPU baseline's core count. */
int orc_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
