// Host-side launchers for the HIP kernels. Plain pointers and sizes only; the
// op layer (ops/attention.cpp) validates tensors and calls these.
#pragma once

#include <cstddef>
#include <cstdint>

namespace llaisys::kernels {

// Page geometry fixed by the MI355X page format.
constexpr int kPageTokens = 16;
constexpr int kHeadDim = 128;
constexpr int kPageElems = kPageTokens * kHeadDim; // bf16 elements per (block, kv head) page

enum class ElemType { F32, F16, BF16 };

// Contiguous causal GQA attention (the reference's self_attention op).
void selfAttention(void *out, const void *q, const void *k, const void *v, ElemType type, int L, int S, int nh,
                   int nkvh, int d, int dv, float scale, void *stream);

// Paged KV append; cu_new may be null (one token per sequence, T == B).
void pagedAppend(uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new, const uint16_t *v_new,
                 const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_new, int T, int B, int nkvh,
                 int max_pages, int num_blocks, int *err, void *stream);

void pagedGather(uint16_t *k_out, uint16_t *v_out, const uint16_t *k_pool, const uint16_t *v_pool,
                 const int32_t *block_table, const int32_t *cu_seqlens, int T, int B, int nkvh, int max_pages,
                 int num_blocks, int *err, void *stream);

// Batched decode (one query per sequence): stream-K over all page pairs, then
// a combine kernel for sequences split across waves.
struct DecodePlan {
    int waves;           // grid of single-wave workgroups
    int stages;          // page pairs in flight per wave
    size_t record_bytes; // workspace for split records
    size_t lds_bytes;    // per-workgroup LDS (length prefix)
};
constexpr int kDecodeMaxBatch = 4096; // sequences per launch (LDS-resident prefix)
DecodePlan planDecode(int B, int nkvh, int group, int max_pages);
void pagedDecode(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                 const int32_t *block_table, const int32_t *ctx_len, int B, int nh, int nkvh, int max_pages,
                 int num_blocks, float scale, const DecodePlan &plan, float *records, int *err, void *stream);

struct PagedAttentionPlan {
    int units;          // (query tile, kv head) work units
    int units_padded;   // rounded up to a multiple of the XCD count
    int max_splits;     // split-KV partitions per unit
    int pages_per_split;
    size_t partial_bytes; // workspace for split partials
};

// Decode (cu_q == nullptr: one query per sequence, T == B) or varlen
// (chunked prefill + decode). out is F32 when out_f32 else BF16.
PagedAttentionPlan planPagedAttention(int B, int T, int nkvh, int group, int max_pages, bool varlen);

void pagedAttention(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                    const int32_t *block_table, const int32_t *ctx_len, const int32_t *cu_q, int B, int T, int nh,
                    int nkvh, int max_pages, int num_blocks, float scale, const PagedAttentionPlan &plan,
                    float *partial, int *counters, int *err, void *stream);

} // namespace llaisys::kernels
