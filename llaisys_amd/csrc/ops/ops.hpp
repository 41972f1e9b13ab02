// Operator layer: validate tensors, pick the device, launch kernels
// (dispatch pattern of the reference's src/ops/add/op.cpp:9-34).
#pragma once

#include "../tensor/tensor.hpp"

namespace llaisys::ops {

void selfAttention(const tensor_t &attn_val, const tensor_t &q, const tensor_t &k, const tensor_t &v, float scale);

void pagedKVAppend(const tensor_t &k_pool, const tensor_t &v_pool, const tensor_t &k_new, const tensor_t &v_new,
                   const tensor_t &block_table, const tensor_t &ctx_len, const tensor_t &cu_new /* may be null */);

void pagedKVGather(const tensor_t &k_out, const tensor_t &v_out, const tensor_t &k_pool, const tensor_t &v_pool,
                   const tensor_t &block_table, const tensor_t &cu_seqlens);
void pagedKVAppendGather(const tensor_t &k_out, const tensor_t &v_out, const tensor_t &k_pool, const tensor_t &v_pool,
                         const tensor_t &k_new, const tensor_t &v_new, const tensor_t &block_table,
                         const tensor_t &ctx_len, const tensor_t &cu_seqlens);

void pagedKVCopyBlocks(const tensor_t &k_pool, const tensor_t &v_pool, const tensor_t &pairs);

void pagedAttention(const tensor_t &out, const tensor_t &q, const tensor_t &k_pool, const tensor_t &v_pool,
                    const tensor_t &block_table, const tensor_t &ctx_len, const tensor_t &cu_q /* null = decode */,
                    float scale);

// Decode attention (pagedAttention with cu_q null) with no device allocation:
// split records in the decode kernel's fixed per-GPU scratch. AMD tensors only.
void pagedAttentionNoAlloc(const tensor_t &out, const tensor_t &q, const tensor_t &k_pool, const tensor_t &v_pool,
                           const tensor_t &block_table, const tensor_t &ctx_len, float scale);

// Model ops of the reference (README.md:145-292), AMD device.
void add(const tensor_t &c, const tensor_t &a, const tensor_t &b);
void argmax(const tensor_t &max_idx, const tensor_t &max_val, const tensor_t &vals);
void embedding(const tensor_t &out, const tensor_t &index, const tensor_t &weight);
void linear(const tensor_t &out, const tensor_t &in, const tensor_t &weight, const tensor_t &bias /* may be null */);
void rearrange(const tensor_t &out, const tensor_t &in);
// linear for decode-sized batches over a weight packed once by linearPackWeight
// (AMD, bf16; M <= 128, K == 1536, N % 16 == 0).
void linearPackWeight(const tensor_t &packed, const tensor_t &weight);
void linearPacked(const tensor_t &out, const tensor_t &in, const tensor_t &packed, const tensor_t &bias);
void rmsNorm(const tensor_t &out, const tensor_t &in, const tensor_t &weight, float eps);
void rope(const tensor_t &out, const tensor_t &in, const tensor_t &pos_ids, float theta);
void swiglu(const tensor_t &out, const tensor_t &gate, const tensor_t &up);

} // namespace llaisys::ops
