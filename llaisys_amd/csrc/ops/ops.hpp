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

void pagedKVCopyBlocks(const tensor_t &k_pool, const tensor_t &v_pool, const tensor_t &pairs);

void pagedAttention(const tensor_t &out, const tensor_t &q, const tensor_t &k_pool, const tensor_t &v_pool,
                    const tensor_t &block_table, const tensor_t &ctx_len, const tensor_t &cu_q /* null = decode */,
                    float scale);

[[noreturn]] void outOfScope(const char *op);

} // namespace llaisys::ops
