// Host (LLAISYS_DEVICE_CPU) implementations of the ops, for tensors that live
// in host memory. The reference dispatches every op on the tensor's device and
// keeps a CPU implementation beside each device one (src/ops/add/op.cpp:16-33,
// src/ops/add/cpu/add_cpu.cpp:7-33); these are that CPU side. Plain pointers
// and sizes, as the HIP launchers in kernels/launch.hpp take them. Math is
// fp32; each result is rounded once to the tensor dtype. Work is split over
// host threads (LLAISYS_CPU_THREADS, default: the CPUs the process may run on).
#pragma once

#include "../../kernels/launch.hpp"

#include <cstddef>
#include <cstdint>

namespace llaisys::cpu {

using kernels::ElemType;

// Host threads the CPU ops use (>= 1).
int threads();

void add(void *c, const void *a, const void *b, ElemType t, size_t n);
void argmax(int64_t *idx, void *val, const void *vals, ElemType t, size_t rows, int64_t n);
// Rows whose index is outside [0, vocab) are skipped and raise error bit 4.
void embedding(void *out, const int64_t *idx, const void *weight, ElemType t, size_t rows, int64_t vocab, int d,
               int *err);
// out[M, N] = in[M, K] . weight[N, K]^T (+ bias[N]); fp32 accumulation.
void linear(void *out, const void *in, const void *weight, const void *bias, ElemType t, int M, int N, int K);
void rearrange(void *out, const void *in, size_t esz, int ndim, const int64_t *shape, const int64_t *out_strides,
               const int64_t *in_strides);
void rmsNorm(void *out, const void *x, const void *w, ElemType t, size_t rows, int d, float eps);
void rope(void *out, const void *in, const int64_t *pos, ElemType t, size_t ntok, int nhead, int d, float theta);
void swiglu(void *out, const void *gate, const void *up, ElemType t, size_t n);

// Contiguous causal GQA attention: query i attends keys j <= i + S - L; query
// head h reads kv head h / (nh / nkvh).
void selfAttention(void *out, const void *q, const void *k, const void *v, ElemType t, int L, int S, int nh,
                   int nkvh, int d, int dv, float scale);

// Paged KV on host pools in the page format documented in include/llaisys/ops.h.
// Error bits as the device kernels raise them: 1 = block id outside the pool,
// 2 = position or rows outside the table / outputs. Flagged rows are skipped.
void pagedAppend(uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new, const uint16_t *v_new,
                 const int32_t *table, const int32_t *ctx, const int32_t *cu_new, int T, int B, int nkvh,
                 int max_pages, int num_blocks, int *err);
void pagedGather(uint16_t *k_out, uint16_t *v_out, const uint16_t *k_pool, const uint16_t *v_pool,
                 const int32_t *table, const int32_t *cu, int T, int B, int nkvh, int max_pages, int num_blocks,
                 int *err);
void pagedAppendGather(uint16_t *k_out, uint16_t *v_out, uint16_t *k_pool, uint16_t *v_pool, const uint16_t *k_new,
                       const uint16_t *v_new, const int32_t *table, const int32_t *ctx, const int32_t *cu, int T,
                       int B, int nkvh, int max_pages, int num_blocks, int *err);
void pagedCopyBlocks(uint16_t *k_pool, uint16_t *v_pool, const int32_t *pairs, int P, int nkvh, int num_blocks,
                     int *err);
// Paged attention. cu_q == nullptr: one query per sequence (row b). Else
// sequence b owns rows [cu_q[b], cu_q[b+1]), bottom-right causal. out is bf16
// or fp32 (out_f32). Sequences flagged with bit 2 get zero rows; pages with a
// bad block id (bit 1) are left out of the softmax.
void pagedAttention(void *out, bool out_f32, const uint16_t *q, const uint16_t *k_pool, const uint16_t *v_pool,
                    const int32_t *table, const int32_t *ctx, const int32_t *cu_q, int B, int T, int nh, int nkvh,
                    int max_pages, int num_blocks, float scale, int *err);

} // namespace llaisys::cpu
