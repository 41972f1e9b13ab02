/*
 * Operator C-ABI.
 *
 * llaisysSelfAttention and the eight other reference ops keep the reference's
 * declarations (include/llaisys/ops.h:7-15) so python/llaisys/libllaisys/ops.py
 * binds unchanged. Every op dispatches on its tensors' device, as the
 * reference's src/ops/add/op.cpp:16-33 does: LLAISYS_DEVICE_AMD tensors run the
 * HIP kernels, LLAISYS_DEVICE_CPU tensors the host implementations (fp32 math,
 * host threads); one call may not mix devices. F32, F16, BF16; indices I64;
 * contiguous unless stated. Contracts are the reference README's
 * (README.md:157-292).
 *
 * The llaisysPagedKV* / llaisysPagedAttention* entry points are new. The
 * reference has no paged KV code; they follow its op conventions
 * (include/llaisys/ops.h:6-16: tensor handles and scalars in, void out, output
 * written in place, errors reported as the reference reports them).
 *
 * Paged KV pool (one per layer, one for K and one for V):
 *   shape [num_blocks, nkvh, 16, 128], dtype BF16, contiguous, on the AMD
 *   device or the host (the same page format on both).
 *   A (block, kv-head) page holds 16 tokens x 128 dims = 4 KiB. Inside a page
 *   the bytes are in the MI355X page format, not row-major [16][128]:
 *     K page: element (token t, dim d) at bf16 index
 *             (d / 8) * 128 + t * 8 + (d % 8)              ([16 dim-chunks][16 t][8])
 *     V page: element (t, d) at bf16 index
 *             (d / 32) * 512 + (t / 4) * 128 + (d % 16) * 8 + ((d / 16) % 2) * 4 + t % 4
 *   so that every 1 KiB of a page is exactly one 64-lane x 16-byte load that
 *   feeds a gfx950 MFMA operand. Only llaisysPagedKVAppend writes this format
 *   and llaisysPagedKVGather reads it back to row-major; callers never need it.
 * Block table: [B, max_pages] I32; entry (b, p) is the physical block holding
 *   tokens [16p, 16p+16) of sequence b. ctx_len: [B] I32 = tokens in the cache.
 */
#ifndef LLAISYS_OPS_H
#define LLAISYS_OPS_H

#include "tensor.h"

__C {
    /* ops.h:7: c = a + b, one shape and dtype. */
    __export void llaisysAdd(llaisysTensor_t c, llaisysTensor_t a, llaisysTensor_t b);
    /* ops.h:8: max over the last dim of vals; max_idx I64 and max_val (may be
     * NULL) hold one element per row (1 for a 1-D vals, README.md:161-167). */
    __export void llaisysArgmax(llaisysTensor_t max_idx, llaisysTensor_t max_val, llaisysTensor_t vals);
    /* ops.h:9: out[i] = weight[index[i]], index I64 (README.md:171-177). */
    __export void llaisysEmbedding(llaisysTensor_t out, llaisysTensor_t index, llaisysTensor_t weight);
    /* ops.h:10: out = in . weight^T + bias, weight [out, in], bias may be NULL
     * (README.md:181-198); a hand-written MFMA GEMM, fp32 accumulation,
     * one rounding; no GEMM library is linked. */
    __export void llaisysLinear(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t weight, llaisysTensor_t bias);
    /* New; no counterpart in the reference (whose linear is ops.h:10). The
     * weight of llaisysLinear, rewritten once into the layout the decode GEMM
     * streams (tiles of 16 rows x 32 columns in MFMA operand order): packed
     * and weight are [N, K] BF16 on the AMD device, N % 16 == 0, K % 32 == 0. */
    __export void llaisysLinearPackWeight(llaisysTensor_t packed, llaisysTensor_t weight);
    /* New; no counterpart in the reference. out = in . W^T + bias (bias may be
     * NULL) as llaisysLinear computes it (fp32 accumulation, one rounding),
     * with W given packed by llaisysLinearPackWeight; for decode-sized batches:
     * in [M, K], out [M, N] BF16 on the AMD device, 1 <= M <= 128, and
     * either K == 1536, N % 16 == 0, or 1536 < K <= 16384, K % 32 == 0,
     * N % 128 == 0 (split over K into fp32 partials in the runtime's device
     * workspace, summed in a fixed order); other shapes: llaisysLinear. */
    __export void llaisysLinearPacked(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t packed,
                                      llaisysTensor_t bias);
    /* ops.h:11: copy between equal shapes with any strides (README.md:286-292). */
    __export void llaisysRearrange(llaisysTensor_t out, llaisysTensor_t in);
    /* ops.h:12: y = w * x / sqrt(mean(x^2) + eps) per row (README.md:202-217). */
    __export void llaisysRmsNorm(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t weight, float eps);
    /* ops.h:13: rotary embedding of [seqlen, nhead, d] by pos_ids I64 (README.md:221-242). */
    __export void llaisysROPE(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t pos_ids, float theta);
    /* ops.h:15: out = up * gate / (1 + exp(-gate)) (README.md:268-278). */
    __export void llaisysSwiGLU(llaisysTensor_t out, llaisysTensor_t gate, llaisysTensor_t up);

    /* Replaces include/llaisys/ops.h:14 (stub src/ops/self_attention/op.cpp:4-6;
     * semantics README.md:244-266, test/ops/self_attention.py:11-28).
     * attn_val [L, nh, dv], q [L, nh, d], k [S, nkvh, d], v [S, nkvh, dv], all
     * contiguous, one dtype (F32, F16 or BF16), nh % nkvh == 0, S >= L,
     * d, dv <= 256. Query i attends keys j <= i + S - L; query head h reads
     * kv head h / (nh / nkvh). Accumulates in fp32, rounds once to the dtype. */
    __export void llaisysSelfAttention(llaisysTensor_t attn_val, llaisysTensor_t q, llaisysTensor_t k,
                                       llaisysTensor_t v, float scale);

    /* New. Scatter new K/V tokens into their pages.
     * k_new, v_new: [T, nkvh, 128] BF16. cu_new: [B+1] I32 prefix offsets, or
     * NULL meaning T == B and one token per sequence. Row r of sequence b
     * (cu_new[b] <= r < cu_new[b+1]) is written at position
     * ctx_len[b] + (r - cu_new[b]), i.e. ctx_len is the length BEFORE the append
     * and is not modified. Pages for every written position must already be
     * mapped in block_table. Bit-exact copy. */
    __export void llaisysPagedKVAppend(llaisysTensor_t k_pool, llaisysTensor_t v_pool, llaisysTensor_t k_new,
                                       llaisysTensor_t v_new, llaisysTensor_t block_table, llaisysTensor_t ctx_len,
                                       llaisysTensor_t cu_new);

    /* New. Copy the first cu_seqlens[b+1]-cu_seqlens[b] tokens of each
     * sequence out of the pool into rows [cu_seqlens[b], cu_seqlens[b+1]) of
     * k_out, v_out: [T, nkvh, 128] BF16 row-major. Bit-exact. */
    __export void llaisysPagedKVGather(llaisysTensor_t k_out, llaisysTensor_t v_out, llaisysTensor_t k_pool,
                                       llaisysTensor_t v_pool, llaisysTensor_t block_table,
                                       llaisysTensor_t cu_seqlens);

    /* New; no counterpart in the reference (its KV cache is a README prompt,
     * README.md:316, :412). llaisysPagedKVAppend of one token per sequence
     * (k_new, v_new: [B, nkvh, 128] BF16, written at position ctx_len[b])
     * followed by llaisysPagedKVGather of the contexts including it, in one
     * launch: cu_seqlens [B+1] must give every sequence ctx_len[b] + 1 output
     * rows (a sequence that does not raises device error flag 2 and is
     * skipped). Same bytes in the pool and in k_out, v_out as the two calls. */
    __export void llaisysPagedKVAppendGather(llaisysTensor_t k_out, llaisysTensor_t v_out, llaisysTensor_t k_pool,
                                             llaisysTensor_t v_pool, llaisysTensor_t k_new, llaisysTensor_t v_new,
                                             llaisysTensor_t block_table, llaisysTensor_t ctx_len,
                                             llaisysTensor_t cu_seqlens);

    /* New. Copy whole (block, all kv heads) pages inside the pools:
     * pairs [P, 2] I32 of (src, dst) block ids, as produced by
     * llaisysKVSeqReserve for copy-on-write of a shared last block. */
    __export void llaisysPagedKVCopyBlocks(llaisysTensor_t k_pool, llaisysTensor_t v_pool, llaisysTensor_t pairs);

    /* New. Batched decode attention (flash-decoding with split-KV and a
     * log-sum-exp combine): q [B, nh, 128] BF16, out [B, nh, 128] BF16 or F32.
     * Sequence b's single query attends all ctx_len[b] (>= 1) cached tokens,
     * which include the token appended for this step.
     * nh % nkvh == 0 and nh / nkvh <= 16. fp32 accumulation. */
    __export void llaisysPagedAttention(llaisysTensor_t out, llaisysTensor_t q, llaisysTensor_t k_pool,
                                        llaisysTensor_t v_pool, llaisysTensor_t block_table, llaisysTensor_t ctx_len,
                                        float scale);

    /* No counterpart in the reference. llaisysPagedAttention (same arguments,
     * same results to fp32 rounding, AMD tensors only) for callers that cannot
     * allocate device memory: HIP graph capture, fixed-memory serving loops.
     * The split records live in a fixed 16 MiB array that each GPU holds for
     * the life of the process; a batch whose records need more (2 x W x G x
     * 130 floats, W = max(1.75 x CUs, pairs / 64)) is refused with an error.
     * Calls that overlap on one GPU (two streams, two host threads) share the
     * array and race. The device's set-up (its first library call) allocates
     * the error word; this entry point itself allocates nothing. */
    __export void llaisysPagedAttentionNoAlloc(llaisysTensor_t out, llaisysTensor_t q, llaisysTensor_t k_pool,
                                               llaisysTensor_t v_pool, llaisysTensor_t block_table,
                                               llaisysTensor_t ctx_len, float scale);

    /* New. Mixed chunked-prefill + decode attention over paged KV.
     * q, out [T, nh, 128]; sequence b owns query rows [cu_q[b], cu_q[b+1]) and
     * Lq = cu_q[b+1]-cu_q[b] (>= 1, <= ctx_len[b]) of its ctx_len[b] cached
     * tokens are those queries' own tokens (already appended). Query i sits at
     * position ctx_len[b] - Lq + i and attends keys at positions <= that
     * (bottom-right causal alignment, test/ops/self_attention.py:18). */
    __export void llaisysPagedAttentionVarlen(llaisysTensor_t out, llaisysTensor_t q, llaisysTensor_t k_pool,
                                              llaisysTensor_t v_pool, llaisysTensor_t block_table,
                                              llaisysTensor_t cu_q, llaisysTensor_t ctx_len, float scale);
}

#endif /* LLAISYS_OPS_H */
