/*
 * Test hooks: the decode step's fused packed-operand kernels called one at a
 * time, for kernel-level parity tests. New; no counterpart in the reference
 * (its model path is declared in include/llaisys/models/qwen2.h:7-40 and has
 * no kernels). The Qwen2 model runs these kernels inside its batched decode
 * step (llaisysQwen2ModelStep / llaisysQwen2ModelDecode); here they take
 * plain device pointers and sizes (bf16 data as 16-bit words, i32 tables),
 * run on the context stream and synchronise it before returning. Errors are
 * reported as by every entry point (stderr line + llaisysGetLastError);
 * device-side bits (a bad block id, a position past the table) go to
 * llaisysGetDeviceErrorFlags.
 *
 * "Packed" rows are the MFMA operand order of an [R, K] matrix (K % 32 == 0):
 * element (r, k) at index
 *   ((r / 16) * (K / 32) + k / 32) * 512 + ((r % 16) + 16 * ((k / 8) % 4)) * 8 + k % 8
 * in a buffer of ceil(R / 16) * 16 * K elements (rows past R are never read
 * back into an output).
 */
#ifndef LLAISYS_TESTING_H
#define LLAISYS_TESTING_H

#include "../llaisys.h"

#include <stdint.h>

__C {
    /* packed[N, K] = w (times fold_g[k] per column, rounded once, when
     * fold_g is not NULL), N % 16 == 0, K % 32 == 0. */
    __export void llaisysTestPackWeight(void *packed, const void *w, const void *fold_g, int N, int K);
    /* A [gate; up] weight of 2 di rows, packed with block b holding gate rows
     * 8b .. 8b + 7 then the matching up rows (di % 8 == 0). */
    __export void llaisysTestPackWeightGateUp(void *packed, const void *w, int di, int K);
    /* y[M, N] (+)= x . W^T, x and W packed, K == 1536, N % 32 == 0,
     * M <= 128; y_packed (may be NULL) also receives y packed. */
    __export void llaisysTestPackedXGemm(void *y, const void *x_packed, const void *w_packed, int M, int N, int K,
                                         int accumulate, void *y_packed);
    /* The QKV projection with its epilogue, one token per row (row m is
     * sequence m at position ctx[m]): y = r (x W^T) + bias with r the row's
     * 1/sqrt(mean(x^2) + eps), q and k heads rotated by RoPE (theta), q to
     * q[M, nh, 128], k and v into their page slot of the pools
     * [num_blocks, nkvh, 16, 128] through table[M, max_pages]. */
    __export void llaisysTestQkvRopeGemm(void *q, void *k_pool, void *v_pool, const void *x_packed,
                                         const void *w_packed, const void *bias, const int32_t *table,
                                         const int32_t *ctx, int M, int nh, int nkvh, int K, int max_pages,
                                         int num_blocks, float eps, float theta);
    /* act[M, di] = up * silu(gate) of r (x [gate; up]^T), W packed by
     * llaisysTestPackWeightGateUp; act_packed: act written packed instead. */
    __export void llaisysTestGateUpSwiglu(void *act, const void *x_packed, const void *w_packed, int M, int di, int K,
                                          float eps, int act_packed);
    /* y[M, N] (+)= x . W^T for 1536 < K <= 16384 (split over K, the fp32
     * partials summed in a fixed order), x and W packed, N % 64 == 0,
     * M <= 128; y_packed (may be NULL) also receives y packed. */
    __export void llaisysTestSplitKPackedGemm(void *y, const void *x_packed, const void *w_packed, int M, int N,
                                              int K, int accumulate, void *y_packed);
    /* The long steps' gate-up: out[2 di, K] = the rows of w [gate (di); up
     * (di)] as 16-row blocks gate 0, up 0, gate 1, ... (di % 16 == 0); then
     * act[M, di] = up * silu(gate) of x[M, K] . out^T in one GEMM launch,
     * gate and up rounded to bf16 before the SwiGLU (x row-major). */
    __export void llaisysTestSwigluInterleave(void *out, const void *w, int di, int K);
    __export void llaisysTestLinearSwiglu(void *act, const void *x, const void *w_interleaved, int M, int di, int K);
}

#endif
