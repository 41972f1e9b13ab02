/*
 * Continuous-batching scheduler (no reference counterpart: the reference's
 * README asks for continuous batching over a KV-cache pool with prefix
 * matching as a project, README.md:421-424, and ships no code for it).
 *
 * Requests (prompt, max_new_tokens, end token) queue up; each Step runs one
 * mixed batch on the model: a single-token decode for every running request,
 * then prefill chunks (at most prefill_chunk prompt tokens per request,
 * max_step_tokens tokens per step in total) of admitted requests, admitting
 * waiting requests in arrival order while max_seqs, the token budget and the
 * KV pool allow. When the pool cannot hold the next decodes the most recently
 * admitted requests are preempted and later recomputed (cached full blocks
 * are reused). Greedy decoding depends only on a request's own tokens, so its
 * output is the same however it was batched, chunked or preempted.
 *
 * Functions return >= 0 on success and -1 on failure (llaisysGetLastError
 * has the message). A scheduler over a model must be destroyed before the
 * model, and is driven from the model's thread.
 */
#ifndef LLAISYS_SERVING_H
#define LLAISYS_SERVING_H

#include "models/qwen2.h"

__C {
    struct LlaisysScheduler;

    /* Request status of llaisysSchedulerStatus. */
    typedef enum {
        LLAISYS_REQUEST_ACTIVE = 0,      /* waiting or running */
        LLAISYS_REQUEST_MAX_TOKENS = 1,  /* finished: max_new_tokens generated */
        LLAISYS_REQUEST_EOS = 2,         /* finished: generated the end token */
        LLAISYS_REQUEST_LENGTH = 3,      /* finished: the sequence reached meta.maxseq */
        LLAISYS_REQUEST_NO_CAPACITY = 4, /* finished: the KV pool cannot hold it */
    } llaisysRequestStatus_t;

    /* Scheduler over a Qwen2 model (its KV pool and llaisysQwen2ModelStep). */
    __export struct LlaisysScheduler *llaisysQwen2SchedulerCreate(struct LlaisysQwen2Model * model, size_t max_seqs,
                                                                   size_t max_step_tokens, size_t prefill_chunk);
    /* Scheduler over a host-only simulated model, for testing without a GPU:
     * a KV pool of num_blocks blocks (the same block manager as the model)
     * and greedy token = FNV-1a-64 hash of the sequence's token history
     * (offset 14695981039346656037, prime 1099511628211, each int64 token
     * XORed in whole) modulo vocab. */
    __export struct LlaisysScheduler *llaisysSimSchedulerCreate(size_t num_blocks, int64_t vocab, size_t max_seq_len,
                                                                 size_t max_seqs, size_t max_step_tokens,
                                                                 size_t prefill_chunk);
    /* Frees the sequences the scheduler still holds. */
    __export void llaisysSchedulerDestroy(struct LlaisysScheduler * s);
    /* Queue a request (eos < 0: none); returns its id. */
    __export int64_t llaisysSchedulerAdd(struct LlaisysScheduler * s, const int64_t *prompt, size_t nprompt,
                                         size_t max_new_tokens, int64_t eos);
    /* One model step; returns the number of unfinished requests. */
    __export int64_t llaisysSchedulerStep(struct LlaisysScheduler * s);
    /* llaisysRequestStatus_t of a request, -1 if unknown. */
    __export int llaisysSchedulerStatus(struct LlaisysScheduler * s, int64_t request);
    /* Tokens generated so far (the first min(count, capacity) copied to out,
     * which may be NULL); returns the count. */
    __export int64_t llaisysSchedulerTokens(struct LlaisysScheduler * s, int64_t request, int64_t *out,
                                            size_t capacity);
    /* Forget a finished request. */
    __export int llaisysSchedulerRelease(struct LlaisysScheduler * s, int64_t request);
    /* out[5] = steps, preemptions, prefill tokens, decode tokens, finished requests. */
    __export int llaisysSchedulerStats(struct LlaisysScheduler * s, int64_t *out);
}

#endif // LLAISYS_SERVING_H
