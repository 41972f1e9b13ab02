#ifndef LLAISYS_MODELS_QWEN2_H
#define LLAISYS_MODELS_QWEN2_H

#include "../tensor.h"

/*
 * Qwen2 decoder on the paged KV path (reference: include/llaisys/models/
 * qwen2.h:7-40, whose declarations the first four functions keep).
 *
 * Device: LLAISYS_DEVICE_AMD, one device (device_ids[0]); meta.dtype must be
 * LLAISYS_DTYPE_BF16 and meta.dh 128 (the page format's head dim).
 *
 * Weights: llaisysQwen2ModelWeights returns tensors the model owns; load each
 * with tensorLoad (the handles stay valid until Destroy). attn_{q,k,v}_{w,b}
 * are row slices of one fused QKV matrix per layer and mlp_{gate,up}_w of one
 * fused gate-up matrix. A handle the caller replaces with its own tensor of
 * the same shape and dtype is copied in at the next Infer/Step.
 *
 * KV cache: a pool of 16-token blocks per layer shared by all sequences, with
 * a prefix cache of full blocks keyed by their token ids.
 *
 * A model is driven from one thread at a time (its calls are not reentrant);
 * work runs on that thread's context stream (llaisysGetContextStream).
 */
__C {
    struct LlaisysQwen2Meta {
        llaisysDataType_t dtype;
        size_t nlayer, hs, nh, nkvh, dh, di, maxseq, voc;
        float epsilon, theta;
        int64_t end_token;
    };

    struct LlaisysQwen2Weights {
        llaisysTensor_t in_embed;
        llaisysTensor_t out_embed;
        llaisysTensor_t out_norm_w;   // a.k.a. model.norm.weight
        llaisysTensor_t *attn_norm_w; // a.k.a. input_layernorm.weight
        llaisysTensor_t *attn_q_w;
        llaisysTensor_t *attn_q_b;
        llaisysTensor_t *attn_k_w;
        llaisysTensor_t *attn_k_b;
        llaisysTensor_t *attn_v_w;
        llaisysTensor_t *attn_v_b;
        llaisysTensor_t *attn_o_w;
        llaisysTensor_t *mlp_norm_w; // a.k.a. post_attention_layernorm.weight
        llaisysTensor_t *mlp_gate_w;
        llaisysTensor_t *mlp_up_w;
        llaisysTensor_t *mlp_down_w;
    };

    struct LlaisysQwen2Model;

    /* qwen2.h:33. KV pool of ceil(maxseq / 16) + 1 blocks (one sequence).
     * NULL on failure (llaisysGetLastError has the message). */
    __export struct LlaisysQwen2Model *llaisysQwen2ModelCreate(const LlaisysQwen2Meta *meta, llaisysDeviceType_t device, int *device_ids, int ndevice);

    /* qwen2.h:35 */
    __export void llaisysQwen2ModelDestroy(struct LlaisysQwen2Model * model);

    /* qwen2.h:37 */
    __export struct LlaisysQwen2Weights *llaisysQwen2ModelWeights(struct LlaisysQwen2Model * model);

    /* qwen2.h:39. token_ids is the whole history of the conversation; returns
     * the greedy next token (-1 on failure). The KV cache of the previous call
     * is reused when its tokens are a prefix of token_ids, so a generate loop
     * that passes history + [next] computes one token per call. */
    __export int64_t llaisysQwen2ModelInfer(struct LlaisysQwen2Model * model, int64_t * token_ids, size_t ntoken);

    /* ---- Batched serving (no reference counterpart: README.md:421-424 asks
     * for continuous batching over a KV-cache pool with prefix matching). */

    /* As Create, with a KV pool of num_blocks blocks per layer. */
    __export struct LlaisysQwen2Model *llaisysQwen2ModelCreatePaged(const LlaisysQwen2Meta *meta, llaisysDeviceType_t device, int *device_ids, int ndevice, size_t num_blocks);

    /* New sequence (id > 0). If tokens != NULL, cached blocks holding a prefix
     * of tokens are mapped and *reused (may be NULL) receives how many leading
     * tokens need no recomputation. -1 on failure. */
    __export int64_t llaisysQwen2SeqCreate(struct LlaisysQwen2Model * model, const int64_t *tokens, size_t ntokens, size_t *reused);
    /* New sequence sharing all of parent's cached tokens (copy-on-write). */
    __export int64_t llaisysQwen2SeqFork(struct LlaisysQwen2Model * model, int64_t parent);
    __export int llaisysQwen2SeqFree(struct LlaisysQwen2Model * model, int64_t seq_id);
    /* Tokens in the sequence's KV cache; -1 if unknown. */
    __export int64_t llaisysQwen2SeqLength(struct LlaisysQwen2Model * model, int64_t seq_id);
    __export int64_t llaisysQwen2NumFreeBlocks(struct LlaisysQwen2Model * model);

    /* One step over nseq distinct sequences: sequence seq_ids[i] appends
     * ntokens[i] >= 1 tokens (all concatenated in token_ids: prefill chunks and
     * single-token decodes mix). next_tokens[i] receives the greedy token after
     * the sequence's last position. Returns 0, or -1 on failure. */
    __export int llaisysQwen2ModelStep(struct LlaisysQwen2Model * model, const int64_t *seq_ids, size_t nseq, const int64_t *token_ids, const size_t *ntokens, int64_t *next_tokens);

    /* nsteps greedy decode steps of nseq distinct sequences in one call, the
     * next token fed back on the device (no host round trip between steps):
     * sequence seq_ids[i] appends first_tokens[i], then its own greedy tokens.
     * out_tokens[s * nseq + i] receives the greedy token after step s. Same
     * results as nsteps calls of llaisysQwen2ModelStep. Returns 0, or -1. */
    __export int llaisysQwen2ModelDecode(struct LlaisysQwen2Model * model, const int64_t *seq_ids, size_t nseq, const int64_t *first_tokens, size_t nsteps, int64_t *out_tokens);

    /* Logits [nseq, voc] (meta.dtype) of the last Infer/Step/Decode step: a new handle the
     * caller destroys; its contents change at the next call. */
    __export llaisysTensor_t llaisysQwen2ModelLogits(struct LlaisysQwen2Model * model);
}
#endif // LLAISYS_MODELS_QWEN2_H
