// Qwen2 decoder on the paged KV path (reference API: include/llaisys/models/
// qwen2.h:7-40; the reference leaves the model unimplemented,
// python/llaisys/models/qwen2.py:9-33).
//
// Layout choices:
//  * q/k/v projections live in one fused [(nh + 2 nkvh) dh, hs] matrix and
//    gate/up in one [2 di, hs] matrix; the reference's per-projection weight
//    tensors are row slices of these, so loading them fills the fused ones and
//    each layer runs one QKV GEMM and one gate-up GEMM;
//  * the K/V cache is one paged pool pair per layer ([blocks, nkvh, 16, dh]
//    bf16, the MI355X page format), shared by every sequence through a
//    BlockManager (prefix cache, forks, copy-on-write);
//  * a step is a varlen batch: each sequence appends n_i >= 1 tokens (prefill
//    chunks and single-token decodes mix freely), and the LM head runs on each
//    sequence's last position only.
#pragma once

#include "../kvcache/block_manager.hpp"
#include "../tensor/tensor.hpp"

#include <cstdint>
#include <functional>
#include <map>
#include <vector>

namespace llaisys::models {

struct Qwen2Config {
    llaisysDataType_t dtype;
    size_t nlayer, hs, nh, nkvh, dh, di, maxseq, voc;
    float epsilon, theta;
    int64_t end_token;
};

struct Qwen2LayerWeights {
    tensor_t attn_norm, qkv_w, qkv_b, o_w, mlp_norm, gate_up_w, down_w;
    // reference-named slices of the fused tensors
    tensor_t q_w, k_w, v_w, q_b, k_b, v_b, gate_w, up_w;
    // qkv_w and gate_up_w with the preceding RMSNorm weight folded into their
    // columns (W diag(w)), and the write versions of (qkv_w, attn_norm,
    // gate_up_w, mlp_norm) they were folded from
    tensor_t qkv_wf, gate_up_wf;
    uint64_t folded_from[4] = {~0ull, ~0ull, ~0ull, ~0ull};
    // The decode GEMM's packed copies (MFMA operand order) of the folded QKV
    // and gate-up weights, of o_w and of down_w (split-K kernel); null when
    // the shapes do not qualify.
    tensor_t qkv_wfp, gate_up_wfp, o_wp, down_wp;
    uint64_t o_packed_from = ~0ull, down_packed_from = ~0ull;
    // gate_up_w in linearSwiglu's row order (gate and up blocks of 16 rows in
    // turn) for the long steps' one-launch gate-up + SwiGLU; null when off.
    tensor_t gate_up_wi;
    uint64_t interleaved_from = ~0ull;
};

class Qwen2Model {
public:
    Qwen2Model(const Qwen2Config &cfg, int device_id, size_t num_blocks);
    ~Qwen2Model();

    const Qwen2Config &config() const { return cfg_; }
    tensor_t inEmbed() const { return in_embed_; }
    tensor_t outEmbed() const { return out_embed_; }
    tensor_t outNorm() const { return out_norm_; }
    const Qwen2LayerWeights &layer(size_t i) const { return layers_.at(i); }

    // The reference's single-sequence Infer: token_ids is the whole token
    // history. The KV cache of the previous call is kept when it is a prefix
    // of token_ids (only the new tokens are computed); otherwise the sequence
    // restarts, reusing cached full blocks of a matching prefix.
    int64_t infer(const int64_t *token_ids, size_t ntoken);

    // Sequences of the batched API. create() maps the cached prefix of tokens
    // (may be null) and returns how many leading tokens it already covers.
    int64_t seqCreate(const int64_t *tokens, size_t ntokens, size_t *reused);
    int64_t seqFork(int64_t parent);
    void seqFree(int64_t id);
    size_t seqLength(int64_t id) const;
    size_t numFreeBlocks() const { return size_t(blocks_.numFree()); }

    // One step: sequence ids[i] appends ntokens[i] >= 1 tokens (concatenated
    // in tokens); next[i] is the argmax of the logits at its last position.
    void step(const int64_t *ids, size_t nseq, const int64_t *tokens, const size_t *ntokens, int64_t *next);

    // nsteps greedy single-token steps of the batch with the next token fed
    // back on the device: sequence ids[i] appends first[i], then its own
    // greedy tokens; out[s * nseq + i] = the greedy token after step s.
    void decode(const int64_t *ids, size_t nseq, const int64_t *first, size_t nsteps, int64_t *out);

    // Logits [nseq, voc] of the last step (a view of the step workspace).
    tensor_t lastLogits() const;

private:
    void ensureWorkspace(size_t T, size_t B, size_t ints32, size_t ints64);
    void forward(size_t T, size_t B, bool decode_only);
    // Refold each layer whose projection or norm weights were written since
    // their folded copies were made (a check of version counters per step).
    void ensureFolded();
    // Y[M, N] (+)= X W^T: the hand-written decode GEMM over `packed` when it
    // exists and M is at most the size where it wins for this N, else the
    // general MFMA GEMM (linear) over the row-major `w`. y_packed: also write Y in
    // operand order (only the split-K path can; the caller checks it is taken).
    void project(const tensor_t &y, const tensor_t &x, const tensor_t &w, const tensor_t &packed, int M, int N, int K,
                 bool accumulate, void *s, uint16_t *y_packed = nullptr) const;
    void decodeGraph(size_t B, size_t width);
    std::vector<int32_t> reserveAll(const int64_t *ids, size_t B, const size_t *n, std::vector<int32_t> &before);

    Qwen2Config cfg_;
    int dev_;
    size_t num_blocks_;
    kvcache::BlockManager blocks_;
    int64_t next_id_ = 1;
    std::vector<int64_t> hist0_; // token history of the Infer sequence (id 0)
    bool have0_ = false;

    tensor_t in_embed_, out_embed_, out_norm_;
    tensor_t out_embed_p_; // packed LM head for the decode GEMM (null when the shape does not qualify)
    uint64_t out_embed_packed_from_ = ~0ull;
    bool decode_gemm_ = true; // LLAISYS_DECODE_GEMM=0: the general GEMM only
    std::vector<Qwen2LayerWeights> layers_;
    std::vector<tensor_t> k_pool_, v_pool_;

    // step workspace (grow-only)
    size_t cap_T_ = 0, cap_B_ = 0, cap_i32_ = 0, cap_i64_ = 0;
    tensor_t x_, h_, qkv_, q_, attn_, gu_, act_, hl_, logits_, next_;
    // x and the attention output in MFMA operand order (packedRowIndex), for
    // the packed-operand qkv and o projections of decode steps.
    tensor_t xp_, ap_, actp_; // actp_: the SwiGLU output, for the packed-X down projection
    tensor_t dev_i32_, dev_i64_;     // per-step indices, uploaded in one copy each
    core::storage_t host32_, host64_; // pinned staging of the same
    tensor_t table_, ctx_before_, ctx_after_, cu_, cow_, tok_, last_; // views of dev_i32_/dev_i64_
    size_t last_B_ = 0;

    // Captured decode steps per batch size (LLAISYS_QWEN2_GRAPHS=0 disables).
    struct DecodeGraph {
        void *exec = nullptr; // hipGraphExec_t
        size_t width = 0;     // block-table width it was captured with
        uint64_t gen = 0;     // workspace generation it was captured with
        uint64_t ws = 0; // runtime workspace generation it was captured with
        bool unit = false; // captured with the one-workgroup-per-unit decode attention
    };
    DecodeGraph capture(const std::function<void()> &work, size_t width);
    bool use_graphs_ = true;
    bool fold_norm_ = true; // LLAISYS_QWEN2_FOLD_NORM=0: separate rms_norm launches instead
    // Decode steps whose contexts are within 2x of each other, with at least
    // kUnitDecodeMinUnits (sequence, kv head) units, run the decode attention
    // with one workgroup per unit (no split records, one launch).
    // LLAISYS_DECODE_UNITS=0 keeps the stream-K kernel for every step.
    bool unit_decode_allowed_ = true;
    bool unit_decode_ = false; // the choice for the step being built
    // With the unit attention, the QKV epilogue runs inside it
    // (pagedDecodeUnitsRope) when the head grouping allows;
    // LLAISYS_DECODE_UNIT_ROPE=0 keeps the separate qkvRopeAppend launch.
    bool unit_rope_ = true;
    // Decode steps on that path (M <= 128, K = 1536) run the qkv and o
    // projections with both operands packed: the embedding, the split-K
    // reduce and the attention write packed copies of their rows.
    // LLAISYS_PACKED_X=0 keeps row-major X there (project()).
    bool packed_x_ = true;
    // On that path the QKV epilogue (bias, 1/rms, RoPE, k/v append) runs in
    // the QKV projection's epilogue, and the attention reads q
    // (LLAISYS_QKV_GEMM_EPILOGUE=0: in the attention kernel instead).
    bool qkv_gemm_epilogue_ = true;
    // On that path the down projection's split-K reads the SwiGLU output
    // packed, streamed through registers (fewer splits than the LDS-staged
    // split-K); LLAISYS_SPLITK_PACKED=0 keeps the LDS-staged kernel.
    bool splitk_packed_ = true;
    // Steps whose gate-up runs the general GEMM: the SwiGLU in its epilogue
    // over gate_up_wi (LLAISYS_GEMM_SWIGLU=0: the GEMM, then swigluRows).
    bool gemm_swiglu_ = true;
    void chooseDecodeAttention(size_t B, int32_t min_ctx, int32_t max_ctx);
    uint64_t ws_gen_ = 0;     // bumped whenever a step workspace buffer moves
    std::map<size_t, DecodeGraph> graphs_;       // one step (step())
    std::map<size_t, DecodeGraph> multi_graphs_; // advance + step + record (decode())
};

} // namespace llaisys::models
