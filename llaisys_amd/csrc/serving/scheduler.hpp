// Continuous-batching scheduler over a paged-KV model.
//
// Requests (prompt, max_new_tokens, eos) queue up; every step() builds one
// mixed batch for the backend: a single-token decode for each running request
// first, then prefill chunks of admitted requests (at most prefill_chunk
// tokens each, max_step_tokens in total), admitting waiting requests in
// arrival order while sequence slots, token budget and KV blocks allow. A
// request's first generated token comes from the step that consumes the last
// token of its prompt. When the KV pool cannot hold the next decodes, the
// most recently admitted requests are preempted: their sequences are freed
// and they re-enter the queue with prompt + generated tokens as the new input
// (recomputed later, cached full blocks reused). Greedy decoding is a function
// of each request's own history, so batching, chunking and preemption never
// change a request's tokens.
//
// The README of the reference asks for this component (README.md:421-424:
// continuous batching over a KV-cache pool with prefix matching); it has no
// code to follow.
#pragma once

#include "../kvcache/block_manager.hpp"

#include <cstddef>
#include <cstdint>
#include <deque>
#include <map>
#include <memory>
#include <unordered_map>
#include <vector>

namespace llaisys::serving {

// What the scheduler needs from a model (paged KV sequences, one mixed step).
class Backend {
public:
    virtual ~Backend() = default;
    // New sequence mapping the cached prefix of tokens; *reused = tokens it covers.
    virtual int64_t seqCreate(const int64_t *tokens, size_t ntokens, size_t *reused) = 0;
    virtual void seqFree(int64_t id) = 0;
    virtual int64_t numFreeBlocks() = 0;
    virtual size_t maxSeqLen() = 0; // tokens a sequence may hold
    // Sequence ids[i] appends ntokens[i] tokens (concatenated); next[i] = greedy token.
    virtual void step(const int64_t *ids, size_t nseq, const int64_t *tokens, const size_t *ntokens,
                      int64_t *next) = 0;
};

struct SchedulerConfig {
    size_t max_seqs = 64;          // requests holding a sequence at once
    size_t max_step_tokens = 2048; // tokens per step (decodes + prefill chunks)
    size_t prefill_chunk = 512;    // prompt tokens of one request per step
};

struct SchedulerStats {
    int64_t steps = 0, preemptions = 0, prefill_tokens = 0, decode_tokens = 0, finished = 0;
};

// NoCapacity: the KV pool cannot hold the request even with every other one preempted.
enum class FinishReason : int { None = 0, MaxTokens = 1, Eos = 2, Length = 3, NoCapacity = 4 };

class Scheduler {
public:
    Scheduler(Backend &backend, const SchedulerConfig &cfg);
    ~Scheduler(); // frees the sequences still held
    Scheduler(const Scheduler &) = delete;
    Scheduler &operator=(const Scheduler &) = delete;

    // Queue a request; returns its id (>= 0). eos < 0: no end token.
    int64_t add(const int64_t *prompt, size_t nprompt, size_t max_new_tokens, int64_t eos);
    // One backend step (nothing when idle); returns the number of unfinished requests.
    size_t step();
    size_t unfinished() const { return unfinished_; }

    bool known(int64_t req) const { return reqs_.count(req) != 0; }
    bool finished(int64_t req) const;
    FinishReason reason(int64_t req) const;
    const std::vector<int64_t> &generated(int64_t req) const;
    void release(int64_t req); // forget a finished request
    const SchedulerStats &stats() const { return stats_; }

private:
    enum class State { Waiting, Prefill, Running, Finished };
    struct Request {
        std::vector<int64_t> prompt, out;
        std::vector<int64_t> input; // tokens the sequence must hold before the next decode
        size_t max_new = 0;
        int64_t eos = -1;
        State state = State::Waiting;
        FinishReason why = FinishReason::None;
        int64_t seq = -1;
        size_t cached = 0;     // tokens of input in the sequence's KV cache
        uint64_t admitted = 0; // admission stamp (preemption picks the latest)
    };

    const Request &get(int64_t req) const;
    static int64_t blocksFor(size_t len, size_t extra);
    void preempt(int64_t req);
    void finish(Request &r, FinishReason why);
    bool stopAfter(Request &r, int64_t token); // true if r finished after emitting token

    Backend &be_;
    SchedulerConfig cfg_;
    std::map<int64_t, Request> reqs_;
    std::deque<int64_t> waiting_;  // arrival order (preempted requests go back to the front)
    std::vector<int64_t> active_;  // holding a sequence, admission order
    int64_t next_req_ = 0;
    uint64_t stamp_ = 0;
    size_t unfinished_ = 0;
    SchedulerStats stats_;
};

// Host-only stand-in for a model, for testing schedulers without a GPU: a
// real BlockManager pool, and a "greedy token" that is a hash of the
// sequence's whole token history (FNV-1a over the int64 values, modulo
// vocab), so any lost, repeated or reordered token changes every later one.
class SimBackend : public Backend {
public:
    SimBackend(int num_blocks, int64_t vocab, size_t max_seq_len);
    int64_t seqCreate(const int64_t *tokens, size_t ntokens, size_t *reused) override;
    void seqFree(int64_t id) override;
    int64_t numFreeBlocks() override { return blocks_.numFree(); }
    size_t maxSeqLen() override { return max_len_; }
    void step(const int64_t *ids, size_t nseq, const int64_t *tokens, const size_t *ntokens, int64_t *next) override;
    int64_t stepsRun() const { return steps_; }
    int64_t maxBatchTokens() const { return max_tokens_; }

    static int64_t greedy(const int64_t *history, size_t n, int64_t vocab);

private:
    kvcache::BlockManager blocks_;
    int64_t vocab_;
    size_t max_len_;
    int64_t next_id_ = 1;
    std::unordered_map<int64_t, std::vector<int64_t>> hist_;
    int64_t steps_ = 0, max_tokens_ = 0;
};

} // namespace llaisys::serving
