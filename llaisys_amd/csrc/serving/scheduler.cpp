#include "scheduler.hpp"

#include "../common.hpp"

#include <algorithm>

namespace llaisys::serving {

using kvcache::kBlockTokens;

Scheduler::Scheduler(Backend &backend, const SchedulerConfig &cfg) : be_(backend), cfg_(cfg) {
    LLAISYS_CHECK(cfg.max_seqs >= 1 && cfg.max_step_tokens >= 1 && cfg.prefill_chunk >= 1,
                  "scheduler: max_seqs, max_step_tokens and prefill_chunk must be >= 1");
}

Scheduler::~Scheduler() {
    for (int64_t id : active_) {
        try {
            be_.seqFree(reqs_.at(id).seq);
        } catch (...) {
        }
    }
}

int64_t Scheduler::add(const int64_t *prompt, size_t nprompt, size_t max_new_tokens, int64_t eos) {
    LLAISYS_CHECK(prompt && nprompt >= 1, "scheduler: a request needs at least one prompt token");
    LLAISYS_CHECK(max_new_tokens >= 1, "scheduler: max_new_tokens must be >= 1");
    LLAISYS_CHECK(nprompt <= be_.maxSeqLen(),
                  "scheduler: prompt of " << nprompt << " tokens exceeds the model's " << be_.maxSeqLen());
    const int64_t id = next_req_++;
    Request &r = reqs_[id];
    r.prompt.assign(prompt, prompt + nprompt);
    r.input = r.prompt;
    r.max_new = max_new_tokens;
    r.eos = eos;
    waiting_.push_back(id);
    ++unfinished_;
    return id;
}

const Scheduler::Request &Scheduler::get(int64_t req) const {
    auto it = reqs_.find(req);
    LLAISYS_CHECK(it != reqs_.end(), "scheduler: unknown request " << req);
    return it->second;
}

bool Scheduler::finished(int64_t req) const { return get(req).state == State::Finished; }
FinishReason Scheduler::reason(int64_t req) const { return get(req).why; }
const std::vector<int64_t> &Scheduler::generated(int64_t req) const { return get(req).out; }

void Scheduler::release(int64_t req) {
    LLAISYS_CHECK(finished(req), "scheduler: request " << req << " is not finished");
    reqs_.erase(req);
}

int64_t Scheduler::blocksFor(size_t len, size_t extra) {
    const size_t b = size_t(kBlockTokens);
    return int64_t((len + extra + b - 1) / b - (len + b - 1) / b);
}

void Scheduler::preempt(int64_t id) {
    Request &r = reqs_.at(id);
    be_.seqFree(r.seq);
    r.seq = -1;
    r.input = r.prompt;
    r.input.insert(r.input.end(), r.out.begin(), r.out.end());
    r.cached = 0;
    r.state = State::Waiting;
    active_.erase(std::find(active_.begin(), active_.end(), id));
    waiting_.push_front(id);
    ++stats_.preemptions;
}

void Scheduler::finish(Request &r, FinishReason why) {
    if (r.seq >= 0) {
        be_.seqFree(r.seq);
        r.seq = -1;
    }
    for (auto it = active_.begin(); it != active_.end(); ++it) {
        if (&reqs_.at(*it) == &r) {
            active_.erase(it);
            break;
        }
    }
    r.state = State::Finished;
    r.why = why;
    r.input.clear();
    --unfinished_;
    ++stats_.finished;
}

bool Scheduler::stopAfter(Request &r, int64_t token) {
    r.out.push_back(token);
    if (r.out.size() >= r.max_new) {
        finish(r, FinishReason::MaxTokens);
    } else if (r.eos >= 0 && token == r.eos) {
        finish(r, FinishReason::Eos);
    } else if (r.cached + 1 > be_.maxSeqLen()) {
        finish(r, FinishReason::Length); // no slot left for the token to decode
    } else {
        return false;
    }
    return true;
}

size_t Scheduler::step() {
    if (active_.empty() && waiting_.empty()) return unfinished_;
    struct Chunk {
        int64_t req;
        size_t n;
    };
    std::vector<int64_t> decodes;
    std::vector<Chunk> prefills;
    for (;;) {
        decodes.clear();
        prefills.clear();
        // 1. One token for every running request; preempt the latest admitted
        //    requests until the pool holds the pages these decodes open.
        int64_t need = 0;
        for (int64_t id : active_) {
            const Request &r = reqs_.at(id);
            if (r.state != State::Running) continue;
            decodes.push_back(id);
            need += blocksFor(r.cached, 1);
        }
        int64_t avail = be_.numFreeBlocks();
        while (need > avail && !active_.empty()) {
            const int64_t victim = active_.back();
            const Request &v = reqs_.at(victim);
            if (v.state == State::Running) {
                need -= blocksFor(v.cached, 1);
                decodes.erase(std::find(decodes.begin(), decodes.end(), victim));
            }
            preempt(victim);
            avail = be_.numFreeBlocks();
        }
        avail -= need;
        size_t budget = cfg_.max_step_tokens > decodes.size() ? cfg_.max_step_tokens - decodes.size() : 0;

        // Largest chunk of r's input (<= want tokens) whose pages fit in avail.
        auto fit = [&](const Request &r, size_t want) {
            const size_t b = size_t(kBlockTokens);
            const size_t room = ((r.cached + b - 1) / b + size_t(std::max<int64_t>(avail, 0))) * b - r.cached;
            return std::min(want, room);
        };
        // 2. Prefill chunks of admitted requests, in admission order.
        for (int64_t id : active_) {
            if (budget == 0) break;
            const Request &r = reqs_.at(id);
            if (r.state != State::Prefill) continue;
            const size_t c = fit(r, std::min({r.input.size() - r.cached, cfg_.prefill_chunk, budget}));
            if (c == 0) continue;
            prefills.push_back({id, c});
            budget -= c;
            avail -= blocksFor(r.cached, c);
        }
        // 3. Admit waiting requests while slots, budget and pages allow.
        while (budget > 0 && active_.size() < cfg_.max_seqs && !waiting_.empty()) {
            const int64_t id = waiting_.front();
            Request &r = reqs_.at(id);
            const int64_t before = be_.numFreeBlocks();
            size_t reused = 0;
            const int64_t seq = be_.seqCreate(r.input.data(), r.input.size(), &reused);
            avail -= before - be_.numFreeBlocks(); // cached blocks taken off the reclaimable list
            r.seq = seq;
            r.cached = reused;
            const size_t c = fit(r, std::min({r.input.size() - r.cached, cfg_.prefill_chunk, budget}));
            if (c == 0) {
                be_.seqFree(seq);
                r.seq = -1;
                r.cached = 0;
                break;
            }
            waiting_.pop_front();
            r.state = State::Prefill;
            r.admitted = ++stamp_;
            active_.push_back(id);
            prefills.push_back({id, c});
            budget -= c;
            avail -= blocksFor(r.cached, c);
        }
        if (!decodes.empty() || !prefills.empty()) break;
        // Nothing can run: prefills stalled on pages. Free the latest admitted
        // request's pages for the others; a lone request the pool cannot hold
        // ends with NoCapacity.
        if (active_.size() > 1) {
            preempt(active_.back());
            continue;
        }
        if (active_.size() == 1) {
            finish(reqs_.at(active_.front()), FinishReason::NoCapacity);
            continue;
        }
        if (!waiting_.empty()) {
            finish(reqs_.at(waiting_.front()), FinishReason::NoCapacity);
            waiting_.pop_front();
            if (active_.empty() && waiting_.empty()) return unfinished_;
            continue;
        }
        return unfinished_;
    }

    // 4. One backend step: decodes first, then prefill chunks.
    std::vector<int64_t> ids, toks, next;
    std::vector<size_t> ntok;
    for (int64_t id : decodes) {
        const Request &r = reqs_.at(id);
        ids.push_back(r.seq);
        ntok.push_back(1);
        toks.push_back(r.out.back());
    }
    for (const Chunk &c : prefills) {
        const Request &r = reqs_.at(c.req);
        ids.push_back(r.seq);
        ntok.push_back(c.n);
        toks.insert(toks.end(), r.input.begin() + std::ptrdiff_t(r.cached),
                    r.input.begin() + std::ptrdiff_t(r.cached + c.n));
    }
    next.assign(ids.size(), -1);
    be_.step(ids.data(), ids.size(), toks.data(), ntok.data(), next.data());
    ++stats_.steps;

    // 5. Results: decodes emit a token; a prefill that consumed the last input
    //    token emits the request's next token and starts decoding.
    size_t i = 0;
    for (int64_t id : decodes) {
        Request &r = reqs_.at(id);
        r.cached += 1;
        ++stats_.decode_tokens;
        stopAfter(r, next[i++]);
    }
    for (const Chunk &c : prefills) {
        Request &r = reqs_.at(c.req);
        r.cached += c.n;
        stats_.prefill_tokens += int64_t(c.n);
        const int64_t tok = next[i++];
        if (r.cached == r.input.size()) {
            r.state = State::Running;
            stopAfter(r, tok);
        }
    }
    return unfinished_;
}

// ---------------------------------------------------------------- SimBackend

SimBackend::SimBackend(int num_blocks, int64_t vocab, size_t max_seq_len)
    : blocks_(num_blocks), vocab_(vocab), max_len_(max_seq_len) {
    LLAISYS_CHECK(vocab >= 1 && max_seq_len >= 1, "sim backend: vocab and max_seq_len must be >= 1");
}

int64_t SimBackend::seqCreate(const int64_t *tokens, size_t ntokens, size_t *reused) {
    const int64_t id = next_id_++;
    const int r = blocks_.create(id, tokens, tokens ? ntokens : 0);
    hist_[id].assign(tokens, tokens + r);
    if (reused) *reused = size_t(r);
    return id;
}

void SimBackend::seqFree(int64_t id) {
    blocks_.release(id);
    hist_.erase(id);
}

int64_t SimBackend::greedy(const int64_t *history, size_t n, int64_t vocab) {
    uint64_t h = 14695981039346656037ull;
    for (size_t i = 0; i < n; ++i) {
        h ^= uint64_t(history[i]);
        h *= 1099511628211ull;
    }
    return int64_t(h % uint64_t(vocab));
}

void SimBackend::step(const int64_t *ids, size_t nseq, const int64_t *tokens, const size_t *ntokens, int64_t *next) {
    LLAISYS_CHECK(nseq > 0 && ids && tokens && ntokens && next, "sim backend: empty or null step");
    for (size_t i = 0; i < nseq; ++i) {
        LLAISYS_CHECK(ntokens[i] >= 1, "sim backend: sequence " << ids[i] << " appends no token");
        LLAISYS_CHECK(hist_.count(ids[i]), "sim backend: unknown sequence " << ids[i]);
        for (size_t j = 0; j < i; ++j) LLAISYS_CHECK(ids[j] != ids[i], "sim backend: sequence repeated in a step");
        LLAISYS_CHECK(hist_[ids[i]].size() + ntokens[i] <= max_len_, "sim backend: sequence past max_seq_len");
    }
    int32_t cow[2];
    for (size_t i = 0; i < nseq; ++i) blocks_.reserve(ids[i], int(ntokens[i]), cow, 1);
    size_t off = 0, total = 0;
    for (size_t i = 0; i < nseq; ++i) {
        blocks_.commit(ids[i], int(ntokens[i]), tokens + off);
        auto &h = hist_[ids[i]];
        h.insert(h.end(), tokens + off, tokens + off + ntokens[i]);
        next[i] = greedy(h.data(), h.size(), vocab_);
        off += ntokens[i];
        total += ntokens[i];
    }
    ++steps_;
    max_tokens_ = std::max<int64_t>(max_tokens_, int64_t(total));
}

} // namespace llaisys::serving
