#include "block_manager.hpp"

#include "../common.hpp"

#include <algorithm>
#include <cstring>

namespace llaisys::kvcache {

namespace {
// splitmix64 finaliser: a well-mixed 64-bit permutation.
uint64_t mix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
} // namespace

BlockManager::BlockManager(int num_blocks, bool scatter) {
    LLAISYS_CHECK(num_blocks > 0, "kv block manager: num_blocks must be positive, got " << num_blocks);
    ref_.assign(num_blocks, 0);
    lru_pos_.resize(num_blocks);
    in_lru_.assign(num_blocks, false);
    hash_of_.assign(num_blocks, 0);
    cached_.assign(num_blocks, false);
    cached_data_.resize(num_blocks);
    free_.reserve(num_blocks);
    // The stack hands out free_.back() first: block order[0], order[1], ...
    // Scattered order: i * stride mod n, stride ~ 0.618 n and coprime to n (a
    // permutation that puts consecutive allocations far apart).
    int64_t stride = 1;
    if (scatter && num_blocks > 2) {
        stride = int64_t(double(num_blocks) * 0.6180339887) | 1;
        auto gcd = [](int64_t a, int64_t b) {
            while (b) {
                const int64_t t = a % b;
                a = b;
                b = t;
            }
            return a;
        };
        while (gcd(stride, num_blocks) != 1) stride += 2;
    }
    for (int64_t i = num_blocks - 1; i >= 0; --i) free_.push_back(int((i * stride) % num_blocks));
}

uint64_t BlockManager::chainHash(uint64_t parent, const int64_t *tokens) {
    uint64_t h = mix(parent ^ 0x6C6C61697379ull);
    for (int i = 0; i < kBlockTokens; ++i) h = mix(h ^ uint64_t(tokens[i]));
    return h;
}

const BlockManager::Seq &BlockManager::seq(int64_t id) const {
    auto it = seqs_.find(id);
    LLAISYS_CHECK(it != seqs_.end(), "kv block manager: unknown sequence " << id);
    return it->second;
}

BlockManager::Seq &BlockManager::seq(int64_t id) {
    auto it = seqs_.find(id);
    LLAISYS_CHECK(it != seqs_.end(), "kv block manager: unknown sequence " << id);
    return it->second;
}

// A free block: uncached ones first, else the least recently released cached
// one (dropping its prefix entry).
int BlockManager::allocate() {
    int b;
    if (!free_.empty()) {
        b = free_.back();
        free_.pop_back();
    } else {
        LLAISYS_CHECK(!lru_.empty(), "kv block manager: out of blocks");
        b = lru_.front();
        lru_.pop_front();
        in_lru_[b] = false;
        prefix_.erase(hash_of_[b]);
        cached_[b] = false;
    }
    ref_[b] = 1;
    return b;
}

void BlockManager::unref(int b) {
    if (--ref_[b] > 0) return;
    if (cached_[b]) {
        lru_pos_[b] = lru_.insert(lru_.end(), b);
        in_lru_[b] = true;
    } else {
        free_.push_back(b);
    }
}

void BlockManager::cacheFullBlock(Seq &s, int block, const int64_t *tokens) {
    const uint64_t h = chainHash(s.chain, tokens);
    if (!cached_[block] && !prefix_.count(h)) {
        prefix_[h] = block;
        hash_of_[block] = h;
        cached_[block] = true;
        cached_data_[block].parent = s.chain;
        std::memcpy(cached_data_[block].tokens.data(), tokens, sizeof(int64_t) * kBlockTokens);
    }
    s.chain = h;
}

int BlockManager::create(int64_t id, const int64_t *tokens, size_t ntokens) {
    LLAISYS_CHECK(!seqs_.count(id), "kv block manager: sequence " << id << " already exists");
    Seq s;
    // Reuse whole cached blocks, but leave at least one prompt token to compute.
    const size_t usable = ntokens ? (ntokens - 1) / kBlockTokens : 0;
    for (size_t k = 0; tokens && k < usable; ++k) {
        const int64_t *blk = tokens + k * kBlockTokens;
        auto it = prefix_.find(chainHash(s.chain, blk));
        if (it == prefix_.end()) break;
        const int b = it->second;
        const CachedBlock &c = cached_data_[b];
        if (c.parent != s.chain || std::memcmp(c.tokens.data(), blk, sizeof(int64_t) * kBlockTokens) != 0) break;
        if (in_lru_[b]) {
            lru_.erase(lru_pos_[b]);
            in_lru_[b] = false;
        }
        ++ref_[b];
        s.blocks.push_back(b);
        s.chain = hash_of_[b];
        s.len += kBlockTokens;
    }
    const int hit = s.len;
    seqs_.emplace(id, std::move(s));
    return hit;
}

void BlockManager::fork(int64_t parent, int64_t child) {
    LLAISYS_CHECK(!seqs_.count(child), "kv block manager: sequence " << child << " already exists");
    Seq copy = seq(parent);
    for (int b : copy.blocks) ++ref_[b];
    seqs_.emplace(child, std::move(copy));
}

int BlockManager::reserve(int64_t id, int ntokens, int32_t *cow, int cow_capacity) {
    LLAISYS_CHECK(ntokens >= 0, "kv block manager: negative token count");
    Seq &s = seq(id);
    const int have = int(s.blocks.size());
    const int need = (s.len + ntokens + kBlockTokens - 1) / kBlockTokens;
    const int fresh = std::max(0, need - have);
    // The partial last block gets written: it must be private.
    const bool partial = s.len % kBlockTokens != 0 && ntokens > 0;
    const bool copy = partial && ref_[s.blocks.back()] > 1;
    LLAISYS_CHECK(!copy || (cow && cow_capacity >= 1),
                  "kv block manager: sequence " << id << " needs a copy-on-write pair but no room was given");
    LLAISYS_CHECK(fresh + (copy ? 1 : 0) <= numFree(), "kv block manager: out of blocks (need "
                                                          << fresh + (copy ? 1 : 0) << ", free " << numFree() << ")");
    int pairs = 0;
    if (copy) {
        const int src = s.blocks.back();
        const int dst = allocate();
        unref(src);
        s.blocks.back() = dst;
        cow[0] = src;
        cow[1] = dst;
        pairs = 1;
    }
    for (int i = 0; i < fresh; ++i) s.blocks.push_back(allocate());
    return pairs;
}

void BlockManager::commit(int64_t id, int ntokens, const int64_t *tokens) {
    Seq &s = seq(id);
    LLAISYS_CHECK(ntokens >= 0, "kv block manager: negative token count");
    LLAISYS_CHECK(s.len + ntokens <= int(s.blocks.size()) * kBlockTokens,
                  "kv block manager: commit of " << ntokens << " tokens past the reserved blocks of sequence " << id);
    if (!tokens) s.hashable = false;
    for (int i = 0; i < ntokens; ++i) {
        if (s.hashable) s.tail.push_back(tokens[i]);
        ++s.len;
        if (s.len % kBlockTokens == 0) {
            if (s.hashable) cacheFullBlock(s, s.blocks[s.len / kBlockTokens - 1], s.tail.data());
            s.tail.clear();
        }
    }
}

void BlockManager::release(int64_t id) {
    Seq &s = seq(id);
    for (int b : s.blocks) unref(b);
    seqs_.erase(id);
}

int BlockManager::length(int64_t id) const { return seq(id).len; }

int BlockManager::buildTable(const int64_t *ids, size_t B, int32_t *table, size_t max_pages, int32_t *ctx_len) const {
    int widest = 0;
    for (size_t b = 0; b < B; ++b) {
        const Seq &s = seq(ids[b]);
        // Reserved blocks past the length are included: appends write there.
        const size_t pages = s.blocks.size();
        widest = std::max(widest, int(pages));
        if (!table) continue;
        LLAISYS_CHECK(pages <= max_pages,
                      "kv block manager: sequence " << ids[b] << " maps " << pages << " pages > max_pages " << max_pages);
        for (size_t p = 0; p < max_pages; ++p) table[b * max_pages + p] = p < s.blocks.size() ? s.blocks[p] : -1;
        if (ctx_len) ctx_len[b] = s.len;
    }
    return widest;
}

} // namespace llaisys::kvcache
