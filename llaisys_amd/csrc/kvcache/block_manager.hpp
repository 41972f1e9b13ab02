// Host-side manager of the paged KV pool: free list, per-sequence block
// lists, reference counts for shared prefixes, copy-on-write of a shared last
// block, and a prefix cache of full blocks keyed by the chained hash of their
// token ids (reused least-recently-released first when the free list runs
// dry). Not thread-safe: one manager per scheduler thread.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <list>
#include <unordered_map>
#include <vector>

namespace llaisys::kvcache {

constexpr int kBlockTokens = 16;

class BlockManager {
public:
    // scatter: hand out fresh blocks in a fixed scattered order instead of
    // 0, 1, 2, ...; consecutive pages of a sequence then land far apart in the
    // pool, which streams faster (the attention kernels' waves start at the
    // same offsets of their sequences, so pools laid out in order concentrate
    // each moment's reads at one stride).
    explicit BlockManager(int num_blocks, bool scatter = false);

    int numBlocks() const { return int(ref_.size()); }
    int numFree() const { return int(free_.size() + lru_.size()); }

    // Returns the number of leading tokens served from the prefix cache.
    int create(int64_t id, const int64_t *tokens, size_t ntokens);
    void fork(int64_t parent, int64_t child);
    // Returns the number of copy-on-write pairs written to cow (0 or 1).
    int reserve(int64_t id, int ntokens, int32_t *cow, int cow_capacity);
    void commit(int64_t id, int ntokens, const int64_t *tokens);
    void release(int64_t id);
    int length(int64_t id) const;
    // Returns the largest page count among the sequences.
    int buildTable(const int64_t *ids, size_t B, int32_t *table, size_t max_pages, int32_t *ctx_len) const;

private:
    struct Seq {
        std::vector<int> blocks;
        int len = 0;
        bool hashable = true;                    // all committed tokens known so far
        uint64_t chain = 0;                      // hash of the full blocks' tokens
        std::vector<int64_t> tail;               // tokens of the partial last block
    };
    struct CachedBlock {
        uint64_t parent = 0;                     // chain hash before this block
        std::array<int64_t, kBlockTokens> tokens{};
    };

    const Seq &seq(int64_t id) const;
    Seq &seq(int64_t id);
    int allocate();
    void unref(int block);
    void cacheFullBlock(Seq &s, int block, const int64_t *tokens);
    static uint64_t chainHash(uint64_t parent, const int64_t *tokens);

    std::vector<int> ref_;                       // sequences mapping each block
    std::vector<int> free_;                      // unreferenced, uncached (stack)
    std::list<int> lru_;                         // unreferenced, cached; front = oldest
    std::vector<std::list<int>::iterator> lru_pos_;
    std::vector<bool> in_lru_;
    std::vector<uint64_t> hash_of_;              // chain hash a cached block is registered under
    std::vector<bool> cached_;
    std::vector<CachedBlock> cached_data_;
    std::unordered_map<uint64_t, int> prefix_;   // chain hash -> block
    std::unordered_map<int64_t, Seq> seqs_;
};

} // namespace llaisys::kvcache
