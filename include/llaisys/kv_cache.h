/*
 * Host-side KV block manager for the paged pool of include/llaisys/ops.h.
 *
 * New (no reference counterpart: the reference only asks for a "KV-Cache pool
 * with prefix matching" and continuous batching as projects, README.md:412,
 * :424). It owns the free list of physical blocks, each sequence's ordered
 * block list and length, block reference counts (sequences forked from a
 * common prefix share blocks), and a prefix cache of full blocks keyed by the
 * chained hash of their token ids, so a new sequence whose prompt starts with
 * cached blocks reuses them instead of recomputing their K/V.
 *
 * Sequences are named by caller-chosen 64-bit ids. Functions return >= 0 on
 * success and -1 on failure (llaisysGetLastError has the message); a failed
 * call changes nothing.
 */
#ifndef LLAISYS_KV_CACHE_H
#define LLAISYS_KV_CACHE_H

#include "../llaisys.h"

__C {
    typedef struct LlaisysKVBlockManager *llaisysKVBlockManager_t;

    /* Pool of num_blocks blocks of 16 tokens (num_blocks = dim 0 of the pool tensors). */
    __export llaisysKVBlockManager_t llaisysKVBlockManagerCreate(int num_blocks);
    __export void llaisysKVBlockManagerDestroy(llaisysKVBlockManager_t m);
    /* Blocks neither mapped by a sequence nor holding a cached prefix, plus
     * cached-but-unreferenced blocks (reclaimed least-recently-used first). */
    __export int llaisysKVNumFreeBlocks(llaisysKVBlockManager_t m);

    /* New empty sequence. If tokens != NULL, the longest run of cached full
     * blocks matching tokens[0 .. 16k) is mapped (shared, refcounted) and its
     * length returned: those positions need no append. Else returns 0. */
    __export int llaisysKVSeqCreate(llaisysKVBlockManager_t m, int64_t seq_id, const int64_t *tokens, size_t ntokens);

    /* child shares all of parent's blocks and length. */
    __export int llaisysKVSeqFork(llaisysKVBlockManager_t m, int64_t parent, int64_t child);

    /* Map blocks so positions [len, len + ntokens) of the sequence are
     * writable. A last block shared with another sequence (or cached) that
     * would be written is replaced by a private copy: the (src, dst) block pair
     * is written to cow_pairs[2*i], cow_pairs[2*i+1] for the caller to copy with
     * llaisysPagedKVCopyBlocks before appending. Returns the number of pairs
     * (0 or 1), -1 if the pool has too few free blocks or cow_capacity is 0 and
     * a copy is needed. Does not change the length. */
    __export int llaisysKVSeqReserve(llaisysKVBlockManager_t m, int64_t seq_id, int ntokens, int32_t *cow_pairs,
                                     int cow_capacity);

    /* Advance the length by ntokens (after their K/V were appended). tokens
     * (may be NULL) are their ids: blocks they complete enter the prefix cache. */
    __export int llaisysKVSeqCommit(llaisysKVBlockManager_t m, int64_t seq_id, int ntokens, const int64_t *tokens);

    /* Drop the sequence; blocks no other sequence maps are freed (cached ones
     * stay reusable until reclaimed). */
    __export int llaisysKVSeqFree(llaisysKVBlockManager_t m, int64_t seq_id);

    __export int llaisysKVSeqLength(llaisysKVBlockManager_t m, int64_t seq_id);

    /* Fill table[B, max_pages] (unused entries -1) and ctx_len[B] for the
     * given sequences, ready to load into the I32 block_table / ctx_len
     * tensors. Mapped-but-uncommitted blocks (from Reserve) are included, as
     * appends write into them. Returns the largest number of mapped blocks;
     * -1 if a sequence maps more than max_pages blocks or is unknown. With
     * table == NULL only the return value is computed (to size the table). */
    __export int llaisysKVBuildBlockTable(llaisysKVBlockManager_t m, const int64_t *seq_ids, size_t B, int32_t *table,
                                          size_t max_pages, int32_t *ctx_len);
}

#endif /* LLAISYS_KV_CACHE_H */
