"""Host-side KV block manager (native, include/llaisys/kv_cache.h). CPU only."""
import numpy as np
import pytest

import llaisys_amd as L
import oracle

P = 16


def table_of(m, sid):
    t, ctx = m.block_table([sid])
    return [int(b) for b in t[0] if b >= 0], int(ctx[0])


def test_allocation_and_exhaustion_leave_state_unchanged():
    m = L.KVBlockManager(4)
    assert m.create(1) == 0 and m.num_free() == 4
    assert m.reserve(1, 33) == [] and m.num_free() == 1  # 3 blocks for 33 tokens
    blocks, ctx = table_of(m, 1)
    assert blocks == [0, 1, 2] and ctx == 0
    m.commit(1, 33)
    assert m.length(1) == 33
    m.create(2)
    with pytest.raises(L.LlaisysError, match="out of blocks"):
        m.reserve(2, 17)  # needs 2, 1 free
    assert m.num_free() == 1 and table_of(m, 2) == ([], 0)
    with pytest.raises(L.LlaisysError, match="past the reserved"):
        m.commit(1, 16)
    m.free(1)
    assert m.num_free() == 4


def test_fork_shares_blocks_and_copy_on_write_of_partial_tail():
    m = L.KVBlockManager(8)
    m.create(1)
    m.reserve(1, 20)
    m.commit(1, 20)
    m.fork(1, 2)
    assert table_of(m, 2) == table_of(m, 1)
    assert m.num_free() == 6
    cow = m.reserve(2, 1)  # writes into the shared partial block 1
    assert len(cow) == 1 and cow[0][0] == 1 and cow[0][1] not in (0, 1)
    b1, _ = table_of(m, 1)
    b2, _ = table_of(m, 2)
    assert b1[0] == b2[0] and b1[1] == 1 and b2[1] == cow[0][1]
    assert m.reserve(1, 1) == []  # the old tail is private to 1 now
    m.free(1)
    m.free(2)
    assert m.num_free() == 8


def test_fork_at_block_boundary_needs_no_copy():
    m = L.KVBlockManager(8)
    m.create(1)
    m.reserve(1, 32)
    m.commit(1, 32)
    m.fork(1, 2)
    assert m.reserve(2, 5) == []
    b1, _ = table_of(m, 1)
    b2, _ = table_of(m, 2)
    assert b2[:2] == b1 and len(b2) == 3


def test_prefix_cache_reuses_full_blocks_and_verifies_tokens():
    m = L.KVBlockManager(16)
    prompt = oracle.randint(1, 40, 0, 50000)
    m.create(1)
    m.reserve(1, 40)
    m.commit(1, 40, prompt)
    b1, _ = table_of(m, 1)
    # Alive: a new sequence shares the 2 full blocks (at least one token left to compute).
    assert m.create(2, np.concatenate([prompt, [7, 8]])) == 32
    b2, ctx2 = table_of(m, 2)
    assert b2 == b1[:2] and ctx2 == 32
    # Exactly 32 tokens: only one block reused (the last token must be computed).
    assert m.create(3, prompt[:32]) == 16
    # Different second block: only the first block matches.
    other = prompt.copy()
    other[20] += 1
    assert m.create(4, other) == 16
    # Freed but cached blocks stay reusable.
    for s in (1, 2, 3, 4):
        m.free(s)
    assert m.num_free() == 16
    assert m.create(5, prompt) == 32 and table_of(m, 5)[0] == b1[:2]
    # Commits without token ids never enter the cache.
    m.create(6)
    m.reserve(6, 16)
    m.commit(6, 16)
    assert m.create(7, np.zeros(17, np.int64)) == 0


def test_cached_blocks_are_reclaimed_oldest_first():
    m = L.KVBlockManager(4)
    a = oracle.randint(2, 33, 0, 1000)
    b = oracle.randint(3, 33, 0, 1000)
    for sid, toks in ((1, a), (2, b)):
        m.create(sid)
        m.reserve(sid, 32)
        m.commit(sid, 32, toks[:32])
    m.free(1)  # a's blocks released first
    m.free(2)
    assert m.num_free() == 4
    m.create(3)
    m.reserve(3, 32)  # takes the two oldest cached blocks: a's
    assert m.create(4, a) == 0
    assert m.create(5, b) == 32


def test_errors():
    m = L.KVBlockManager(2)
    with pytest.raises(L.LlaisysError, match="unknown sequence"):
        m.reserve(9, 1)
    m.create(1)
    with pytest.raises(L.LlaisysError, match="already exists"):
        m.create(1)
    with pytest.raises(L.LlaisysError, match="positive"):
        L.KVBlockManager(0)
    m.reserve(1, 32)
    with pytest.raises(L.LlaisysError, match="max_pages"):
        m.block_table([1], max_pages=1)


def test_random_operations_keep_refcount_invariants():
    # Model: free blocks = pool minus the union of mapped blocks (cached
    # unreferenced blocks count as free); a block is shared only through fork
    # or prefix reuse; after reserve the partial tail block is private.
    rng = np.random.default_rng(0)
    nb = 64
    m = L.KVBlockManager(nb)
    live = {}
    next_id = 0
    for step in range(600):
        op = rng.integers(0, 5)
        if op == 0 or not live:
            toks = rng.integers(0, 4, size=int(rng.integers(1, 60)))
            hit = m.create(next_id, toks)
            assert hit % P == 0 and hit <= len(toks) - 1
            live[next_id] = list(toks[:hit])
            next_id += 1
        elif op == 1:
            sid = int(rng.choice(list(live)))
            n = int(rng.integers(1, 40))
            try:
                m.reserve(sid, n)
            except L.LlaisysError:
                continue
            toks = list(rng.integers(0, 4, size=n))
            m.commit(sid, n, toks)
            live[sid] += toks
        elif op == 2:
            sid = int(rng.choice(list(live)))
            m.fork(sid, next_id)
            live[next_id] = list(live[sid])
            next_id += 1
        else:
            sid = int(rng.choice(list(live)))
            m.free(sid)
            del live[sid]
        mapped = set()
        for sid, toks in live.items():
            blocks, ctx = table_of(m, sid)
            assert ctx == len(toks)
            assert len(blocks) >= (ctx + P - 1) // P
            mapped |= set(blocks)
        assert m.num_free() == nb - len(mapped)
