"""Continuous-batching scheduler (include/llaisys/serving.h) over the host-only
simulated model: every generated token must equal the simulated model's
greedy continuation of the request's own history (a hash of all its tokens),
whatever the batching, chunking and preemption; plus the stop conditions,
prefix reuse and argument errors. No GPU: the simulated model uses the same
KV block manager as the Qwen2 model and no HIP call."""
import random

import pytest

import llaisys_amd as L
from llaisys_amd.serving import RequestStatus, Scheduler, sim_greedy

VOCAB = 5000


def expected(prompt, n, vocab=VOCAB):
    h, out = list(prompt), []
    for _ in range(n):
        t = sim_greedy(h, vocab)
        out.append(t)
        h.append(t)
    return out


def test_sim_greedy_is_fnv1a_64():
    # FNV-1a 64 of the empty history is the offset basis; one zero token
    # multiplies it by the prime once.
    assert sim_greedy([], 1 << 64) == 14695981039346656037
    assert sim_greedy([0], 1 << 64) == (14695981039346656037 * 1099511628211) % (1 << 64)
    assert sim_greedy([1, 2], 97) == sim_greedy([1, 2], 1 << 64) % 97


@pytest.mark.parametrize("max_seqs,budget,chunk,blocks", [
    (1, 64, 64, 256),     # one request at a time
    (4, 40, 16, 256),     # chunked prefill mixed with decodes
    (16, 4096, 512, 512), # everything at once
    (8, 24, 8, 40),       # tight pool: preemption and recomputation
])
def test_outputs_match_each_requests_own_greedy_continuation(max_seqs, budget, chunk, blocks):
    rng = random.Random(max_seqs * 1000 + budget)
    s = Scheduler.simulated(blocks, VOCAB, 4096, max_seqs=max_seqs, max_step_tokens=budget, prefill_chunk=chunk)
    reqs = {}
    for _ in range(12):
        p = [rng.randrange(VOCAB) for _ in range(rng.randint(1, 120))]
        n = rng.randint(1, 60)
        reqs[s.add(p, max_new_tokens=n)] = (p, n)
    steps = s.run()
    st = s.stats()
    assert st["finished"] == len(reqs) and steps == st["steps"]
    for rid, (p, n) in reqs.items():
        assert s.status(rid) == RequestStatus.MAX_TOKENS
        assert s.tokens(rid) == expected(p, n), f"request {rid}"
    # every generated token but each request's first comes from a decode
    assert st["decode_tokens"] >= sum(n - 1 for _, n in reqs.values())
    assert st["prefill_tokens"] >= sum(len(p) for p, _ in reqs.values()) - 16 * len(reqs)
    if blocks == 40:
        assert st["preemptions"] > 0


def test_requests_added_while_serving():
    rng = random.Random(5)
    s = Scheduler.simulated(128, VOCAB, 4096, max_seqs=4, max_step_tokens=32, prefill_chunk=8)
    reqs = {}
    for wave in range(5):
        for _ in range(3):
            p = [rng.randrange(VOCAB) for _ in range(rng.randint(1, 40))]
            reqs[s.add(p, max_new_tokens=10)] = p
        for _ in range(7):
            s.step()
    s.run()
    for rid, p in reqs.items():
        assert s.tokens(rid) == expected(p, 10)


def test_eos_ends_a_request_at_the_end_token():
    p = [7, 8, 9]
    full = expected(p, 10)
    eos = full[3]
    assert eos not in full[:3]
    s = Scheduler.simulated(64, VOCAB, 4096)
    rid = s.add(p, max_new_tokens=10, eos=eos)
    s.run()
    assert s.status(rid) == RequestStatus.EOS
    assert s.tokens(rid) == full[:4]


def test_length_limit_ends_a_request_at_max_seq_len():
    s = Scheduler.simulated(64, VOCAB, 50)
    p = list(range(40))
    rid = s.add(p, max_new_tokens=100)
    s.run()
    assert s.status(rid) == RequestStatus.LENGTH
    out = s.tokens(rid)
    # the cache holds 50 tokens; the last generated token has no slot left
    assert len(p) + len(out) == 51 and out == expected(p, len(out))


def test_prefix_cache_reuse_skips_recomputation():
    p = list(range(100, 170))  # 70 tokens: 4 full blocks cacheable
    s = Scheduler.simulated(64, VOCAB, 4096, max_seqs=1)
    a = s.add(p, max_new_tokens=3)
    b = s.add(p, max_new_tokens=3)
    s.run()
    assert s.tokens(a) == s.tokens(b) == expected(p, 3)
    # b reuses a's 4 full blocks (64 tokens) and computes the last 6
    assert s.stats()["prefill_tokens"] == 70 + 6


def test_request_larger_than_the_pool_ends_with_no_capacity():
    s = Scheduler.simulated(3, VOCAB, 4096, max_seqs=4, max_step_tokens=64, prefill_chunk=16)
    big = s.add(list(range(200)), max_new_tokens=5)  # 13 blocks: never fits
    small = s.add([1, 2, 3], max_new_tokens=5)
    s.run(max_steps=200)
    assert s.status(big) == RequestStatus.NO_CAPACITY
    assert s.status(small) == RequestStatus.MAX_TOKENS
    assert s.tokens(small) == expected([1, 2, 3], 5)


def test_release_and_errors():
    s = Scheduler.simulated(16, VOCAB, 64)
    with pytest.raises(L.LlaisysError):
        s.add([], max_new_tokens=1)
    with pytest.raises(L.LlaisysError):
        s.add([1], max_new_tokens=0)
    with pytest.raises(L.LlaisysError):
        s.add(list(range(65)), max_new_tokens=1)  # longer than max_seq_len
    rid = s.add([1, 2], max_new_tokens=2)
    with pytest.raises(L.LlaisysError):
        s.release(rid)  # not finished
    s.run()
    s.release(rid)
    with pytest.raises(KeyError):
        s.status(rid)
    assert s.step() == 0  # idle: no step runs
    with pytest.raises(L.LlaisysError):
        Scheduler.simulated(16, VOCAB, 64, max_seqs=0)
