"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each check is chosen so a plausible slip fails it: a torch library routine in
float64 (scaled_dot_product_attention) for the general formula; closed forms
that isolate the causal mask offset (scale=0 -> prefix means), the GQA head
map (per-head constant values) and the single-key case; known answers for the
PRNG and the bf16 rounding; and, for the page format and the paged copies,
an independent reshape/transpose derivation plus round-trip and
untouched-bytes invariants on small pools.
"""
import numpy as np
import pytest
import torch

import oracle

REF_SHAPES = [(2, 2, 1, 1, 4), (5, 11, 4, 2, 8)]  # test/ops/self_attention.py:71-75


def sdpa64(q, k, v, scale):
    """float64 torch restatement: bottom-right causal mask, GQA via enable_gqa."""
    L, nh, d = q.shape
    S, nkvh, _ = k.shape
    qt = torch.from_numpy(q.astype(np.float64)).transpose(0, 1)
    kt = torch.from_numpy(k.astype(np.float64)).transpose(0, 1)
    vt = torch.from_numpy(v.astype(np.float64)).transpose(0, 1)
    mask = torch.ones(L, S, dtype=torch.bool).tril(diagonal=S - L)
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask, scale=scale,
                                                           enable_gqa=(nh != nkvh))
    return out.transpose(0, 1).numpy()


@pytest.mark.parametrize("L,S,nh,nkvh,d", REF_SHAPES + [(1, 513, 12, 2, 128), (7, 7, 6, 1, 16), (3, 40, 12, 2, 128)])
def test_self_attention_matches_torch_sdpa(L, S, nh, nkvh, d):
    q = oracle.randn(1, (L, nh, d))
    k = oracle.randn(2, (S, nkvh, d))
    v = oracle.randn(3, (S, nkvh, d))
    scale = 1.0 / d**0.5
    got = oracle.self_attention(q, k, v, scale)
    ref = sdpa64(q, k, v, scale)
    assert np.max(np.abs(got - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_single_key_returns_v():
    q = oracle.randn(4, (1, 4, 8))
    k = oracle.randn(5, (1, 2, 8))
    v = oracle.randn(6, (1, 2, 8))
    out = oracle.self_attention(q, k, v, 0.35)
    for h in range(4):
        np.testing.assert_array_equal(out[0, h], v[0, h // 2])


@pytest.mark.parametrize("L,S", [(1, 9), (4, 4), (5, 11)])
def test_zero_scale_gives_causal_prefix_means(L, S):
    # scale 0 -> uniform weights over exactly the visible keys j <= i + S - L.
    q = oracle.randn(7, (L, 2, 8))
    k = oracle.randn(8, (S, 1, 8))
    v = oracle.randn(9, (S, 1, 8))
    out = oracle.self_attention(q, k, v, 0.0)
    for i in range(L):
        want = v[: i + S - L + 1, 0].astype(np.float64).mean(axis=0)
        np.testing.assert_allclose(out[i, 0], want, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(out[i, 1], want, rtol=1e-5, atol=1e-6)


def test_gqa_head_map_is_repeat_interleave():
    # kv head j holds the constant j: query head h must read j = h // (nh/nkvh),
    # not h % nkvh (that would be repeat, not repeat_interleave).
    nh, nkvh = 12, 4
    q = oracle.randn(10, (3, nh, 8))
    k = oracle.randn(11, (6, nkvh, 8))
    v = np.broadcast_to(np.arange(nkvh, dtype=np.float32)[None, :, None], (6, nkvh, 8)).copy()
    out = oracle.self_attention(q, k, v, 0.3)
    for h in range(nh):
        np.testing.assert_allclose(out[:, h], h // (nh // nkvh), atol=1e-6)


def test_splitmix64_known_answer_and_randn_moments():
    # Published splitmix64 sequence from state 0.
    assert int(oracle.splitmix64(0, 1)[0]) == 0xE220A8397B1DCDAF
    assert int(oracle.splitmix64(0, 2)[1]) == 0x6E789E6AA1B965F4
    z = oracle.randn(123, (200000,))
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    np.testing.assert_array_equal(z, oracle.randn(123, (200000,)))


def test_bf16_round_to_nearest_even():
    one = np.float32(1.0)
    vals = np.array([1.0, 1 + 2**-8, 1 + 3 * 2**-8, -2.5, 65504.0, 1e-40], np.float32)
    got = oracle.f32_to_bf16(vals)
    assert got[0] == 0x3F80 and got[1] == 0x3F80 and got[2] == 0x3F82
    x = oracle.randn(5, (10000,)) * 100
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(oracle.f32_to_bf16(x), ref)
    np.testing.assert_array_equal(oracle.bf16_to_f32(oracle.f32_to_bf16(x)), torch.from_numpy(x).to(torch.bfloat16).float().numpy())
    assert oracle.bf16_to_f32(np.array([0x3F80], np.uint16))[0] == one


def test_page_format_two_derivations_agree_and_round_trip():
    x = (np.arange(5 * 16 * 128) % 65521).astype(np.uint16).reshape(5, 16, 128)
    for is_v in (False, True):
        a = oracle.pack_pages_np(x, is_v)
        np.testing.assert_array_equal(a, oracle.pack_pages_c(x, is_v))
        np.testing.assert_array_equal(oracle.unpack_pages_np(a, is_v), x)
        np.testing.assert_array_equal(oracle.unpack_pages_c(a, is_v), x)
    # Spot values: K (t=3, d=17) -> (17//8)*128 + 3*8 + 1 = 281.
    lin = np.arange(16 * 128, dtype=np.uint16).reshape(1, 16, 128)
    kp = oracle.pack_pages_np(lin, False).reshape(-1)
    assert kp[281] == 3 * 128 + 17
    # V (t=6, d=50) -> 1*512 + 1*128 + 2*8 + 1*4 + 2 = 662.
    vp = oracle.pack_pages_np(lin, True).reshape(-1)
    assert vp[662] == 6 * 128 + 50


def _random_layout(seed, B, max_len, nb, nkvh=2):
    lens = oracle.randint(seed, B, 0, max_len)
    maxp = max(1, int(np.max((lens + 16) // 16)))
    perm = oracle.permutation(seed + 1, nb)
    table = np.full((B, maxp), -1, np.int32)
    used = 0
    for b in range(B):
        need = (lens[b] + 16) // 16  # pages for len+1 tokens
        table[b, :need] = perm[used:used + need]
        used += need
    assert used <= nb
    return lens.astype(np.int32), table


def test_append_then_gather_round_trips_and_leaves_other_bytes():
    B, nb, nkvh = 6, 64, 2
    lens, table = _random_layout(3, B, 120, nb, nkvh)
    k_pool = oracle.randint(4, nb * nkvh * 16 * 128, 0, 65535).astype(np.uint16).reshape(nb, nkvh, 16, 128)
    v_pool = oracle.randint(5, nb * nkvh * 16 * 128, 0, 65535).astype(np.uint16).reshape(nb, nkvh, 16, 128)
    k0, v0 = k_pool.copy(), v_pool.copy()
    total = int(lens.sum())
    ks = oracle.randint(6, total * nkvh * 128, 0, 65535).astype(np.uint16).reshape(total, nkvh, 128)
    vs = oracle.randint(7, total * nkvh * 128, 0, 65535).astype(np.uint16).reshape(total, nkvh, 128)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    # Prefill-style append of every sequence's tokens in one call (ctx = 0).
    assert oracle.paged_append(k_pool, v_pool, ks, vs, table, np.zeros(B, np.int32), cu) == 0
    gk, gv = oracle.paged_gather(k_pool, v_pool, table, cu)
    np.testing.assert_array_equal(gk, ks)
    np.testing.assert_array_equal(gv, vs)
    # Bytes of pages/slots no sequence owns are untouched.
    touched = np.zeros((nb, 16), bool)
    for b in range(B):
        for p in range(lens[b]):
            touched[table[b, p // 16], p % 16] = True
    np.testing.assert_array_equal(k_pool[~touched[:, None, :].repeat(nkvh, 1)], k0[~touched[:, None, :].repeat(nkvh, 1)])
    np.testing.assert_array_equal(v_pool[~touched[:, None, :].repeat(nkvh, 1)], v0[~touched[:, None, :].repeat(nkvh, 1)])
    # A decode append (one token each at ctx = lens) then gather of len+1.
    kn = oracle.randint(8, B * nkvh * 128, 0, 65535).astype(np.uint16).reshape(B, nkvh, 128)
    vn = oracle.randint(9, B * nkvh * 128, 0, 65535).astype(np.uint16).reshape(B, nkvh, 128)
    assert oracle.paged_append(k_pool, v_pool, kn, vn, table, lens, None) == 0
    cu1 = np.concatenate([[0], np.cumsum(lens + 1)]).astype(np.int32)
    gk, gv = oracle.paged_gather(k_pool, v_pool, table, cu1)
    for b in range(B):
        np.testing.assert_array_equal(gk[cu1[b]:cu1[b + 1] - 1], ks[cu[b]:cu[b + 1]])
        np.testing.assert_array_equal(gk[cu1[b + 1] - 1], kn[b])
        np.testing.assert_array_equal(gv[cu1[b + 1] - 1], vn[b])


def test_append_reports_unmapped_page():
    k_pool = np.zeros((2, 1, 16, 128), np.uint16)
    v_pool = np.zeros_like(k_pool)
    table = np.array([[0, -1]], np.int32)
    kn = np.ones((1, 1, 128), np.uint16)
    assert oracle.paged_append(k_pool, v_pool, kn, kn, table, np.array([16], np.int32)) == 1
    assert oracle.paged_append(k_pool, v_pool, kn, kn, table, np.array([15], np.int32)) == 0


@pytest.mark.parametrize("varlen", [False, True])
def test_paged_attention_is_gather_plus_self_attention(varlen):
    B, nb, nkvh, nh = 5, 80, 2, 12
    lens, table = _random_layout(11, B, 150, nb, nkvh)
    ctx = lens + 1
    k_pool = oracle.f32_to_bf16(oracle.randn(12, (nb, nkvh, 16, 128)))
    v_pool = oracle.f32_to_bf16(oracle.randn(13, (nb, nkvh, 16, 128)))
    lq = np.minimum(oracle.randint(14, B, 1, 9), ctx).astype(np.int32) if varlen else np.ones(B, np.int32)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    T = int(cu_q[-1])
    q = oracle.f32_to_bf16(oracle.randn(15, (T, nh, 128)))
    scale = 1 / 128**0.5
    out = oracle.paged_attention(q, k_pool, v_pool, table, ctx, scale, cu_q if varlen else None)
    cu_kv = np.concatenate([[0], np.cumsum(ctx)]).astype(np.int32)
    gk, gv = oracle.paged_gather(k_pool, v_pool, table, cu_kv)
    for b in range(B):
        kb = oracle.bf16_to_f32(gk[cu_kv[b]:cu_kv[b + 1]])
        vb = oracle.bf16_to_f32(gv[cu_kv[b]:cu_kv[b + 1]])
        qb = oracle.bf16_to_f32(q[cu_q[b]:cu_q[b + 1]])
        ref = sdpa64(qb, kb, vb, scale)
        np.testing.assert_allclose(out[cu_q[b]:cu_q[b + 1]], ref, rtol=1e-5, atol=1e-5)
