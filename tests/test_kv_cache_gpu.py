"""A decode loop driven by the native block manager on the GPU: ragged prefill
append, per-step reserve / copy-on-write / append / commit / attention, with a
fork mid-way. KV history is tracked in numpy; gathers must be bit-exact and
attention must match the fp32 oracle on that history."""
import numpy as np
import pytest
import torch

import llaisys_amd as L
import oracle
from utils import bits, from_bits, to_llaisys, to_torch

pytestmark = pytest.mark.gpu

NKVH, NH, D = 2, 12, 128
SCALE = 1.0 / D**0.5


def _i32(a):
    return to_llaisys(torch.from_numpy(np.ascontiguousarray(a, np.int32)))


def _rows(seed, n):
    return oracle.f32_to_bf16(oracle.randn(seed, (n, NKVH, D)))


def test_decode_loop_with_block_manager_fork_and_cow():
    nb = 128
    m = L.KVBlockManager(nb)
    kp = to_llaisys(torch.zeros((nb, NKVH, 16, D), dtype=torch.bfloat16, device="cuda"))
    vp = to_llaisys(torch.zeros((nb, NKVH, 16, D), dtype=torch.bfloat16, device="cuda"))
    hist_k, hist_v = {}, {}

    # Ragged prefill of six sequences in one append.
    prompts = {0: 5, 1: 16, 2: 17, 3: 40, 4: 1, 5: 33}
    ids = list(prompts)
    for sid, n in prompts.items():
        assert m.create(sid) == 0
        m.reserve(sid, n)
    table, ctx = m.block_table(ids)
    new = np.array([prompts[s] for s in ids], np.int32)
    cu = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    kn, vn = _rows(1, int(cu[-1])), _rows(2, int(cu[-1]))
    L.Ops.paged_kv_append(kp, vp, to_llaisys(from_bits(kn)), to_llaisys(from_bits(vn)), _i32(table), _i32(ctx), _i32(cu))
    for i, sid in enumerate(ids):
        m.commit(sid, int(new[i]))
        hist_k[sid] = kn[cu[i]:cu[i + 1]].copy()
        hist_v[sid] = vn[cu[i]:cu[i + 1]].copy()
    assert L.device_error_flags() == 0

    def check_gather(live):
        table, ctx = m.block_table(live)
        cu = np.concatenate([[0], np.cumsum(ctx)]).astype(np.int32)
        T = int(cu[-1])
        ko = to_llaisys(torch.zeros((T, NKVH, D), dtype=torch.bfloat16, device="cuda"))
        vo = to_llaisys(torch.zeros((T, NKVH, D), dtype=torch.bfloat16, device="cuda"))
        L.Ops.paged_kv_gather(ko, vo, kp, vp, _i32(table), _i32(cu))
        gk, gv = bits(to_torch(ko)), bits(to_torch(vo))
        for i, sid in enumerate(live):
            np.testing.assert_array_equal(gk[cu[i]:cu[i + 1]], hist_k[sid])
            np.testing.assert_array_equal(gv[cu[i]:cu[i + 1]], hist_v[sid])

    check_gather(ids)
    live = list(ids)
    for step in range(8):
        if step == 3:  # fork the 40-token sequence (partial tail): the child's first write copies the tail
            m.fork(3, 100)
            hist_k[100], hist_v[100] = hist_k[3].copy(), hist_v[3].copy()
            live.append(100)
        pairs = []
        for sid in live:
            pairs += m.reserve(sid, 1)
        if pairs:
            L.Ops.paged_kv_copy_blocks(kp, vp, _i32(np.array(pairs, np.int32).reshape(-1, 2)))
        table, ctx = m.block_table(live)
        B = len(live)
        kn, vn = _rows(10 + step, B), _rows(20 + step, B)
        L.Ops.paged_kv_append(kp, vp, to_llaisys(from_bits(kn)), to_llaisys(from_bits(vn)), _i32(table), _i32(ctx))
        for i, sid in enumerate(live):
            m.commit(sid, 1)
            hist_k[sid] = np.concatenate([hist_k[sid], kn[i:i + 1]])
            hist_v[sid] = np.concatenate([hist_v[sid], vn[i:i + 1]])
        q = oracle.f32_to_bf16(oracle.randn(30 + step, (B, NH, D)))
        out = to_llaisys(torch.zeros((B, NH, D), dtype=torch.float32, device="cuda"))
        L.Ops.paged_attention(out, to_llaisys(from_bits(q)), kp, vp, _i32(table), _i32(ctx + 1), SCALE)
        got = to_torch(out).cpu().numpy()
        assert L.device_error_flags() == 0
        for i, sid in enumerate(live):
            ref = oracle.self_attention(oracle.bf16_to_f32(q[i:i + 1]), oracle.bf16_to_f32(hist_k[sid]),
                                        oracle.bf16_to_f32(hist_v[sid]), SCALE)
            assert np.max(np.abs(got[i] - ref[0])) <= 1e-4 * np.max(np.abs(ref)), (step, sid)
        if step == 3:
            assert pairs, "the fork's first append must have copied the shared tail"
    check_gather(live)
    for sid in live:
        m.free(sid)
    assert m.num_free() == nb
