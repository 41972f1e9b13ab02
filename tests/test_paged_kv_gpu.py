"""Paged KV append/gather on the GPU: bit-exact against the oracle (logical
copies) and against the oracle's page-format packing of the pool bytes."""
import numpy as np
import pytest
import torch

import llaisys_amd as L
import oracle
from utils import bits, from_bits, to_llaisys, to_torch

pytestmark = pytest.mark.gpu


def _setup(seed, lens, nb, nkvh=2, extra_pages=0):
    """Tables mapping enough pages for len+1 tokens per sequence, random pool bytes."""
    lens = np.asarray(lens, np.int32)
    need = (lens + 16) // 16
    maxp = int(need.max(initial=1)) + extra_pages
    assert need.sum() <= nb
    perm = oracle.permutation(seed, nb)
    table = np.full((len(lens), maxp), -1, np.int32)
    used = 0
    for b, p in enumerate(need):
        table[b, :p] = perm[used:used + p]
        used += p
    k_log = oracle.randint(seed + 1, nb * nkvh * 2048, 0, 65535).astype(np.uint16).reshape(nb, nkvh, 16, 128)
    v_log = oracle.randint(seed + 2, nb * nkvh * 2048, 0, 65535).astype(np.uint16).reshape(nb, nkvh, 16, 128)
    return lens, table, k_log, v_log


def _dev(k_log, v_log):
    return (to_llaisys(from_bits(oracle.pack_pages_np(k_log, False))),
            to_llaisys(from_bits(oracle.pack_pages_np(v_log, True))))


def _pool_logical(p, is_v, shape):
    return oracle.unpack_pages_np(bits(to_torch(p)).reshape(shape), is_v)


def _i32(a):
    return to_llaisys(torch.from_numpy(np.ascontiguousarray(a, np.int32)))


def test_config2_append_then_gather_bit_exact():
    # 32 sequences, len U[1,2048], 4096-block pool, 1 new token each.
    B, nb, nkvh = 32, 4096, 2
    seed = 0
    while True:
        lens = oracle.randint(seed, B, 1, 2048).astype(np.int32)
        if ((lens + 16) // 16).sum() <= nb:
            break
        seed += 1
    lens, table, k_log, v_log = _setup(100, lens, nb, nkvh)
    kp, vp = _dev(k_log, v_log)
    kn = oracle.f32_to_bf16(oracle.randn(7, (B, nkvh, 128)))
    vn = oracle.f32_to_bf16(oracle.randn(8, (B, nkvh, 128)))
    L.Ops.paged_kv_append(kp, vp, to_llaisys(from_bits(kn)), to_llaisys(from_bits(vn)), _i32(table), _i32(lens))
    assert L.device_error_flags() == 0
    assert oracle.paged_append(k_log, v_log, kn, vn, table, lens) == 0
    # Pool bytes equal the oracle's pool in page format.
    np.testing.assert_array_equal(_pool_logical(kp, False, k_log.shape), k_log)
    np.testing.assert_array_equal(_pool_logical(vp, True, v_log.shape), v_log)
    cu = np.concatenate([[0], np.cumsum(lens + 1)]).astype(np.int32)
    T = int(cu[-1])
    ko = to_llaisys(torch.zeros((T, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    vo = to_llaisys(torch.zeros((T, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    L.Ops.paged_kv_gather(ko, vo, kp, vp, _i32(table), _i32(cu))
    assert L.device_error_flags() == 0
    gk, gv = oracle.paged_gather(k_log, v_log, table, cu)
    np.testing.assert_array_equal(bits(to_torch(ko)), gk)
    np.testing.assert_array_equal(bits(to_torch(vo)), gv)


@pytest.mark.parametrize("nkvh", [1, 2, 5])
def test_ragged_prefill_append_with_empty_and_boundary_sequences(nkvh):
    ctx = np.array([0, 15, 16, 3, 40, 0, 31], np.int32)        # tokens already cached
    new = np.array([5, 1, 16, 0, 33, 17, 2], np.int32)         # tokens appended now
    total = ctx + new
    nb = int(((total + 16) // 16).sum()) + 4
    _, table, k_log, v_log = _setup(5, total, nb, nkvh)
    kp, vp = _dev(k_log, v_log)
    cu = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    T = int(cu[-1])
    kn = oracle.randint(20, T * nkvh * 128, 0, 65535).astype(np.uint16).reshape(T, nkvh, 128)
    vn = oracle.randint(21, T * nkvh * 128, 0, 65535).astype(np.uint16).reshape(T, nkvh, 128)
    L.Ops.paged_kv_append(kp, vp, to_llaisys(from_bits(kn)), to_llaisys(from_bits(vn)), _i32(table), _i32(ctx), _i32(cu))
    assert L.device_error_flags() == 0
    assert oracle.paged_append(k_log, v_log, kn, vn, table, ctx, cu) == 0
    np.testing.assert_array_equal(_pool_logical(kp, False, k_log.shape), k_log)
    np.testing.assert_array_equal(_pool_logical(vp, True, v_log.shape), v_log)
    cug = np.concatenate([[0], np.cumsum(total)]).astype(np.int32)
    Tg = int(cug[-1])
    ko = to_llaisys(torch.zeros((Tg, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    vo = to_llaisys(torch.zeros((Tg, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    L.Ops.paged_kv_gather(ko, vo, kp, vp, _i32(table), _i32(cug))
    gk, gv = oracle.paged_gather(k_log, v_log, table, cug)
    np.testing.assert_array_equal(bits(to_torch(ko)), gk)
    np.testing.assert_array_equal(bits(to_torch(vo)), gv)


def test_unmapped_page_and_overlong_context_set_error_flags():
    lens, table, k_log, v_log = _setup(9, [20, 3], 8, 2)
    kp, vp = _dev(k_log, v_log)
    kn = to_llaisys(torch.zeros((2, 2, 128), dtype=torch.bfloat16, device="cuda"))
    bad = table.copy()
    bad[0, 1] = 1000  # block id outside the pool
    L.Ops.paged_kv_append(kp, vp, kn, kn, _i32(bad), _i32(lens))
    assert L.device_error_flags() & 1
    L.Ops.paged_kv_append(kp, vp, kn, kn, _i32(table), _i32(np.array([20, 16 * table.shape[1]], np.int32)))
    assert L.device_error_flags() & 2
    assert L.device_error_flags() == 0  # cleared by the read
    # The untouched pool still matches (the bad rows were skipped, the good ones written).


@pytest.mark.parametrize("nkvh", [2, 3])
def test_gather_skips_unmapped_pages_and_flags_them(nkvh):
    # A multi-page sequence with an unmapped page in the middle: that page's rows
    # stay untouched and flag 1 is raised; every other page is gathered exactly.
    lens, table, k_log, v_log = _setup(11, [100, 37], 16, nkvh)
    kp, vp = _dev(k_log, v_log)
    bad = table.copy()
    bad[0, 2] = -1
    cu = np.array([0, 100, 137], np.int32)
    ko = to_llaisys(torch.zeros((137, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    vo = to_llaisys(torch.zeros((137, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    L.Ops.paged_kv_gather(ko, vo, kp, vp, _i32(bad), _i32(cu))
    assert L.device_error_flags() == 1
    gk, gv = oracle.paged_gather(k_log, v_log, table, cu)
    keep = np.ones(137, bool)
    keep[32:48] = False
    for got, want in ((bits(to_torch(ko)), gk), (bits(to_torch(vo)), gv)):
        np.testing.assert_array_equal(got[keep], want[keep])
        assert not got[~keep].any()
    # Lengths past the table's pages: flag 2, the mapped pages still gathered.
    cu_long = np.array([0, 16 * table.shape[1] + 5], np.int32)
    ko2 = to_llaisys(torch.zeros((int(cu_long[-1]), nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    vo2 = to_llaisys(torch.zeros((int(cu_long[-1]), nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    L.Ops.paged_kv_gather(ko2, vo2, kp, vp, _i32(table[:1]), _i32(cu_long))
    assert L.device_error_flags() == 2
    n = 16 * int((table[0] >= 0).sum())
    gk2, _ = oracle.paged_gather(k_log, v_log, table[:1], np.array([0, n], np.int32))
    np.testing.assert_array_equal(bits(to_torch(ko2))[:n], gk2)


def test_empty_calls_are_noops():
    _, table, k_log, v_log = _setup(3, [4], 4, 2)
    kp, vp = _dev(k_log, v_log)
    empty = to_llaisys(torch.zeros((0, 2, 128), dtype=torch.bfloat16, device="cuda"))
    L.Ops.paged_kv_append(kp, vp, empty, empty, _i32(table), _i32([4]), _i32([0, 0]))
    np.testing.assert_array_equal(_pool_logical(kp, False, k_log.shape), k_log)


def _fused_case(lens, nkvh, seed, nb=None):
    lens = np.asarray(lens, np.int32)
    nb = nb or int(((lens + 16) // 16).sum()) + 3
    lens, table, k_log, v_log = _setup(seed, lens, nb, nkvh)
    B = len(lens)
    kn = oracle.randint(seed + 3, B * nkvh * 128, 0, 65535).astype(np.uint16).reshape(B, nkvh, 128)
    vn = oracle.randint(seed + 4, B * nkvh * 128, 0, 65535).astype(np.uint16).reshape(B, nkvh, 128)
    return lens, table, k_log, v_log, kn, vn


@pytest.mark.parametrize("nkvh", [1, 2, 3])
def test_fused_append_gather_equals_append_then_gather(nkvh):
    # Contexts that put the new token at a page start (0, 16, 32), a page end
    # (15, 31), mid-page, and one long sequence: same pool and output bytes as
    # the oracle's append followed by its gather.
    lens, table, k_log, v_log, kn, vn = _fused_case([0, 15, 16, 31, 32, 7, 300, 1], nkvh, 31)
    kp, vp = _dev(k_log, v_log)
    cu = np.concatenate([[0], np.cumsum(lens + 1)]).astype(np.int32)
    T = int(cu[-1])
    ko = to_llaisys(torch.zeros((T, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    vo = to_llaisys(torch.zeros((T, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    L.Ops.paged_kv_append_gather(ko, vo, kp, vp, to_llaisys(from_bits(kn)), to_llaisys(from_bits(vn)), _i32(table),
                                 _i32(lens), _i32(cu))
    assert L.device_error_flags() == 0
    assert oracle.paged_append(k_log, v_log, kn, vn, table, lens) == 0
    np.testing.assert_array_equal(_pool_logical(kp, False, k_log.shape), k_log)
    np.testing.assert_array_equal(_pool_logical(vp, True, v_log.shape), v_log)
    gk, gv = oracle.paged_gather(k_log, v_log, table, cu)
    np.testing.assert_array_equal(bits(to_torch(ko)), gk)
    np.testing.assert_array_equal(bits(to_torch(vo)), gv)


def test_fused_append_gather_config2_bit_exact():
    # BASELINE config 2 through the fused entry point.
    B, nb, nkvh = 32, 4096, 2
    seed = 0
    while True:
        lens = oracle.randint(seed, B, 1, 2048).astype(np.int32)
        if ((lens + 16) // 16).sum() <= nb:
            break
        seed += 1
    lens, table, k_log, v_log = _setup(100, lens, nb, nkvh)
    kp, vp = _dev(k_log, v_log)
    kn = oracle.f32_to_bf16(oracle.randn(7, (B, nkvh, 128)))
    vn = oracle.f32_to_bf16(oracle.randn(8, (B, nkvh, 128)))
    cu = np.concatenate([[0], np.cumsum(lens + 1)]).astype(np.int32)
    T = int(cu[-1])
    ko = to_llaisys(torch.zeros((T, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    vo = to_llaisys(torch.zeros((T, nkvh, 128), dtype=torch.bfloat16, device="cuda"))
    L.Ops.paged_kv_append_gather(ko, vo, kp, vp, to_llaisys(from_bits(kn)), to_llaisys(from_bits(vn)), _i32(table),
                                 _i32(lens), _i32(cu))
    assert L.device_error_flags() == 0
    assert oracle.paged_append(k_log, v_log, kn, vn, table, lens) == 0
    np.testing.assert_array_equal(_pool_logical(kp, False, k_log.shape), k_log)
    np.testing.assert_array_equal(_pool_logical(vp, True, v_log.shape), v_log)
    gk, gv = oracle.paged_gather(k_log, v_log, table, cu)
    np.testing.assert_array_equal(bits(to_torch(ko)), gk)
    np.testing.assert_array_equal(bits(to_torch(vo)), gv)


def test_fused_append_gather_flags_bad_rows_and_blocks():
    lens, table, k_log, v_log, kn, vn = _fused_case([20, 3], 2, 9)
    kp, vp = _dev(k_log, v_log)
    knd, vnd = to_llaisys(from_bits(kn)), to_llaisys(from_bits(vn))
    ko = to_llaisys(torch.zeros((40, 2, 128), dtype=torch.bfloat16, device="cuda"))
    vo = to_llaisys(torch.zeros((40, 2, 128), dtype=torch.bfloat16, device="cuda"))
    # 5 rows for sequence 1, whose ctx + 1 is 4: flag 2, sequence skipped, sequence 0 done
    cu = np.array([0, 21, 26], np.int32)
    L.Ops.paged_kv_append_gather(ko, vo, kp, vp, knd, vnd, _i32(table), _i32(lens), _i32(cu))
    assert L.device_error_flags() == 2
    assert oracle.paged_append(k_log, v_log, kn[:1], vn[:1], table[:1], lens[:1]) == 0
    gk, _ = oracle.paged_gather(k_log, v_log, table[:1], cu[:2])
    np.testing.assert_array_equal(bits(to_torch(ko))[:21], gk)
    # a block id outside the pool: flag 1
    bad = table.copy()
    bad[0, 1] = 1000
    L.Ops.paged_kv_append_gather(ko, vo, kp, vp, knd, vnd, _i32(bad), _i32(lens), _i32(np.array([0, 21, 25], np.int32)))
    assert L.device_error_flags() & 1
    assert L.device_error_flags() == 0
