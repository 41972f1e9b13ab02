"""The library's host (LLAISYS_DEVICE_CPU) paged KV path and self_attention
through the C-ABI, against the fp32 C oracle: append and gather bit-exact
(BASELINE config 2 at full size), decode and varlen attention within the
north-star tolerances (fp32 output max|err| <= 1e-4 * max|ref|, bf16 output
max|err| <= 2e-2), self_attention at config 1, and the error bits the device
kernels raise. No GPU needed."""
import numpy as np
import pytest
import torch

import llaisys_amd as L
import oracle
from paged_cases import make_case, queries
from utils import bits, from_bits, to_llaisys, to_torch

SCALE = 1.0 / 128**0.5
F32_REL = 1e-4
BF16_ABS = 2e-2


def cpu(t: torch.Tensor):
    return to_llaisys(t, device="cpu")


def cbits(b):
    return cpu(from_bits(b, device="cpu"))


def i32(a):
    return cpu(torch.from_numpy(np.ascontiguousarray(a, np.int32)))


def pools(k_log, v_log):
    return cbits(oracle.pack_pages_np(k_log, False)), cbits(oracle.pack_pages_np(v_log, True))


def pool_logical(p, is_v, shape):
    return oracle.unpack_pages_np(bits(to_torch(p)).reshape(shape), is_v)


def table_for(seed, lens, nb, nkvh=2, extra_pages=0):
    lens = np.asarray(lens, np.int32)
    need = (lens + 16) // 16
    maxp = int(need.max(initial=1)) + extra_pages
    perm = oracle.permutation(seed, nb)
    table = np.full((len(lens), maxp), -1, np.int32)
    used = 0
    for b, p in enumerate(need):
        table[b, :p] = perm[used:used + p]
        used += p
    k_log = oracle.randint(seed + 1, nb * nkvh * 2048, 0, 65535).astype(np.uint16).reshape(nb, nkvh, 16, 128)
    v_log = oracle.randint(seed + 2, nb * nkvh * 2048, 0, 65535).astype(np.uint16).reshape(nb, nkvh, 16, 128)
    return table, k_log, v_log


def test_config2_append_then_gather_bit_exact():
    B, nb, nkvh = 32, 4096, 2
    lens = oracle.randint(0, B, 1, 2048).astype(np.int32)
    table, k_log, v_log = table_for(100, lens, nb, nkvh)
    kp, vp = pools(k_log, v_log)
    kn = oracle.f32_to_bf16(oracle.randn(7, (B, nkvh, 128)))
    vn = oracle.f32_to_bf16(oracle.randn(8, (B, nkvh, 128)))
    L.Ops.paged_kv_append(kp, vp, cbits(kn), cbits(vn), i32(table), i32(lens))
    assert L.device_error_flags() == 0
    assert oracle.paged_append(k_log, v_log, kn, vn, table, lens) == 0
    np.testing.assert_array_equal(pool_logical(kp, False, k_log.shape), k_log)
    np.testing.assert_array_equal(pool_logical(vp, True, v_log.shape), v_log)
    cu = np.concatenate([[0], np.cumsum(lens + 1)]).astype(np.int32)
    T = int(cu[-1])
    ko = cpu(torch.zeros((T, nkvh, 128), dtype=torch.bfloat16))
    vo = cpu(torch.zeros((T, nkvh, 128), dtype=torch.bfloat16))
    L.Ops.paged_kv_gather(ko, vo, kp, vp, i32(table), i32(cu))
    assert L.device_error_flags() == 0
    gk, gv = oracle.paged_gather(k_log, v_log, table, cu)
    np.testing.assert_array_equal(bits(to_torch(ko)), gk)
    np.testing.assert_array_equal(bits(to_torch(vo)), gv)


@pytest.mark.parametrize("nkvh", [1, 2, 5])
def test_ragged_prefill_append_and_fused_append_gather(nkvh):
    ctx = np.array([0, 15, 16, 3, 40, 0, 31], np.int32)
    new = np.array([5, 1, 16, 0, 33, 17, 2], np.int32)
    total = ctx + new
    nb = int(((total + 16) // 16).sum()) + 4
    table, k_log, v_log = table_for(5, total, nb, nkvh)
    kp, vp = pools(k_log, v_log)
    cu = np.concatenate([[0], np.cumsum(new)]).astype(np.int32)
    T = int(cu[-1])
    kn = oracle.randint(20, T * nkvh * 128, 0, 65535).astype(np.uint16).reshape(T, nkvh, 128)
    vn = oracle.randint(21, T * nkvh * 128, 0, 65535).astype(np.uint16).reshape(T, nkvh, 128)
    L.Ops.paged_kv_append(kp, vp, cbits(kn), cbits(vn), i32(table), i32(ctx), i32(cu))
    assert L.device_error_flags() == 0
    assert oracle.paged_append(k_log, v_log, kn, vn, table, ctx, cu) == 0
    np.testing.assert_array_equal(pool_logical(kp, False, k_log.shape), k_log)
    np.testing.assert_array_equal(pool_logical(vp, True, v_log.shape), v_log)
    # One more token per sequence, appended and gathered in one call.
    B = len(total)
    k1 = oracle.randint(30, B * nkvh * 128, 0, 65535).astype(np.uint16).reshape(B, nkvh, 128)
    v1 = oracle.randint(31, B * nkvh * 128, 0, 65535).astype(np.uint16).reshape(B, nkvh, 128)
    cug = np.concatenate([[0], np.cumsum(total + 1)]).astype(np.int32)
    Tg = int(cug[-1])
    ko = cpu(torch.zeros((Tg, nkvh, 128), dtype=torch.bfloat16))
    vo = cpu(torch.zeros((Tg, nkvh, 128), dtype=torch.bfloat16))
    L.Ops.paged_kv_append_gather(ko, vo, kp, vp, cbits(k1), cbits(v1), i32(table), i32(total), i32(cug))
    assert L.device_error_flags() == 0
    assert oracle.paged_append(k_log, v_log, k1, v1, table, total) == 0
    gk, gv = oracle.paged_gather(k_log, v_log, table, cug)
    np.testing.assert_array_equal(bits(to_torch(ko)), gk)
    np.testing.assert_array_equal(bits(to_torch(vo)), gv)
    np.testing.assert_array_equal(pool_logical(kp, False, k_log.shape), k_log)
    np.testing.assert_array_equal(pool_logical(vp, True, v_log.shape), v_log)


def test_copy_blocks_and_error_bits():
    table, k_log, v_log = table_for(9, [20, 3], 8, 2)
    kp, vp = pools(k_log, v_log)
    L.Ops.paged_kv_copy_blocks(kp, vp, i32(np.array([[1, 6], [2, 7]])))
    assert L.device_error_flags() == 0
    k_log[6], k_log[7], v_log[6], v_log[7] = k_log[1], k_log[2], v_log[1], v_log[2]
    np.testing.assert_array_equal(pool_logical(kp, False, k_log.shape), k_log)
    np.testing.assert_array_equal(pool_logical(vp, True, v_log.shape), v_log)
    kn = cpu(torch.zeros((2, 2, 128), dtype=torch.bfloat16))
    bad = table.copy()
    bad[0, 1] = 1000
    L.Ops.paged_kv_append(kp, vp, kn, kn, i32(bad), i32([20, 3]))
    assert L.device_error_flags() & 1
    L.Ops.paged_kv_append(kp, vp, kn, kn, i32(table), i32([20, 16 * table.shape[1]]))
    assert L.device_error_flags() & 2
    assert L.device_error_flags() == 0  # cleared by the read
    L.Ops.paged_kv_copy_blocks(kp, vp, i32(np.array([[0, 99]])))
    assert L.device_error_flags() == 1


def run(case, q_bits, out_dtype, cu_q=None):
    kp, vp = cbits(oracle.pack_pages_np(case.k_log, False)), cbits(oracle.pack_pages_np(case.v_log, True))
    table, ctx = i32(case.table), i32(case.ctx)
    out = cpu(torch.zeros((q_bits.shape[0], case.nh, 128), dtype=out_dtype))
    if cu_q is None:
        L.Ops.paged_attention(out, cbits(q_bits), kp, vp, table, ctx, SCALE)
    else:
        L.Ops.paged_attention_varlen(out, cbits(q_bits), kp, vp, table, i32(cu_q), ctx, SCALE)
    assert L.device_error_flags() == 0
    return to_torch(out).float().numpy()


def check(got_f32, got_bf16, ref):
    assert np.max(np.abs(got_f32 - ref)) / np.max(np.abs(ref)) <= F32_REL
    assert np.max(np.abs(got_bf16 - ref)) <= BF16_ABS


@pytest.mark.parametrize("nh,nkvh", [(12, 2), (16, 1), (4, 4)])
def test_decode_edge_lengths(nh, nkvh):
    case = make_case(10 + nh, np.array([1, 2, 15, 16, 17, 31, 32, 33, 100, 257], np.int32), nh=nh, nkvh=nkvh)
    q = queries(99, case.B, nh)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE)
    check(run(case, q, torch.float32), run(case, q, torch.bfloat16), ref)


def test_decode_config3_shape_sample():
    # config 3's shape (GQA 12:2, ctx U[512, 8192]) on 8 of its 64 sequences,
    # with NaN / -inf bytes in every unused slot.
    ctx = oracle.randint(3, 8, 512, 8192).astype(np.int32)
    case = make_case(31, ctx, stale_nan=True)
    q = queries(32, case.B, 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, nthreads=8)
    check(run(case, q, torch.float32), run(case, q, torch.bfloat16), ref)


def test_varlen_mixed_prefill_and_decode():
    ctx = np.array([600, 37, 1, 300, 1024 + 64], np.int32)
    lq = np.array([64, 1, 1, 17, 64], np.int32)
    case = make_case(41, ctx)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = queries(42, int(cu_q[-1]), 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, cu_q=cu_q, nthreads=8)
    check(run(case, q, torch.float32, cu_q), run(case, q, torch.bfloat16, cu_q), ref)


def test_attention_error_bits():
    case = make_case(61, np.array([40, 20], np.int32))
    q = queries(62, 2, 12)
    kp, vp = cbits(oracle.pack_pages_np(case.k_log, False)), cbits(oracle.pack_pages_np(case.v_log, True))
    out = cpu(torch.zeros((2, 12, 128), dtype=torch.float32))
    bad = case.table.copy()
    bad[0, 1] = 10**6
    L.Ops.paged_attention(out, cbits(q), kp, vp, i32(bad), i32(case.ctx), SCALE)
    assert L.device_error_flags() == 1
    L.Ops.paged_attention(out, cbits(q), kp, vp, i32(case.table), i32([40, 16 * case.table.shape[1] + 1]), SCALE)
    assert L.device_error_flags() == 2


@pytest.mark.parametrize("L_,S,nh,nkvh,d,dv", [
    (1, 513, 12, 2, 128, 128),
    (17, 300, 12, 2, 128, 128),
    (3, 130, 8, 1, 256, 256),
    (6, 20, 6, 3, 32, 48),
])
def test_self_attention_against_fp32_oracle(L_, S, nh, nkvh, d, dv):
    qn, kn, vn = oracle.randn(1, (L_, nh, d)), oracle.randn(2, (S, nkvh, d)), oracle.randn(3, (S, nkvh, dv))
    ref = oracle.self_attention(qn, kn, vn, 1.0 / d**0.5)
    out = cpu(torch.zeros((L_, nh, dv)))
    L.Ops.self_attention(out, cpu(torch.from_numpy(qn)), cpu(torch.from_numpy(kn)), cpu(torch.from_numpy(vn)),
                         1.0 / d**0.5)
    got = to_torch(out).numpy()
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-5

