"""Paged decode / varlen attention on the GPU vs the fp32 C oracle
(gather + self_attention). Tolerances from BASELINE north_star: fp32 output
max|err| <= 1e-4 * max|ref|; bf16 output max|err| <= 2e-2."""
import os

import numpy as np
import pytest
import torch

import llaisys_amd as L
import oracle
from paged_cases import make_case, queries
from utils import from_bits, to_llaisys, to_torch

pytestmark = pytest.mark.gpu

SCALE = 1.0 / 128**0.5
F32_REL = 1e-4
BF16_ABS = 2e-2


def run_decode(case, q_bits, out_dtype):
    kp, vp = case.device_pools()
    table, ctx = case.device_meta()
    out = to_llaisys(torch.zeros((case.B, case.nh, 128), dtype=out_dtype, device="cuda"))
    L.Ops.paged_attention(out, to_llaisys(from_bits(q_bits)), kp, vp, table, ctx, SCALE)
    assert L.device_error_flags() == 0
    return to_torch(out).float().cpu().numpy()


def run_varlen(case, q_bits, cu_q, out_dtype):
    kp, vp = case.device_pools()
    table, ctx = case.device_meta()
    T = q_bits.shape[0]
    out = to_llaisys(torch.zeros((T, case.nh, 128), dtype=out_dtype, device="cuda"))
    L.Ops.paged_attention_varlen(out, to_llaisys(from_bits(q_bits)), kp, vp, table,
                                 to_llaisys(torch.from_numpy(cu_q)), ctx, SCALE)
    assert L.device_error_flags() == 0
    return to_torch(out).float().cpu().numpy()


def check(got_f32, got_bf16, ref):
    err = np.max(np.abs(got_f32 - ref)) / np.max(np.abs(ref))
    assert err <= F32_REL, f"fp32 relative error {err:.3g}"
    abs_err = np.max(np.abs(got_bf16 - ref))
    assert abs_err <= BF16_ABS, f"bf16 abs error {abs_err:.3g}"


@pytest.mark.parametrize("nh,nkvh", [(12, 2), (16, 1), (4, 4), (8, 2)])
def test_decode_edge_lengths(nh, nkvh):
    ctx = np.array([1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 257], np.int32)
    case = make_case(10 + nh, ctx, nh=nh, nkvh=nkvh)
    q = queries(99, case.B, nh)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE)
    check(run_decode(case, q, torch.float32), run_decode(case, q, torch.bfloat16), ref)


@pytest.mark.parametrize("slots", ["1", "0"])
@pytest.mark.parametrize("waves", ["1", "7", "64", "1024", "5000"])
def test_decode_wave_count_invariance(waves, slots, monkeypatch):
    # The grid size only changes where sequences are cut into records: from
    # every unit whole in one wave to more waves than page pairs (empty ranges).
    ctx = oracle.randint(5, 9, 1, 3000).astype(np.int32)
    case = make_case(21, ctx)
    q = queries(22, case.B, 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE)
    monkeypatch.setenv("LLAISYS_DECODE_WAVES", waves)
    monkeypatch.setenv("LLAISYS_DECODE_SLOTS", slots)
    check(run_decode(case, q, torch.float32), run_decode(case, q, torch.bfloat16), ref)


def test_decode_record_slots_reset_between_calls(monkeypatch):
    # Split units merge through per-unit record slots whose headers the
    # combine returns to zero: calls of different batches in a row (one whose
    # long sequences overflow the slots) each match the oracle, and a repeat
    # of the first batch gives bit-identical output.
    a = make_case(51, oracle.randint(14, 64, 512, 8192).astype(np.int32))
    qa = queries(52, a.B, 12)
    ref_a = oracle.paged_attention(qa, a.k_log, a.v_log, a.table, a.ctx, SCALE, nthreads=16)
    b = make_case(53, np.array([30000, 40], np.int32))  # one unit spread over many waves: overflow
    qb = queries(54, b.B, 12)
    ref_b = oracle.paged_attention(qb, b.k_log, b.v_log, b.table, b.ctx, SCALE)
    c = make_case(55, oracle.randint(15, 9, 1, 3000).astype(np.int32))
    qc = queries(56, c.B, 12)
    ref_c = oracle.paged_attention(qc, c.k_log, c.v_log, c.table, c.ctx, SCALE)
    # a small batch whose units use the slots (one pair per wave), so its
    # records land where a larger batch's slot headers would sit in a shared
    # layout
    d = make_case(57, np.array([100, 150, 200, 250], np.int32))
    qd = queries(58, d.B, 12)
    ref_d = oracle.paged_attention(qd, d.k_log, d.v_log, d.table, d.ctx, SCALE)
    first = run_decode(a, qa, torch.float32)
    check(first, run_decode(a, qa, torch.bfloat16), ref_a)
    for _ in range(3):
        check(run_decode(b, qb, torch.float32), run_decode(b, qb, torch.bfloat16), ref_b)
        check(run_decode(c, qc, torch.float32), run_decode(c, qc, torch.bfloat16), ref_c)
        assert np.array_equal(run_decode(a, qa, torch.float32), first)
        check(run_decode(d, qd, torch.float32), run_decode(d, qd, torch.bfloat16), ref_d)
        assert np.array_equal(run_decode(a, qa, torch.float32), first)
    monkeypatch.setenv("LLAISYS_DECODE_SLOTS", "0")
    per_wave = run_decode(a, qa, torch.float32)
    assert np.max(np.abs(per_wave - first)) <= 1e-6 * np.max(np.abs(first))


@pytest.mark.parametrize("stages", ["2", "3"])
def test_decode_ring_depth(stages, monkeypatch):
    ctx = oracle.randint(6, 11, 1, 2000).astype(np.int32)
    case = make_case(23, ctx)
    q = queries(24, case.B, 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE)
    monkeypatch.setenv("LLAISYS_DECODE_STAGES", stages)
    check(run_decode(case, q, torch.float32), run_decode(case, q, torch.bfloat16), ref)


@pytest.mark.parametrize("pps", ["2", "16", "64"])
def test_varlen_split_invariance(pps, monkeypatch):
    ctx = oracle.randint(7, 6, 20, 2500).astype(np.int32)
    lq = np.array([1, 5, 1, 20, 1, 3], np.int32)
    case = make_case(25, ctx)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = queries(26, int(cu_q[-1]), 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, cu_q=cu_q)
    monkeypatch.setenv("LLAISYS_PAGES_PER_SPLIT", pps)
    check(run_varlen(case, q, cu_q, torch.float32), run_varlen(case, q, cu_q, torch.bfloat16), ref)


@pytest.mark.parametrize("pps", ["2", "16", "64"])
def test_prefill_work_queue_matches_one_workgroup_per_split(pps, monkeypatch):
    # The persistent prefill kernel (item tables built in LDS, items taken
    # from a device counter, full splits first) runs the same per-item code
    # as the kernel with one workgroup per (block, split) grid slot: outputs
    # are bit-identical, also over repeated calls (the counter and the done
    # count return to zero at the end of each launch).
    ctx = np.array([700, 33, 1300, 90, 2049, 18], np.int32)
    lq = np.array([300, 1, 257, 90, 2, 18], np.int32)
    case = make_case(27, ctx)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = queries(28, int(cu_q[-1]), 12)
    monkeypatch.setenv("LLAISYS_PAGES_PER_SPLIT", pps)
    monkeypatch.setenv("LLAISYS_PREFILL_QUEUE", "0")
    grid = [run_varlen(case, q, cu_q, dt) for dt in (torch.float32, torch.bfloat16)]
    monkeypatch.setenv("LLAISYS_PREFILL_QUEUE", "1")
    for _ in range(3):
        for dt, want in zip((torch.float32, torch.bfloat16), grid):
            assert np.array_equal(run_varlen(case, q, cu_q, dt), want)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, cu_q=cu_q)
    check(grid[0], grid[1], ref)


def test_prefill_kernel_takes_decode_sequences(monkeypatch):
    # The persistent prefill kernel also runs a mixed batch's single-query
    # sequences (one item per kv head, all 8 waves, LDS merge) instead of the
    # stream-K decode kernel: same results to fp32 rounding, repeated calls
    # bit-identical, and a single-query sequence with an invalid length still
    # raises error bit 2 and leaves its row alone.
    ctx = np.array([700, 33, 1300, 1, 2049, 18, 4000, 250], np.int32)
    lq = np.array([300, 1, 257, 1, 2, 1, 1, 1], np.int32)
    case = make_case(35, ctx)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = queries(36, int(cu_q[-1]), 12)
    monkeypatch.setenv("LLAISYS_PREFILL_TAKES_DECODE", "0")
    base = [run_varlen(case, q, cu_q, dt) for dt in (torch.float32, torch.bfloat16)]
    monkeypatch.setenv("LLAISYS_PREFILL_TAKES_DECODE", "1")
    got = [run_varlen(case, q, cu_q, dt) for dt in (torch.float32, torch.bfloat16)]
    assert np.max(np.abs(got[0] - base[0])) <= 1e-5 * np.max(np.abs(base[0]))
    assert np.max(np.abs(got[1] - base[1])) <= BF16_ABS
    assert np.array_equal(run_varlen(case, q, cu_q, torch.float32), got[0])
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, cu_q=cu_q)
    check(got[0], got[1], ref)
    # sequence 5 (one query) with length 0: flagged, its output row untouched
    bad = ctx.copy()
    bad[5] = 0
    kp, vp = case.device_pools()
    table, _ = case.device_meta()
    out = to_llaisys(torch.full((int(cu_q[-1]), 12, 128), 7.0, dtype=torch.float32, device="cuda"))
    L.Ops.paged_attention_varlen(out, to_llaisys(from_bits(q)), kp, vp, table, to_llaisys(torch.from_numpy(cu_q)),
                                 to_llaisys(torch.from_numpy(bad)), SCALE)
    assert L.device_error_flags() & 2
    o = to_torch(out).cpu().numpy()
    assert np.all(o[cu_q[5]] == 7.0)
    rows = np.r_[cu_q[0]:cu_q[5], cu_q[6]:cu_q[-1]]
    assert np.array_equal(o[rows], got[0][rows])


@pytest.mark.parametrize("nseq", [300, 1100])
def test_varlen_large_mixed_batches(nseq):
    # Past 256 sequences the single queries go back to the stream-K decode
    # kernel beside the persistent prefill kernel; past 1024 the prefill runs
    # one workgroup per grid slot (its item tables no longer fit in LDS).
    ctx = oracle.randint(37, nseq, 20, 120).astype(np.int32)
    lq = np.ones(nseq, np.int32)
    lq[::97] = np.minimum(ctx[::97], 17)  # a few multi-query sequences
    case = make_case(38, ctx)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = queries(39, int(cu_q[-1]), 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, cu_q=cu_q, nthreads=16)
    check(run_varlen(case, q, cu_q, torch.float32), run_varlen(case, q, cu_q, torch.bfloat16), ref)


def test_prefill_bad_geometry_flags_error():
    # A multi-query sequence with more new tokens than context (Lq > ctx) is
    # skipped with error bit 2; the other sequences' rows come out as when
    # that sequence is valid.
    ctx = np.array([64, 10, 80], np.int32)
    lq = np.array([16, 12, 20], np.int32)
    case = make_case(29, ctx)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = to_llaisys(from_bits(queries(30, int(cu_q[-1]), 12)))
    kp, vp = case.device_pools()
    table, _ = case.device_meta()
    rows = np.r_[cu_q[0]:cu_q[1], cu_q[2]:cu_q[3]]
    outs = []
    for c1 in (10, 12):  # 12 new tokens over a 10-token context, then over 12
        out = to_llaisys(torch.zeros((int(cu_q[-1]), 12, 128), dtype=torch.float32, device="cuda"))
        c = ctx.copy()
        c[1] = c1
        L.Ops.paged_attention_varlen(out, q, kp, vp, table, to_llaisys(torch.from_numpy(cu_q)),
                                     to_llaisys(torch.from_numpy(c)), SCALE)
        flags = L.device_error_flags()
        assert bool(flags & 2) == (c1 == 10)
        outs.append(to_torch(out).cpu().numpy()[rows])
    assert np.array_equal(outs[0], outs[1])


def test_decode_ignores_stale_nan_slots():
    ctx = np.array([5, 16, 33, 70, 129], np.int32)
    case = make_case(31, ctx, stale_nan=True, extra_pages=2)
    q = queries(32, case.B, 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE)
    got = run_decode(case, q, torch.float32)
    assert np.isfinite(got).all()
    check(got, run_decode(case, q, torch.bfloat16), ref)


def test_config3_batch64_decode():
    # B=64, ctx U[512, 8192], 12:2 GQA, d=128, bf16.
    ctx = oracle.randint(0, 64, 512, 8192).astype(np.int32)
    case = make_case(40, ctx)
    q = queries(41, 64, 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, nthreads=16)
    check(run_decode(case, q, torch.float32), run_decode(case, q, torch.bfloat16), ref)


def test_varlen_small_mixed_batch():
    ctx = np.array([40, 7, 100, 1, 35, 64], np.int32)
    lq = np.array([40, 3, 17, 1, 1, 16], np.int32)  # new tokens already in the cache
    case = make_case(50, ctx)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = queries(51, int(cu_q[-1]), 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, cu_q=cu_q)
    check(run_varlen(case, q, cu_q, torch.float32), run_varlen(case, q, cu_q, torch.bfloat16), ref)


def test_varlen_with_decode_only_agrees_with_decode():
    # Same math through the two kernels (varlen tiles vs decode stream-K).
    ctx = oracle.randint(55, 7, 1, 900).astype(np.int32)
    case = make_case(56, ctx)
    q = queries(57, case.B, 12)
    cu_q = np.arange(case.B + 1, dtype=np.int32)
    a = run_varlen(case, q, cu_q, torch.float32)
    b = run_decode(case, q, torch.float32)
    assert np.max(np.abs(a - b)) <= 1e-5 * np.max(np.abs(b))


def test_config4_mixed_prefill_and_decode():
    # 4 chunks of 512 over priors {0,1024,2048,4096} + 60 decode, ctx U[256,4096].
    priors = np.array([0, 1024, 2048, 4096], np.int32)
    dec = oracle.randint(60, 60, 256, 4096).astype(np.int32)
    ctx = np.concatenate([priors + 512, dec]).astype(np.int32)
    lq = np.concatenate([np.full(4, 512), np.ones(60)]).astype(np.int32)
    case = make_case(61, ctx)
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = queries(62, int(cu_q[-1]), 12)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, cu_q=cu_q, nthreads=16)
    check(run_varlen(case, q, cu_q, torch.float32), run_varlen(case, q, cu_q, torch.bfloat16), ref)


def test_paged_attention_equals_self_attention_of_gather():
    ctx = np.array([300, 17, 1024], np.int32)
    case = make_case(70, ctx)
    q = queries(71, case.B, 12)
    got = run_decode(case, q, torch.float32)
    kp, vp = case.device_pools()
    table, _ = case.device_meta()
    cu = np.concatenate([[0], np.cumsum(ctx)]).astype(np.int32)
    ko = to_llaisys(torch.zeros((int(cu[-1]), 2, 128), dtype=torch.bfloat16, device="cuda"))
    vo = to_llaisys(torch.zeros((int(cu[-1]), 2, 128), dtype=torch.bfloat16, device="cuda"))
    L.Ops.paged_kv_gather(ko, vo, kp, vp, table, to_llaisys(torch.from_numpy(cu)))
    kt, vt = to_torch(ko).float(), to_torch(vo).float()
    qt = from_bits(q).float()
    for b in range(case.B):
        o = to_llaisys(torch.zeros((1, 12, 128), device="cuda"))
        L.Ops.self_attention(o, to_llaisys(qt[b:b + 1]), to_llaisys(kt[cu[b]:cu[b + 1]]),
                             to_llaisys(vt[cu[b]:cu[b + 1]]), SCALE)
        sa = to_torch(o).cpu().numpy()[0]
        assert np.max(np.abs(sa - got[b])) <= F32_REL * np.max(np.abs(sa))


def test_bad_block_id_and_overlong_context_flag_errors():
    ctx = np.array([40, 20], np.int32)
    case = make_case(80, ctx)
    kp, vp = case.device_pools()
    bad = case.table.copy()
    bad[1, 0] = 10 ** 6
    out = to_llaisys(torch.zeros((2, 12, 128), dtype=torch.bfloat16, device="cuda"))
    q = to_llaisys(from_bits(queries(81, 2, 12)))
    L.Ops.paged_attention(out, q, kp, vp, to_llaisys(torch.from_numpy(bad)),
                          to_llaisys(torch.from_numpy(ctx)), SCALE)
    assert L.device_error_flags() & 1
    long_ctx = np.array([40, 16 * case.table.shape[1] + 1], np.int32)
    L.Ops.paged_attention(out, q, kp, vp, to_llaisys(torch.from_numpy(case.table)),
                          to_llaisys(torch.from_numpy(long_ctx)), SCALE)
    assert L.device_error_flags() & 2


def spread_case(seed, ctx, nh=12, nkvh=2):
    """Scores that differ by far more than fp32's exponent range within every
    page: keys in slots 4-15 of a page have a dot product with q about 2^8
    larger (in exp2 units) than those in slots 0-3. A softmax whose running
    max leaves out any of a page's key groups overflows exp2 to inf on such
    keys; the normalised result is the mean of V over the largest keys."""
    case = make_case(seed, np.asarray(ctx, np.int32), nh=nh, nkvh=nkvh)
    big = np.zeros(16, bool)
    big[4:] = True
    k = oracle.bf16_to_f32(case.k_log) * 0.25
    k[:, :, big, :] += 12.0
    case.k_log[:] = oracle.f32_to_bf16(k)
    q = oracle.f32_to_bf16(np.abs(oracle.randn(seed + 5, (case.B, nh, 128))) * 0.5 + 1.0)
    return case, q


@pytest.mark.parametrize("ctx", [[40, 300, 1000], [16, 17, 2049]])
def test_decode_softmax_max_covers_every_key_group(ctx):
    case, q = spread_case(77, ctx)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE)
    got32, got16 = run_decode(case, q, torch.float32), run_decode(case, q, torch.bfloat16)
    assert np.isfinite(got32).all() and np.isfinite(got16).all()
    check(got32, got16, ref)


def test_varlen_softmax_max_covers_every_key_group():
    # one prefill chunk of 40 queries over 300 prior tokens, plus two decodes
    ctx = np.array([340, 200, 1000], np.int32)
    case, _ = spread_case(78, ctx)
    lq = np.array([40, 1, 1])
    cu_q = np.concatenate([[0], np.cumsum(lq)]).astype(np.int32)
    q = oracle.f32_to_bf16(np.abs(oracle.randn(83, (int(cu_q[-1]), 12, 128))) * 0.5 + 1.0)
    ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, cu_q=cu_q)
    got32 = run_varlen(case, q, cu_q, torch.float32)
    got16 = run_varlen(case, q, cu_q, torch.bfloat16)
    assert np.isfinite(got32).all() and np.isfinite(got16).all()
    check(got32, got16, ref)
