"""llaisysPagedAttentionNoAlloc (the decode attention with its split records in
a fixed per-GPU scratch array, no device allocation) against
llaisysPagedAttention on the same inputs and against the fp32 oracle, on two
calls in a row (the second with a smaller batch), plus the size limit."""
import numpy as np
import pytest
import torch

import llaisys_amd as L
import oracle
from paged_cases import make_case, queries
from utils import from_bits, to_llaisys, to_torch

pytestmark = pytest.mark.gpu

SCALE = 1.0 / 128**0.5


def _run(case, q_bits, out_dtype, no_alloc):
    kp, vp = case.device_pools()
    table, ctx = case.device_meta()
    out = to_llaisys(torch.zeros((case.B, case.nh, 128), dtype=out_dtype, device="cuda"))
    fn = L.Ops.paged_attention_no_alloc if no_alloc else L.Ops.paged_attention
    fn(out, to_llaisys(from_bits(q_bits)), kp, vp, table, ctx, SCALE)
    assert L.device_error_flags() == 0
    return to_torch(out).float().cpu().numpy()


def test_no_alloc_matches_paged_attention_on_two_calls():
    big = make_case(71, oracle.randint(16, 64, 512, 8192).astype(np.int32))
    small = make_case(73, oracle.randint(17, 9, 1, 700).astype(np.int32))
    for name, case, seed in (("B=64 ctx U[512,8192]", big, 72), ("B=9 ctx U[1,700]", small, 74)):
        print(f"[no_alloc] {name}", flush=True)
        q = queries(seed, case.B, 12)
        ref = oracle.paged_attention(q, case.k_log, case.v_log, case.table, case.ctx, SCALE, nthreads=16)
        for dt in (torch.float32, torch.bfloat16):
            got = _run(case, q, dt, True)
            want = _run(case, q, dt, False)
            if dt == torch.float32:
                assert np.max(np.abs(got - ref)) <= 1e-4 * np.max(np.abs(ref))
                assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))
            else:
                assert np.max(np.abs(got - ref)) <= 2e-2
                assert np.max(np.abs(got - want)) <= 2 ** -7 * np.max(np.abs(want))


def test_no_alloc_refuses_a_batch_beyond_its_scratch():
    # A table 100000 pages wide: the plan's split records exceed 16 MiB and the
    # call is refused on the host, before any launch.
    case = make_case(75, np.array([20, 30, 40, 50], np.int32))
    kp, vp = case.device_pools()
    wide = np.full((4, 100000), -1, np.int32)
    wide[:, :case.table.shape[1]] = case.table
    out = to_llaisys(torch.zeros((4, 12, 128), dtype=torch.bfloat16, device="cuda"))
    q = to_llaisys(from_bits(queries(76, 4, 12)))
    with pytest.raises(L.LlaisysError, match="scratch"):
        L.Ops.paged_attention_no_alloc(out, q, kp, vp, to_llaisys(torch.from_numpy(wide)),
                                       to_llaisys(torch.from_numpy(case.ctx)), SCALE)
    assert L.device_error_flags() == 0
