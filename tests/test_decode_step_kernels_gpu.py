"""Kernel-level parity of the decode step's fused packed-operand kernels
(include/llaisys/testing.h): each kernel alone against float64 torch.

The bound everywhere is the one test_model_ops_gpu.py's decode-GEMM tests use:
one bf16 rounding of the result (2^-8 of its magnitude, twice the half-ulp)
plus an fp32 accumulation term 1e-6 sqrt(K) times the sum of |products|. The
epilogues add their own terms, each stated where it enters:
* RMSNorm factor r: computed in fp32 from the bf16 row (relative 1e-6).
* RoPE: the angle pos / theta^(2j/128) in fp32 (relative ~2^-23, so ~2.5e-4
  rad at position 2048): 1e-6 * pos times the pair's magnitude.
* SwiGLU: silu'(g) <= 1.1, so errors of gate and up enter scaled by |up| and
  |silu(gate)|.
A wrong tile, a transposed operand, a RoPE pair or position off by one, or a
k/v token in the wrong page slot moves values by O(|value|), far outside.
Page slots: every byte of the pools is checked; the rows the kernel appended
must sit where the oracle's paged_append (oracle/oracle.c) puts the same
values, and nothing else may change.
Rows: M in {1, 17, 64, 100, 128} (partial 16- and 32-row tiles)."""
import ctypes

import numpy as np
import pytest
import torch

import llaisys_amd as L
import oracle
from llaisys_amd.libllaisys import LIB_LLAISYS as LIB, check_last_error

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
BF = torch.bfloat16
HS, NH, NKVH, DH, DI = 1536, 12, 2, 128, 8960
MS = [1, 17, 64, 100, 128]


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def rnd(shape, scale, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(BF)


def packed_index(R, K):
    r = np.arange(R)[:, None]
    k = np.arange(K)[None, :]
    idx = ((r // 16) * (K // 32) + k // 32) * 512 + ((r % 16) + 16 * ((k // 8) % 4)) * 8 + k % 8
    return torch.from_numpy(idx.reshape(-1)).to(DEV)


def pack_rows(x):
    R, K = x.shape
    buf = torch.zeros(((R + 15) // 16) * 16 * K, dtype=x.dtype, device=DEV)
    buf[packed_index(R, K)] = x.reshape(-1)
    return buf


def unpack_rows(buf, R, K):
    return buf[packed_index(R, K)].reshape(R, K)


def pack_weight(w, fold_g=None):
    N, K = w.shape
    out = torch.empty_like(w)
    LIB.llaisysTestPackWeight(ptr(out), ptr(w), ptr(fold_g), N, K)
    check_last_error()
    return out


def acc_term(xa, wa, K):
    # fp32 accumulation of K products: 1e-6 sqrt(K) sum |x w|
    return 1e-6 * K ** 0.5 * (xa @ wa.T)


def assert_within(got, ref, bound, what):
    err = (got - ref).abs()
    ratio = float((err / bound).max())
    assert ratio <= 1.0, f"{what}: max |err| / bound = {ratio:.3g} (max |err| {float(err.max()):.3g})"


def rms(x64, eps):
    return 1.0 / torch.sqrt((x64 ** 2).mean(-1, keepdim=True) + eps)


@pytest.mark.parametrize("M", MS)
@pytest.mark.parametrize("accumulate", [False, True])
def test_packed_x_gemm(M, accumulate):
    # The o projection of the step: y (+)= x W^T over packed x and W, y also
    # written packed for the next kernel.
    K, N = HS, HS
    x, w = rnd((M, K), 0.5, M), rnd((N, K), 0.05, M + 1)
    y0 = rnd((M, N), 1.0, M + 2)
    y = y0.clone()
    yp = torch.full((((M + 15) // 16) * 16 * N,), float("nan"), dtype=BF, device=DEV)
    LIB.llaisysTestPackedXGemm(ptr(y), ptr(pack_rows(x)), ptr(pack_weight(w)), M, N, K, int(accumulate), ptr(yp))
    check_last_error()
    x64, w64 = x.double(), w.double()
    ref = x64 @ w64.T + (y0.double() if accumulate else 0)
    bound = ref.abs() * 2.0 ** -8 + acc_term(x64.abs(), w64.abs(), K) + 1e-30
    assert_within(y.double(), ref, bound, "packedXGemm")
    assert torch.equal(unpack_rows(yp, M, N).view(torch.int16), y.view(torch.int16)), "packed copy of y differs"


@pytest.mark.parametrize("M", MS)
@pytest.mark.parametrize("act_packed", [False, True])
def test_gate_up_swiglu(M, act_packed):
    # act = up * silu(gate) of r (x [gate; up]^T), the RMSNorm weight g folded
    # into the columns of the packed weight (one bf16 rounding of W * g).
    K, eps = HS, 1e-6
    x = rnd((M, K), 1.0, 10 + M)
    w = rnd((2 * DI, K), 0.02, 11)
    g = (1.0 + 0.1 * torch.randn(K, generator=torch.Generator(device=DEV).manual_seed(12), device=DEV)).to(BF)
    wf = (w.float() * g.float()).to(BF)  # the fold, rounded once as the model does
    wp = torch.empty_like(wf)
    LIB.llaisysTestPackWeightGateUp(ptr(wp), ptr(wf), DI, K)
    check_last_error()
    if act_packed:
        act = torch.full((((M + 15) // 16) * 16 * DI,), float("nan"), dtype=BF, device=DEV)
    else:
        act = torch.full((M, DI), float("nan"), dtype=BF, device=DEV)
    LIB.llaisysTestGateUpSwiglu(ptr(act), ptr(pack_rows(x)), ptr(wp), M, DI, K, eps, int(act_packed))
    check_last_error()
    got = (unpack_rows(act, M, DI) if act_packed else act).double()
    x64, w64 = x.double(), wf.double()
    r = rms(x64, eps)
    gl, ul = r * (x64 @ w64[:DI].T), r * (x64 @ w64[DI:].T)
    silu = gl / (1 + torch.exp(-gl))
    ref = ul * silu
    xa = x64.abs()
    eg = r * acc_term(xa, w64[:DI].abs(), K) + 2e-6 * gl.abs()
    eu = r * acc_term(xa, w64[DI:].abs(), K) + 2e-6 * ul.abs()
    bound = ref.abs() * 2.0 ** -8 + 1.1 * ul.abs() * eg + silu.abs() * eu + 1e-30
    assert_within(got, ref, bound, "gateUpSwiglu")


@pytest.mark.parametrize("M", MS)
@pytest.mark.parametrize("accumulate", [True, False])
def test_split_k_packed_gemm(M, accumulate):
    # The down projection: K = 8960 split over workgroups, fp32 partials summed
    # in a fixed order by the reduce, which adds the residual and also writes y
    # packed. Twice: the second call must not depend on the first's partials.
    K, N = DI, HS
    x, w = rnd((M, K), 0.5, 20 + M), rnd((N, K), 0.02, 21)
    y0 = rnd((M, N), 1.0, 22)
    xp, wp = pack_rows(x), pack_weight(w)
    x64, w64 = x.double(), w.double()
    ref = x64 @ w64.T + (y0.double() if accumulate else 0)
    bound = ref.abs() * 2.0 ** -8 + acc_term(x64.abs(), w64.abs(), K) + 1e-30
    first = None
    for _ in range(2):
        y = y0.clone()
        yp = torch.full((((M + 15) // 16) * 16 * N,), float("nan"), dtype=BF, device=DEV)
        LIB.llaisysTestSplitKPackedGemm(ptr(y), ptr(xp), ptr(wp), M, N, K, int(accumulate), ptr(yp))
        check_last_error()
        assert_within(y.double(), ref, bound, "splitKPackedGemm")
        assert torch.equal(unpack_rows(yp, M, N).view(torch.int16), y.view(torch.int16))
        if first is None:
            first = y.clone()
        else:
            assert torch.equal(first.view(torch.int16), y.view(torch.int16)), "split-K result differs between calls"


def rope64(v, pos, theta):
    # test/ops/rope.py:11-33 in float64: pairs (j, j + 64) turned by pos / theta^(2j/128)
    j = torch.arange(64, dtype=torch.float64, device=DEV)
    phi = pos.double()[:, None, None] / theta ** (2 * j / DH)
    a, b = v[..., :64], v[..., 64:]
    return torch.cat([a * torch.cos(phi) - b * torch.sin(phi), b * torch.cos(phi) + a * torch.sin(phi)], -1)


@pytest.mark.parametrize("M", MS)
def test_qkv_rope_gemm(M):
    # y = r (x W'^T) + bias over the fused [q; k; v] weight (RMSNorm weight
    # folded in); q and k heads rotated at each row's position; q to q[M, 12,
    # 128], the new token's k and v into its page slot.
    K, eps, theta = HS, 1e-6, 10000.0
    NQKV = (NH + 2 * NKVH) * DH
    x = rnd((M, K), 1.0, 30 + M)
    w = rnd((NQKV, K), 0.02, 31)
    g = (1.0 + 0.1 * torch.randn(K, generator=torch.Generator(device=DEV).manual_seed(32), device=DEV)).to(BF)
    bias = rnd((NQKV,), 0.5, 33)
    wf = (w.float() * g.float()).to(BF)
    # Each row m: a sequence at position pos[m] (0, page boundaries, long);
    # table over a permuted pool, pools filled with seeded values.
    rng = np.random.default_rng(34 + M)
    pos = rng.integers(0, 2100, M).astype(np.int32)
    pos[:min(M, 4)] = [0, 15, 16, 2047][:min(M, 4)]
    maxp = int(pos.max()) // 16 + 1
    nb = M * maxp + 3
    perm = oracle.permutation(35 + M, nb)
    table = perm[:M * maxp].reshape(M, maxp).astype(np.int32)
    k_log = oracle.f32_to_bf16(oracle.randn(36, (nb, NKVH, 16, DH)))
    v_log = oracle.f32_to_bf16(oracle.randn(37, (nb, NKVH, 16, DH)))
    to_dev = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(DEV)
    kp, vp = to_dev(oracle.pack_pages_np(k_log, False)), to_dev(oracle.pack_pages_np(v_log, True))
    t_table, t_pos = torch.from_numpy(table).to(DEV), torch.from_numpy(pos).to(DEV)
    q = torch.full((M, NH, DH), float("nan"), dtype=BF, device=DEV)
    LIB.llaisysTestQkvRopeGemm(ptr(q), ptr(kp), ptr(vp), ptr(pack_rows(x)), ptr(pack_weight(wf)), ptr(bias),
                               ptr(t_table), ptr(t_pos), M, NH, NKVH, K, maxp, nb, eps, theta)
    check_last_error()
    assert L.device_error_flags() == 0

    x64, w64 = x.double(), wf.double()
    r = rms(x64, eps)
    lin = x64 @ w64.T
    pre = r * lin + bias.double()
    e_pre = r * acc_term(x64.abs(), w64.abs(), K) + 2e-6 * (r * lin).abs()  # + r's own fp32 error
    heads = pre.view(M, NH + 2 * NKVH, DH)
    e_heads = e_pre.view(M, NH + 2 * NKVH, DH)
    t_pos64 = torch.from_numpy(pos.astype(np.int64)).to(DEV)
    rot = rope64(heads[:, :NH + NKVH], t_pos64, theta)
    # rotation error: the two inputs' errors, plus the angle's fp32 error
    # (1e-6 pos rad) times the pair's magnitude
    e_rot = e_heads[:, :NH + NKVH]
    e_rot = torch.cat([e_rot[..., :64] + e_rot[..., 64:]] * 2, -1)
    mag = torch.cat([heads[:, :NH + NKVH, :64].abs() + heads[:, :NH + NKVH, 64:].abs()] * 2, -1)
    e_rot = e_rot + 1e-6 * (t_pos64.double()[:, None, None] + 1) * mag
    ref_q, e_q = rot[:, :NH], e_rot[:, :NH]
    assert_within(q.double(), ref_q, ref_q.abs() * 2.0 ** -8 + e_q + 1e-30, "qkvRopeGemm q")

    # The pools: the kernel's k/v rows must sit exactly where paged_append
    # puts them, every other byte unchanged.
    k_got = oracle.unpack_pages_np(kp.cpu().numpy().view(np.uint16).reshape(nb, NKVH, 16, DH), False)
    v_got = oracle.unpack_pages_np(vp.cpu().numpy().view(np.uint16).reshape(nb, NKVH, 16, DH), True)
    k_new = np.stack([k_got[table[m, pos[m] // 16], :, pos[m] % 16] for m in range(M)])  # [M, nkvh, 128]
    v_new = np.stack([v_got[table[m, pos[m] // 16], :, pos[m] % 16] for m in range(M)])
    k_exp, v_exp = k_log.copy(), v_log.copy()
    assert oracle.paged_append(k_exp, v_exp, k_new, v_new, table, pos) == 0
    assert np.array_equal(k_got, k_exp), "k pool bytes differ from the oracle's append of the kernel's rows"
    assert np.array_equal(v_got, v_exp), "v pool bytes differ from the oracle's append of the kernel's rows"
    # ... and their values are the reference's k (rotated) and v
    kb = torch.from_numpy(oracle.bf16_to_f32(k_new)).to(DEV).double()
    vb = torch.from_numpy(oracle.bf16_to_f32(v_new)).to(DEV).double()
    ref_k, e_k = rot[:, NH:], e_rot[:, NH:]
    ref_v, e_v = heads[:, NH + NKVH:], e_heads[:, NH + NKVH:]
    assert_within(kb, ref_k, ref_k.abs() * 2.0 ** -8 + e_k + 1e-30, "qkvRopeGemm k")
    assert_within(vb, ref_v, ref_v.abs() * 2.0 ** -8 + e_v + 1e-30, "qkvRopeGemm v")


def test_qkv_rope_gemm_flags_a_bad_block_and_leaves_the_pool():
    # A table entry outside the pool raises bit 1 and writes nothing.
    M, K = 4, HS
    NQKV = (NH + 2 * NKVH) * DH
    x, wf, bias = rnd((M, K), 1.0, 40), rnd((NQKV, K), 0.02, 41), rnd((NQKV,), 0.5, 42)
    nb, maxp = 8, 2
    table = torch.tensor([[0, 1], [2, 3], [99, 4], [5, 6]], dtype=torch.int32, device=DEV)
    pos = torch.tensor([3, 17, 5, 20], dtype=torch.int32, device=DEV)
    kp = torch.zeros(nb * NKVH * 16 * DH, dtype=torch.int16, device=DEV)
    vp = torch.zeros_like(kp)
    q = torch.zeros((M, NH, DH), dtype=BF, device=DEV)
    L.device_error_flags()
    LIB.llaisysTestQkvRopeGemm(ptr(q), ptr(kp), ptr(vp), ptr(pack_rows(x)), ptr(pack_weight(wf)), ptr(bias),
                               ptr(table), ptr(pos), M, NH, NKVH, K, maxp, nb, 1e-6, 10000.0)
    check_last_error()
    assert L.device_error_flags() & 1
    kpg = kp.view(nb, NKVH, 16 * DH)
    # rows 0, 1, 3 appended into blocks 0, 3 (pos 17 -> page 1) and 6; nothing else
    touched = {0, 3, 6}
    for b in range(nb):
        assert bool(kpg[b].any()) == (b in touched), b
