"""The long steps' gate-up projection with the SwiGLU in the GEMM's epilogue
(linearSwiglu over a swigluInterleave'd weight, include/llaisys/testing.h)
against float64 torch, and bit for bit against the two-launch path it
replaces (llaisysLinear, then the swiglu op) where that path sums K in one
pass.

Bound: the gate and up sums each carry one bf16 rounding (2^-8 of their
magnitude, twice the half-ulp: the kernel rounds them before the SwiGLU) and
the fp32 accumulation term 1e-6 sqrt(K) sum |x w|; silu'(g) <= 1.1, so they
enter scaled by |up| and |silu(gate)|; the result is rounded once more. A
gate and up block from different rows, a swapped pair or a column off by a
block moves values by O(|value|), far outside."""
import ctypes

import pytest
import torch

import llaisys_amd as L
from llaisys_amd.libllaisys import LIB_LLAISYS as LIB, check_last_error
from utils import to_llaisys, to_torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
BF = torch.bfloat16


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def rnd(shape, scale, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(BF)


def interleave(w, di):
    out = torch.full_like(w, float("nan"))
    LIB.llaisysTestSwigluInterleave(ptr(out), ptr(w), di, w.shape[1])
    check_last_error()
    return out


def test_swiglu_interleave_is_a_row_permutation():
    di, K = 48, 72
    w = rnd((2 * di, K), 1.0, 1)
    got = interleave(w, di)
    blocks = torch.arange(di // 16, device=DEV)
    order = torch.stack([blocks * 16, di + blocks * 16], 1).reshape(-1)  # gate block j, up block j, ...
    rows = (order[:, None] + torch.arange(16, device=DEV)[None, :]).reshape(-1)
    assert torch.equal(got.view(torch.int16), w[rows].view(torch.int16))


SHAPES = [(1, 16, 64), (17, 48, 1536), (100, 112, 264), (333, 8960, 1536), (600, 8960, 1536), (4099, 128, 1536),
          (2048, 8960, 1536)]


@pytest.mark.parametrize("M,di,K", SHAPES, ids=[f"{m}x{d}x{k}" for m, d, k in SHAPES])
def test_linear_swiglu_against_float64(M, di, K):
    x = rnd((M, K), 1.0, M + di)
    w = rnd((2 * di, K), 0.03, K + di)
    act = torch.full((M, di), float("nan"), dtype=BF, device=DEV)
    LIB.llaisysTestLinearSwiglu(ptr(act), ptr(x), ptr(interleave(w, di)), M, di, K)
    check_last_error()
    x64, w64 = x.double(), w.double()
    g, u = x64 @ w64[:di].T, x64 @ w64[di:].T
    silu = g / (1 + torch.exp(-g))
    ref = u * silu
    xa = x64.abs()
    acc = 1e-6 * K ** 0.5
    eg = acc * (xa @ w64[:di].abs().T) + 2.0 ** -8 * g.abs()
    eu = acc * (xa @ w64[di:].abs().T) + 2.0 ** -8 * u.abs()
    bound = ref.abs() * 2.0 ** -8 + 1.1 * u.abs() * eg + silu.abs() * eu + 1e-30
    err = (act.double() - ref).abs()
    assert not torch.isnan(act).any(), "an act column was never written"
    ratio = float((err / bound).max())
    assert ratio <= 1.0, f"max |err| / bound = {ratio:.3g}"


def test_linear_swiglu_equals_linear_then_swiglu():
    # M = 2048 over 2 x 8960 columns fills the chip without a K split, so
    # llaisysLinear sums K in one pass exactly as the fused launch does: the
    # two paths agree bit for bit.
    M, di, K = 2048, 8960, 1536
    x = rnd((M, K), 1.0, 5)
    w = rnd((2 * di, K), 0.03, 6)
    gu = to_llaisys(torch.zeros((M, 2 * di), dtype=BF, device=DEV))
    L.Ops.linear(gu, to_llaisys(x), to_llaisys(w), None)
    gut = to_torch(gu)
    ref = to_llaisys(torch.zeros((M, di), dtype=BF, device=DEV))
    L.Ops.swiglu(ref, to_llaisys(gut[:, :di]), to_llaisys(gut[:, di:]))
    act = torch.full((M, di), float("nan"), dtype=BF, device=DEV)
    LIB.llaisysTestLinearSwiglu(ptr(act), ptr(x), ptr(interleave(w, di)), M, di, K)
    check_last_error()
    assert torch.equal(act.view(torch.int16), to_torch(ref).view(torch.int16))
