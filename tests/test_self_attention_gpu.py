"""llaisysSelfAttention on the AMD device vs the reference's own torch formula
(test/ops/self_attention.py:11-28, shapes :71-75, tolerances :76-81) and vs the
fp32 C oracle."""
import numpy as np
import pytest
import torch

import llaisys_amd as L
import oracle
from utils import to_llaisys, to_torch

pytestmark = pytest.mark.gpu

DTYPES = [(torch.float32, 1e-5, 1e-5), (torch.float16, 1e-3, 1e-3), (torch.bfloat16, 1e-2, 1e-2)]


def torch_self_attention(query, key, value, scale):
    # test/ops/self_attention.py:11-28, computed in the input dtype as there.
    query, key, value = (x.transpose(-2, -3) for x in (query, key, value))
    Lq, S = query.size(-2), key.size(-2)
    bias = torch.zeros(Lq, S, dtype=query.dtype, device=query.device)
    mask = torch.ones(Lq, S, dtype=torch.bool, device=query.device).tril(diagonal=S - Lq)
    bias.masked_fill_(mask.logical_not(), float("-inf"))
    key = key.repeat_interleave(query.size(-3) // key.size(-3), -3)
    value = value.repeat_interleave(query.size(-3) // value.size(-3), -3)
    w = query @ key.transpose(-2, -1) * scale
    w += bias
    w = torch.softmax(w, dim=-1)
    return (w @ value).transpose(-2, -3)


def run(q, k, v, scale, dv=None):
    out = torch.zeros(q.shape[0], q.shape[1], v.shape[2], dtype=q.dtype, device=q.device)
    lo = to_llaisys(out)
    L.Ops.self_attention(lo, to_llaisys(q), to_llaisys(k), to_llaisys(v), scale)
    return to_torch(lo)


@pytest.mark.parametrize("shape", [(2, 2, 1, 1, 4), (5, 11, 4, 2, 8)])
@pytest.mark.parametrize("dtype,atol,rtol", DTYPES)
def test_reference_shapes_and_tolerances(shape, dtype, atol, rtol):
    qlen, kvlen, nh, nkvh, hd = shape
    g = torch.Generator(device="cuda").manual_seed(hash(shape) % 1000)
    q = torch.rand((qlen, nh, hd), generator=g, device="cuda").to(dtype)
    k = torch.rand((kvlen, nkvh, hd), generator=g, device="cuda").to(dtype)
    v = torch.rand((kvlen, nkvh, hd), generator=g, device="cuda").to(dtype)
    scale = 1.0 / hd**0.5
    got = run(q, k, v, scale)
    want = torch_self_attention(q, k, v, scale)
    assert torch.allclose(got, want, atol=atol, rtol=rtol)


@pytest.mark.parametrize("L_,S,nh,nkvh,d,dv", [
    (1, 513, 12, 2, 128, 128),
    (17, 300, 12, 2, 128, 128),
    (9, 9, 4, 4, 64, 64),
    (3, 130, 8, 1, 256, 256),
    (6, 20, 6, 3, 32, 48),
    (40, 1000, 12, 2, 128, 128),  # many key chunks per wave
    (2, 70, 2, 1, 64, 128),
])
def test_against_fp32_oracle(L_, S, nh, nkvh, d, dv):
    qn = oracle.randn(1, (L_, nh, d))
    kn = oracle.randn(2, (S, nkvh, d))
    vn = oracle.randn(3, (S, nkvh, dv))
    scale = 1.0 / d**0.5
    ref = oracle.self_attention(qn, kn, vn, scale)
    got = run(torch.from_numpy(qn).cuda(), torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda(), scale)
    err = np.max(np.abs(got.cpu().numpy() - ref)) / np.max(np.abs(ref))
    assert err <= 1e-5, err
    # bf16 inputs: widened exactly for the oracle; output rounded once.
    qb, kb, vb = (torch.from_numpy(x).cuda().to(torch.bfloat16) for x in (qn, kn, vn))
    refb = oracle.self_attention(qb.float().cpu().numpy(), kb.float().cpu().numpy(), vb.float().cpu().numpy(), scale)
    gotb = run(qb, kb, vb, scale).float().cpu().numpy()
    assert np.max(np.abs(gotb - refb)) <= 2e-2
