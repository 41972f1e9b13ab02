"""The reference's model ops on the AMD device, against a plain torch fp32
statement of each formula rounded once to the tensor dtype. Shapes and
tolerances follow the reference's test/ops/*.py (add.py:47-53, argmax.py:45-46,
embedding.py:48-57, linear.py:54-63, rms_norm.py:51-57, rope.py:69-76,
swiglu.py:47-53)."""
import pytest
import torch

import llaisys_amd as L
from llaisys_amd import DataType, DeviceType
from utils import to_llaisys, to_torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
DTYPES = [(torch.float32, 1e-5, 1e-5), (torch.float16, 1e-3, 1e-3), (torch.bfloat16, 1e-2, 1e-2)]
IDS = ["f32", "f16", "bf16"]


def rnd(shape, dtype, scale=1.0, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.rand(shape, generator=g, device=DEV, dtype=torch.float32) * 2 - 1).mul_(scale).to(dtype)


def empty_like_ll(t):
    return to_llaisys(torch.zeros_like(t))


def close(got, ref, atol, rtol):
    torch.testing.assert_close(got.float(), ref.float(), atol=atol, rtol=rtol)


@pytest.mark.parametrize("shape", [(2, 3), (512, 4096)])
@pytest.mark.parametrize("dtype,atol,rtol", DTYPES, ids=IDS)
def test_add(shape, dtype, atol, rtol):
    a, b = rnd(shape, dtype, seed=1), rnd(shape, dtype, seed=2)
    c = empty_like_ll(a)
    L.Ops.add(c, to_llaisys(a), to_llaisys(b))
    close(to_torch(c), (a.float() + b.float()).to(dtype), atol, rtol)


@pytest.mark.parametrize("shape", [(4,), (4096,), (151936,)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=IDS)
def test_argmax(shape, dtype):
    vals = rnd(shape, dtype, seed=3)
    idx, val = to_llaisys(torch.zeros(1, dtype=torch.int64, device=DEV)), to_llaisys(torch.zeros(1, dtype=dtype, device=DEV))
    L.Ops.argmax(idx, val, to_llaisys(vals))
    i = int(to_torch(idx)[0])
    # exact: the first index holding the maximum, and that maximum
    first = int(torch.nonzero(vals == vals.max())[0, 0])
    assert i == first
    assert to_torch(val)[0] == vals.max()


def test_argmax_rows_and_ties():
    # per-row argmax over the last dim (the batched greedy step), ties -> first index
    vals = rnd((37, 1000), torch.bfloat16, seed=4)
    vals[5, :] = 0.5
    vals[9, 10] = vals[9, 700] = 3.0
    idx = to_llaisys(torch.zeros(37, dtype=torch.int64, device=DEV))
    L.Ops.argmax(idx, None, to_llaisys(vals))
    got = to_torch(idx)
    ref = torch.tensor([int(torch.nonzero(r == r.max())[0, 0]) for r in vals], device=DEV)
    assert torch.equal(got, ref)
    assert got[5] == 0 and got[9] == 10


@pytest.mark.parametrize("n,vocab,d", [(1, 2, 3), (50, 512, 4096)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=IDS)
def test_embedding(n, vocab, d, dtype):
    w = rnd((vocab, d), dtype, seed=5)
    g = torch.Generator(device=DEV).manual_seed(6)
    idx = torch.randint(0, vocab, (n,), generator=g, device=DEV, dtype=torch.int64)
    out = to_llaisys(torch.zeros(n, d, dtype=dtype, device=DEV))
    L.Ops.embedding(out, to_llaisys(idx), to_llaisys(w))
    assert torch.equal(to_torch(out), w[idx])


def test_embedding_out_of_range_flag():
    w = rnd((8, 16), torch.float32, seed=7)
    idx = torch.tensor([1, 8], dtype=torch.int64, device=DEV)
    out = to_llaisys(torch.zeros(2, 16, device=DEV))
    L.Ops.embedding(out, to_llaisys(idx), to_llaisys(w))
    torch.cuda.synchronize()
    assert L.device_error_flags() & 4
    assert L.device_error_flags() == 0


LINEAR = [((2, 3), (2, 4), (3, 4)), ((512, 4096), (512, 4096), (4096, 4096)), ((128, 1536), (128, 1536), (1536, 1536))]


@pytest.mark.parametrize("shapes", LINEAR, ids=["tiny", "512x4096", "qwen2-1.5b-o"])
@pytest.mark.parametrize("use_bias", [True, False])
@pytest.mark.parametrize("dtype,atol,rtol", DTYPES, ids=IDS)
def test_linear(shapes, use_bias, dtype, atol, rtol):
    out_shape, x_shape, w_shape = shapes
    x, w = rnd(x_shape, dtype, 0.1, seed=8), rnd(w_shape, dtype, 0.01, seed=9)
    b = rnd((w_shape[0],), dtype, seed=10) if use_bias else None
    out = to_llaisys(torch.zeros(out_shape, dtype=dtype, device=DEV))
    L.Ops.linear(out, to_llaisys(x), to_llaisys(w), to_llaisys(b) if use_bias else None)
    ref = torch.matmul(x.double(), w.double().T)
    if use_bias:
        ref += b.double()
    # f32 through the MFMA GEMM accumulates in fp32: K=4096 sums of |x w| <= 1e-3 each
    close(to_torch(out), ref.to(dtype), atol, rtol)


@pytest.mark.parametrize("shape", [(1, 4), (512, 4096), (128, 1536)])
@pytest.mark.parametrize("dtype,atol,rtol", DTYPES, ids=IDS)
def test_rms_norm(shape, dtype, atol, rtol):
    x, w = rnd(shape, dtype, seed=11), rnd((shape[1],), dtype, seed=12)
    out = empty_like_ll(x)
    eps = 1e-5
    L.Ops.rms_norm(out, to_llaisys(x), to_llaisys(w), eps)
    xf = x.double()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.double()).to(dtype)
    close(to_torch(out), ref, atol, rtol)


def torch_rope(x, pos, theta):
    # test/ops/rope.py:11-33 in fp32
    d = x.shape[-1]
    xa, xb = x.float()[..., : d // 2], x.float()[..., d // 2 :]
    i = torch.arange(0, d // 2, dtype=torch.float32, device=x.device)
    freqs = pos.float().unsqueeze(1) / (theta ** (2 * i / d))
    s, c = freqs.sin().unsqueeze(1), freqs.cos().unsqueeze(1)
    return torch.cat([xa * c - xb * s, xb * c + xa * s], dim=-1).to(x.dtype)


@pytest.mark.parametrize("shape,se", [((2, 1, 4), (0, 2)), ((512, 4, 4096), (512, 1024)), ((64, 12, 128), (4000, 4064))])
@pytest.mark.parametrize("dtype,atol,rtol", [(torch.float32, 1e-4, 1e-4), (torch.float16, 1e-3, 1e-3), (torch.bfloat16, 1e-2, 1e-2)], ids=IDS)
def test_rope(shape, se, dtype, atol, rtol):
    x = rnd(shape, dtype, seed=13)
    pos = torch.arange(se[0], se[1], dtype=torch.int64, device=DEV)
    out = empty_like_ll(x)
    L.Ops.rope(out, to_llaisys(x), to_llaisys(pos), 10000.0)
    close(to_torch(out), torch_rope(x, pos, 10000.0), atol, rtol)


@pytest.mark.parametrize("shape", [(2, 3), (512, 4096)])
@pytest.mark.parametrize("dtype,atol,rtol", DTYPES, ids=IDS)
def test_swiglu(shape, dtype, atol, rtol):
    gate, up = rnd(shape, dtype, 4.0, seed=14), rnd(shape, dtype, seed=15)
    out = empty_like_ll(gate)
    L.Ops.swiglu(out, to_llaisys(gate), to_llaisys(up))
    g = gate.double()
    close(to_torch(out), (up.double() * g / (1 + torch.exp(-g))).to(dtype), atol, rtol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int64], ids=["f32", "bf16", "i64"])
def test_rearrange(dtype):
    src = (torch.arange(2 * 3 * 5 * 7, device=DEV) * 3 - 40).to(dtype).reshape(2, 3, 5, 7)
    lin = to_llaisys(src)
    view = lin.permute(2, 0, 3, 1)  # non-contiguous source
    out = L.Tensor((5, 2, 7, 3), dtype=view.dtype(), device=DeviceType.AMD)
    L.Ops.rearrange(out, view)
    assert torch.equal(to_torch(out), src.permute(2, 0, 3, 1).contiguous())
    # and into a strided destination
    dst = to_llaisys(torch.zeros(3, 2, 7, 5, dtype=dtype, device=DEV))
    dview = dst.permute(3, 1, 2, 0)
    L.Ops.rearrange(dview, view)
    assert torch.equal(to_torch(dst), src.permute(1, 0, 3, 2))


def test_model_ops_refuse_mixed_devices():
    # Host tensors run the CPU implementations; one op may not mix devices.
    a = L.Tensor((4,), dtype=DataType.F32, device=DeviceType.CPU)
    g = to_llaisys(torch.zeros(4, device=DEV))
    with pytest.raises(L.LlaisysError, match="different devices"):
        L.Ops.add(g, a, g)


SKINNY = [(1, 1, 64), (3, 7, 64), (5, 15, 128), (16, 16, 192), (17, 33, 1536), (64, 2048, 1536), (100, 1536, 8960),
          (128, 17920, 1536), (128, 2049, 192), (128, 151936, 128), (128, 1536, 8960), (2, 3, 8), (128, 100, 264)]


@pytest.mark.parametrize("M,N,K", SKINNY, ids=[f"{m}x{n}x{k}" for m, n, k in SKINNY])
@pytest.mark.parametrize("use_bias", [True, False])
def test_linear_bf16_decode_batches(M, N, K, use_bias):
    # Decode-sized batches: fp32 sums of exact bf16 products, bias entering
    # before the single rounding to bf16.
    x, w = rnd((M, K), torch.bfloat16, 0.5, seed=M + K), rnd((N, K), torch.bfloat16, 0.05, seed=N)
    b = rnd((N,), torch.bfloat16, seed=17) if use_bias else None
    out = to_llaisys(torch.zeros(M, N, dtype=torch.bfloat16, device=DEV))
    L.Ops.linear(out, to_llaisys(x), to_llaisys(w), to_llaisys(b) if use_bias else None)
    ref = x.double() @ w.double().T
    if use_bias:
        ref += b.double()
    got = to_torch(out).double()
    # one bf16 rounding (2^-9 relative) plus fp32 accumulation of K products
    bound = ref.abs() * 2.0 ** -8 + 1e-6 * (x.double().abs() @ w.double().abs().T) * K ** 0.5 + 1e-30
    assert ((got - ref).abs() <= bound).all(), float(((got - ref).abs() / bound).max())


# Prefill and serving shapes of the Qwen2-1.5B projections (M token rows), and
# ragged ones: together they take every tile of the GEMM planner, with and
# without a K split (fp32 partials summed by the reduce kernel).
PREFILL = [(2048, 2048, 1536), (2048, 1536, 8960), (8192, 1536, 1536), (600, 17920, 1536), (600, 1536, 1536),
           (1000, 2048, 1536), (333, 1536, 8960), (4099, 264, 1536), (2048, 17920, 1536), (7999, 1528, 1536),
           (6000, 1530, 1536), (1300, 1544, 1536), (1999, 1530, 1536), (900, 1536, 8960)]


@pytest.mark.parametrize("M,N,K", PREFILL, ids=[f"{m}x{n}x{k}" for m, n, k in PREFILL])
def test_linear_bf16_prefill_shapes(M, N, K):
    # Row-sampled float64 check (all columns of every 7th row and the last
    # row): one bf16 rounding plus fp32 accumulation, bias included.
    x, w = rnd((M, K), torch.bfloat16, 0.5, seed=M + N), rnd((N, K), torch.bfloat16, 0.05, seed=N + K)
    b = rnd((N,), torch.bfloat16, seed=29)
    out = to_llaisys(torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV))
    L.Ops.linear(out, to_llaisys(x), to_llaisys(w), to_llaisys(b))
    rows = torch.cat([torch.arange(0, M, 7, device=DEV), torch.tensor([M - 1], device=DEV)])
    xs = x[rows].double()
    ref = xs @ w.double().T + b.double()
    got = to_torch(out)[rows].double()
    bound = ref.abs() * 2.0 ** -8 + 1e-6 * (xs.abs() @ w.double().abs().T) * K ** 0.5 + 1e-30
    assert ((got - ref).abs() <= bound).all(), float(((got - ref).abs() / bound).max())


NARROW = [(8192, 1536, 1536), (1999, 1530, 1536), (900, 1536, 8960)]


@pytest.mark.parametrize("M,N,K", NARROW, ids=[f"{m}x{n}x{k}" for m, n, k in NARROW])
def test_linear_f16_narrow_tiles(M, N, K):
    # f16 through the 256 x 192 and 128 x 96 tiles (waves 48 columns wide,
    # spare W loads masked), same bound as bf16 (f16 rounds finer).
    x, w = rnd((M, K), torch.float16, 0.5, seed=M + 1), rnd((N, K), torch.float16, 0.05, seed=N + 2)
    out = to_llaisys(torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV))
    L.Ops.linear(out, to_llaisys(x), to_llaisys(w), None)
    rows = torch.cat([torch.arange(0, M, 5, device=DEV), torch.tensor([M - 1], device=DEV)])
    xs = x[rows].double()
    ref = xs @ w.double().T
    got = to_torch(out)[rows].double()
    bound = ref.abs() * 2.0 ** -8 + 1e-6 * (xs.abs() @ w.double().abs().T) * K ** 0.5 + 1e-30
    assert ((got - ref).abs() <= bound).all(), float(((got - ref).abs() / bound).max())


PACKED = [(1, 16), (7, 2048), (16, 1536), (33, 2048), (64, 4096), (100, 1536), (128, 2048), (128, 17920),
          (128, 1536), (120, 151936)]


@pytest.mark.parametrize("M,N", PACKED, ids=[f"{m}x{n}" for m, n in PACKED])
@pytest.mark.parametrize("use_bias", [True, False])
def test_linear_packed_decode_gemm(M, N, use_bias):
    # The hand-written decode GEMM (llaisysLinearPacked over a weight packed by
    # llaisysLinearPackWeight) against float64 torch, to the same bound as the
    # library path: one bf16 rounding plus fp32 accumulation.
    K = 1536
    x, w = rnd((M, K), torch.bfloat16, 0.5, seed=M + 3), rnd((N, K), torch.bfloat16, 0.05, seed=N + 5)
    b = rnd((N,), torch.bfloat16, seed=19) if use_bias else None
    packed = to_llaisys(torch.zeros(N, K, dtype=torch.bfloat16, device=DEV))
    L.Ops.linear_pack_weight(packed, to_llaisys(w))
    out = to_llaisys(torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV))
    L.Ops.linear_packed(out, to_llaisys(x), packed, to_llaisys(b) if use_bias else None)
    ref = x.double() @ w.double().T
    if use_bias:
        ref += b.double()
    got = to_torch(out).double()
    bound = ref.abs() * 2.0 ** -8 + 1e-6 * (x.double().abs() @ w.double().abs().T) * K ** 0.5 + 1e-30
    assert ((got - ref).abs() <= bound).all(), float(((got - ref).abs() / bound).max())


SPLIT_K = [(1, 1536, 8960), (16, 1536, 8960), (37, 128, 4096), (100, 1536, 8960), (128, 1536, 8960),
           (128, 256, 16384)]


@pytest.mark.parametrize("M,N,K", SPLIT_K, ids=[f"{m}x{n}x{k}" for m, n, k in SPLIT_K])
@pytest.mark.parametrize("use_bias", [True, False])
def test_linear_packed_split_k(M, N, K, use_bias):
    # Long K (the down projection's 8960): llaisysLinearPacked takes the
    # split-K kernel (fp32 partials summed in a fixed order, one rounding),
    # to the same bound as above. Twice in a row: the second call must not
    # depend on partials the first left behind.
    x, w = rnd((M, K), torch.bfloat16, 0.5, seed=M + 7), rnd((N, K), torch.bfloat16, 0.05, seed=N + K)
    b = rnd((N,), torch.bfloat16, seed=23) if use_bias else None
    packed = to_llaisys(torch.zeros(N, K, dtype=torch.bfloat16, device=DEV))
    L.Ops.linear_pack_weight(packed, to_llaisys(w))
    ref = x.double() @ w.double().T
    if use_bias:
        ref += b.double()
    bound = ref.abs() * 2.0 ** -8 + 1e-6 * (x.double().abs() @ w.double().abs().T) * K ** 0.5 + 1e-30
    first = None
    for _ in range(2):
        out = to_llaisys(torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV))
        L.Ops.linear_packed(out, to_llaisys(x), packed, to_llaisys(b) if use_bias else None)
        got = to_torch(out).double()
        assert ((got - ref).abs() <= bound).all(), float(((got - ref).abs() / bound).max())
        if first is None:
            first = got.clone()
        else:
            assert torch.equal(first, got), "split-K result differs between identical calls"


def test_linear_pack_weight_refuses_overlapping_storage():
    # The pack kernel reads W while it writes the tiled copy: in place would
    # corrupt both, so it is refused.
    w = to_llaisys(torch.zeros(64, 1536, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(L.LlaisysError, match="overlap"):
        L.Ops.linear_pack_weight(w, w)
    with pytest.raises(L.LlaisysError, match="overlap"):
        L.Ops.linear_pack_weight(w.slice(0, 16, 48), w.slice(0, 0, 32))
    # disjoint halves of one allocation are fine
    L.Ops.linear_pack_weight(w.slice(0, 32, 64), w.slice(0, 0, 32))


def test_linear_packed_refuses_unsupported_shapes():
    x = to_llaisys(torch.zeros(129, 1536, dtype=torch.bfloat16, device=DEV))
    w = to_llaisys(torch.zeros(32, 1536, dtype=torch.bfloat16, device=DEV))
    out = to_llaisys(torch.zeros(129, 32, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(L.LlaisysError, match="M <= 128"):
        L.Ops.linear_packed(out, x, w)
    # Long K needs N % 128 == 0.
    x = to_llaisys(torch.zeros(4, 8960, dtype=torch.bfloat16, device=DEV))
    w = to_llaisys(torch.zeros(48, 8960, dtype=torch.bfloat16, device=DEV))
    out = to_llaisys(torch.zeros(4, 48, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(L.LlaisysError, match="N % 128 == 0"):
        L.Ops.linear_packed(out, x, w)
