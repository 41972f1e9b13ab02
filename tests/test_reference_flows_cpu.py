"""The reference's op tests in their default `--device cpu` flow, restated
against llaisys_amd: tensors made by torch.rand and copied into llaisys
tensors with RuntimeAPI.memcpy_sync (test/test_utils.py:5-32), the op called
through the ctypes wrapper `Ops`, and the result read back through a strided
view and compared with torch.allclose at the reference's tolerances
(test_utils.py:113-158). Shapes, dtypes and tolerances are those of
test/ops/{add,argmax,embedding,linear,rms_norm,rope,self_attention,swiglu}.py.

These run the library's host implementations (LLAISYS_DEVICE_CPU); nothing
here needs a GPU."""
import pytest
import torch

import llaisys_amd as llaisys

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "i64": torch.int64}
LDT = {"f32": llaisys.DataType.F32, "f16": llaisys.DataType.F16, "bf16": llaisys.DataType.BF16,
       "i64": llaisys.DataType.I64}
PREC = [("f32", 1e-5, 1e-5), ("f16", 1e-3, 1e-3), ("bf16", 1e-2, 1e-2)]


def _ll(t: torch.Tensor, name: str):
    lt = llaisys.Tensor(tuple(t.shape), dtype=LDT[name], device=llaisys.DeviceType.CPU)
    n = t.numel() * t.element_size()
    if n:
        llaisys.RuntimeAPI(llaisys.DeviceType.CPU).memcpy_sync(lt.data_ptr(), t.data_ptr(), n,
                                                               llaisys.MemcpyKind.D2D)
    return lt


def random_tensor(shape, name, scale=None, bias=None):
    t = torch.rand(shape, dtype=DT[name])
    if scale is not None:
        t *= scale
    if bias is not None:
        t += bias
    return t, _ll(t, name)


def check_equal(lt, ans, atol=1e-5, rtol=1e-5, strict=False):
    shape, strides = lt.shape(), lt.strides()
    assert shape == ans.shape
    right = sum(s * (n - 1) for s, n in zip(strides, shape))
    tmp = torch.zeros((right + 1,), dtype=ans.dtype)
    res = torch.as_strided(tmp, shape, strides)
    llaisys.RuntimeAPI(lt.device_type()).memcpy_sync(res.data_ptr(), lt.data_ptr(), (right + 1) * tmp.element_size(),
                                                      llaisys.MemcpyKind.D2D)
    if strict:
        return torch.equal(res, ans)
    return torch.allclose(res, ans, atol=atol, rtol=rtol)


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(0)


@pytest.mark.parametrize("shape", [(2, 3), (512, 4096)])
@pytest.mark.parametrize("name,atol,rtol", [("f32", 1e-5, 1e-5), ("f16", 1e-3, 1e-3), ("bf16", 1e-3, 1e-3)])
def test_add(shape, name, atol, rtol):  # test/ops/add.py
    a, a_ = random_tensor(shape, name)
    b, b_ = random_tensor(shape, name)
    c, c_ = random_tensor(shape, name)
    torch.add(a, b, out=c)
    llaisys.Ops.add(c_, a_, b_)
    assert check_equal(c_, c, atol, rtol)


@pytest.mark.parametrize("shape", [(4,), (4096,)])
@pytest.mark.parametrize("name", ["f32", "f16", "bf16"])
def test_argmax(shape, name):  # test/ops/argmax.py
    vals, vals_ = random_tensor(shape, name)
    mi = torch.zeros((1,), dtype=torch.int64)
    mv = torch.zeros((1,), dtype=DT[name])
    mi_, mv_ = _ll(mi, "i64"), _ll(mv, name)
    torch.max(vals, keepdim=True, dim=-1, out=(mv, mi))
    llaisys.Ops.argmax(mi_, mv_, vals_)
    assert check_equal(mv_, mv, strict=True) or check_equal(mi_, mi, strict=True)


@pytest.mark.parametrize("idx_shape,embd_shape", [((1,), (2, 3)), ((50,), (512, 4096))])
@pytest.mark.parametrize("name", ["f32", "f16", "bf16"])
def test_embedding(idx_shape, embd_shape, name):  # test/ops/embedding.py
    embd, embd_ = random_tensor(embd_shape, name)
    idx = torch.randint(0, embd_shape[0], idx_shape, dtype=torch.int64)
    idx_ = _ll(idx, "i64")
    out, out_ = random_tensor((idx_shape[0], embd_shape[1]), name)
    out[:] = embd[idx]
    llaisys.Ops.embedding(out_, idx_, embd_)
    assert check_equal(out_, out, strict=True)


@pytest.mark.parametrize("out_shape,x_shape,w_shape", [((2, 3), (2, 4), (3, 4)),
                                                       ((512, 4096), (512, 4096), (4096, 4096))])
@pytest.mark.parametrize("name,atol,rtol", PREC)
def test_linear(out_shape, x_shape, w_shape, name, atol, rtol):  # test/ops/linear.py
    x, x_ = random_tensor(x_shape, name, scale=0.1)
    w, w_ = random_tensor(w_shape, name, scale=0.01)
    b, b_ = random_tensor((w_shape[0],), name)
    out, out_ = random_tensor(out_shape, name)
    torch.nn.functional.linear(x, w, b, out=out)
    llaisys.Ops.linear(out_, x_, w_, b_)
    assert check_equal(out_, out, atol, rtol)


@pytest.mark.parametrize("shape", [(1, 4), (512, 4096)])
@pytest.mark.parametrize("name,atol,rtol", PREC)
def test_rms_norm(shape, name, atol, rtol):  # test/ops/rms_norm.py
    x, x_ = random_tensor(shape, name)
    w, w_ = random_tensor((shape[1],), name)
    ans, ans_ = random_tensor(shape, name)
    eps = 1e-5
    torch.pow(x, 2, out=ans)
    mean = torch.mean(ans, dim=-1, keepdim=True).add_(eps)
    torch.rsqrt(mean, out=mean)
    torch.mul(x, mean, out=ans)
    ans.mul_(w)
    llaisys.Ops.rms_norm(ans_, x_, w_, eps)
    assert check_equal(ans_, ans, atol, rtol)


def _torch_rope(y, x, pos, theta):
    d = y.shape[-1]
    xa, xb = x[..., : d // 2], x[..., d // 2:]
    p = pos.to(torch.float32).unsqueeze(1)
    i = torch.arange(0, d // 2, dtype=torch.float32)
    f = p / (theta ** (2 * i / d))
    s, c = f.sin().unsqueeze(1), f.cos().unsqueeze(1)
    y[..., : d // 2] = xa * c - xb * s
    y[..., d // 2:] = xb * c + xa * s


@pytest.mark.parametrize("shape,rng", [((2, 1, 4), (0, 2)), ((512, 4, 4096), (512, 1024))])
@pytest.mark.parametrize("name,atol,rtol", [("f32", 1e-4, 1e-4), ("f16", 1e-3, 1e-3), ("bf16", 1e-2, 1e-2)])
def test_rope(shape, rng, name, atol, rtol):  # test/ops/rope.py
    x, x_ = random_tensor(shape, name)
    pos = torch.arange(rng[0], rng[1])
    pos_ = _ll(pos, "i64")
    y, y_ = random_tensor(shape, name)
    _torch_rope(y, x, pos, 10000.0)
    llaisys.Ops.rope(y_, x_, pos_, 10000.0)
    assert check_equal(y_, y, atol, rtol)


def _torch_self_attention(out, q, k, v, scale):
    q, k, v = (t.transpose(-2, -3) for t in (q, k, v))
    Lq, S = q.size(-2), k.size(-2)
    bias = torch.zeros(Lq, S, dtype=q.dtype)
    mask = torch.ones(Lq, S, dtype=torch.bool).tril(diagonal=S - Lq)
    bias.masked_fill_(mask.logical_not(), float("-inf"))
    k = k.repeat_interleave(q.size(-3) // k.size(-3), -3)
    v = v.repeat_interleave(q.size(-3) // v.size(-3), -3)
    w = q @ k.transpose(-2, -1) * scale
    w += bias
    w = torch.softmax(w, dim=-1)
    out[:] = (w @ v).transpose(-2, -3)


@pytest.mark.parametrize("shape", [(2, 2, 1, 1, 4), (5, 11, 4, 2, 8)])
@pytest.mark.parametrize("name,atol,rtol", PREC)
def test_self_attention(shape, name, atol, rtol):  # test/ops/self_attention.py
    qlen, kvlen, nh, nkvh, hd = shape
    q, q_ = random_tensor((qlen, nh, hd), name)
    k, k_ = random_tensor((kvlen, nkvh, hd), name)
    v, v_ = random_tensor((kvlen, nkvh, hd), name)
    scale = 1.0 / hd ** 0.5
    a, a_ = random_tensor((qlen, nh, hd), name)
    _torch_self_attention(a, q, k, v, scale)
    llaisys.Ops.self_attention(a_, q_, k_, v_, scale)
    assert check_equal(a_, a, atol, rtol)


@pytest.mark.parametrize("shape", [(2, 3), (512, 4096)])
@pytest.mark.parametrize("name,atol,rtol", PREC)
def test_swiglu(shape, name, atol, rtol):  # test/ops/swiglu.py
    g, g_ = random_tensor(shape, name)
    u, u_ = random_tensor(shape, name)
    out, out_ = random_tensor(shape, name)
    torch.mul(u, g / (1 + torch.exp(-g.float()).to(out.dtype)), out=out)
    llaisys.Ops.swiglu(out_, g_, u_)
    assert check_equal(out_, out, atol, rtol)
