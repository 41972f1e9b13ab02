"""Tensor meta ops on CPU tensors, restating the reference's test/test_tensor.py:8-49
(load, view, permute, slice: shapes, strides, contiguity and values vs torch)."""
import pytest
import torch

import llaisys_amd as L
from utils import to_torch


def make():
    t = torch.arange(60, dtype=torch.int64).reshape(3, 4, 5)
    lt = L.Tensor((3, 4, 5), dtype=L.DataType.I64, device=L.DeviceType.CPU)
    lt.load(t.data_ptr())
    return t, lt


def test_load_view_permute_slice_like_reference():
    t, lt = make()
    assert lt.is_contiguous() and torch.equal(to_torch(lt), t)
    v, lv = t.view(6, 10), lt.view(6, 10)
    assert lv.shape() == v.shape and lv.strides() == v.stride() and torch.equal(to_torch(lv), v)
    p, lp = t.permute(2, 0, 1), lt.permute(2, 0, 1)
    assert lp.shape() == p.shape and lp.strides() == p.stride()
    assert not lp.is_contiguous() and torch.equal(to_torch(lp), p)
    s, ls = t[:, :, 1:4], lt.slice(2, 1, 4)
    assert ls.shape() == s.shape and ls.strides() == s.stride() and torch.equal(to_torch(ls), s)
    assert not ls.is_contiguous()


@pytest.mark.parametrize("shape", [(60,), (3, 20), (1, 60), (3, 1, 4, 5, 1), (12, 5)])
def test_view_compatible_shapes_match_torch(shape):
    t, lt = make()
    assert lt.view(*shape).strides() == t.view(*shape).stride()


def test_view_of_sliced_tensor_merges_only_contiguous_runs():
    t, lt = make()
    s, ls = t[:, 1:3, :], lt.slice(1, 1, 3)  # (3,2,5) strides (20,5,1): last two dims merge
    assert ls.view(3, 10).strides() == s.view(3, 10).stride()
    with pytest.raises(L.LlaisysError):
        ls.view(30)  # dims 0 and 1 are not contiguous with each other
    with pytest.raises(L.LlaisysError):
        lt.permute(2, 0, 1).view(60)


def test_errors_raise_instead_of_abort():
    _, lt = make()
    with pytest.raises(L.LlaisysError, match="slice"):
        lt.slice(2, 3, 9)
    with pytest.raises(L.LlaisysError, match="permute"):
        lt.permute(0, 0, 1)
    with pytest.raises(L.LlaisysError):
        lt.view(7, 9)


def test_debug_prints_values(capfd):
    _, lt = make()
    lt.slice(0, 2, 3).debug()
    out = capfd.readouterr().out
    assert "shape[ 1 4 5 ]" in out and "59" in out
