"""Shared test helpers: torch <-> llaisys_amd bridging in the manner of the
reference's test/test_utils.py:5-160 (tensors cross by memcpy_sync from a torch
tensor on the same device) and the tolerance checks."""
from __future__ import annotations

import numpy as np
import torch

import llaisys_amd as L
from llaisys_amd import DataType, DeviceType, MemcpyKind

_TORCH_OF = {
    DataType.F32: torch.float32,
    DataType.F16: torch.float16,
    DataType.BF16: torch.bfloat16,
    DataType.I32: torch.int32,
    DataType.I64: torch.int64,
    DataType.U8: torch.uint8,
}
_LL_OF = {v: k for k, v in _TORCH_OF.items()}


def device_of(name: str) -> DeviceType:
    return {"cpu": DeviceType.CPU, "amd": DeviceType.AMD}[name]


def torch_device(name: str) -> torch.device:
    return torch.device("cpu") if name == "cpu" else torch.device("cuda:0")


def to_llaisys(t: torch.Tensor, device: str = "amd") -> L.Tensor:
    """Fresh llaisys tensor holding a copy of `t` (contiguous)."""
    t = t.contiguous()
    lt = L.Tensor(tuple(t.shape), dtype=_LL_OF[t.dtype], device=device_of(device))
    nbytes = t.numel() * t.element_size()
    if nbytes:
        api = L.RuntimeAPI(device_of(device))
        if device == "cpu":
            api.memcpy_sync(lt.data_ptr(), t.cpu().data_ptr(), nbytes, MemcpyKind.H2H)
        else:
            src = t.to(torch_device(device))
            api.memcpy_sync(lt.data_ptr(), src.data_ptr(), nbytes, MemcpyKind.D2D)
    return lt


def to_torch(lt: L.Tensor) -> torch.Tensor:
    """Copy a (possibly strided) llaisys tensor into a torch tensor on its device
    (strided read-back as test_utils.py:116-150)."""
    shape, strides = lt.shape(), lt.strides()
    dev = "cpu" if lt.device_type() == DeviceType.CPU else "amd"
    span = 1 + sum(s * (n - 1) for s, n in zip(strides, shape)) if all(shape) else 0
    tmp = torch.zeros((max(span, 1),), dtype=_TORCH_OF[lt.dtype()], device=torch_device(dev))
    if span:
        api = L.RuntimeAPI(lt.device_type())
        kind = MemcpyKind.H2H if dev == "cpu" else MemcpyKind.D2D
        api.memcpy_sync(tmp.data_ptr(), lt.data_ptr(), span * tmp.element_size(), kind)
    return torch.as_strided(tmp, shape, strides).clone()


def bits(t: torch.Tensor) -> np.ndarray:
    """uint16 bit patterns of a bf16/f16 tensor."""
    return t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray, device: str = "amd") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(torch_device(device))


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got-ref| / max(|ref|), the relative measure the fp32 tolerance uses."""
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))
