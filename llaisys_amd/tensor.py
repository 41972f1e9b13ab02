"""Python Tensor over a libllaisys handle (reference: python/llaisys/tensor.py:14-97).

Same constructor and methods as the reference. Failures inside the library
raise LlaisysError here (the reference's wrapper would abort the process).
"""
from ctypes import c_int, c_size_t, c_ssize_t, c_void_p
from typing import Sequence, Tuple

from .libllaisys import (
    LIB_LLAISYS,
    DataType,
    DeviceType,
    check_last_error,
    llaisysDataType_t,
    llaisysDeviceType_t,
    llaisysTensor_t,
)


class Tensor:
    def __init__(
        self,
        shape: Sequence[int] = None,
        dtype: DataType = DataType.F32,
        device: DeviceType = DeviceType.CPU,
        device_id: int = 0,
        tensor: llaisysTensor_t = None,
    ):
        if tensor:
            self._tensor = tensor
            return
        ndim = 0 if shape is None else len(shape)
        c_shape = (c_size_t * max(ndim, 1))(*(shape or ()))
        self._tensor = LIB_LLAISYS.tensorCreate(
            c_shape, c_size_t(ndim), llaisysDataType_t(dtype), llaisysDeviceType_t(device), c_int(device_id)
        )
        check_last_error()

    def __del__(self):
        if getattr(self, "_tensor", None) is not None:
            LIB_LLAISYS.tensorDestroy(self._tensor)
            self._tensor = None

    def ndim(self) -> int:
        return int(LIB_LLAISYS.tensorGetNdim(self._tensor))

    def shape(self) -> Tuple[int, ...]:
        n = self.ndim()
        buf = (c_size_t * max(n, 1))()
        LIB_LLAISYS.tensorGetShape(self._tensor, buf)
        return tuple(int(buf[i]) for i in range(n))

    def strides(self) -> Tuple[int, ...]:
        n = self.ndim()
        buf = (c_ssize_t * max(n, 1))()
        LIB_LLAISYS.tensorGetStrides(self._tensor, buf)
        return tuple(int(buf[i]) for i in range(n))

    def dtype(self) -> DataType:
        return DataType(LIB_LLAISYS.tensorGetDataType(self._tensor))

    def device_type(self) -> DeviceType:
        return DeviceType(LIB_LLAISYS.tensorGetDeviceType(self._tensor))

    def device_id(self) -> int:
        return int(LIB_LLAISYS.tensorGetDeviceId(self._tensor))

    def data_ptr(self) -> c_void_p:
        return LIB_LLAISYS.tensorGetData(self._tensor)

    def lib_tensor(self) -> llaisysTensor_t:
        return self._tensor

    def debug(self):
        LIB_LLAISYS.tensorDebug(self._tensor)
        check_last_error()

    def __repr__(self):
        return f"<Tensor shape={self.shape()}, dtype={self.dtype().name}, device={self.device_type().name}:{self.device_id()}>"

    def load(self, data: c_void_p):
        LIB_LLAISYS.tensorLoad(self._tensor, data)
        check_last_error()

    def is_contiguous(self) -> bool:
        return bool(LIB_LLAISYS.tensorIsContiguous(self._tensor))

    def _wrap(self, handle) -> "Tensor":
        check_last_error()
        return Tensor(tensor=handle)

    def view(self, *shape: int) -> "Tensor":
        c_shape = (c_size_t * max(len(shape), 1))(*shape)
        return self._wrap(LIB_LLAISYS.tensorView(self._tensor, c_shape, c_size_t(len(shape))))

    def permute(self, *perm: int) -> "Tensor":
        assert len(perm) == self.ndim()
        c_perm = (c_size_t * max(len(perm), 1))(*perm)
        return self._wrap(LIB_LLAISYS.tensorPermute(self._tensor, c_perm))

    def slice(self, dim: int, start: int, end: int) -> "Tensor":
        return self._wrap(LIB_LLAISYS.tensorSlice(self._tensor, c_size_t(dim), c_size_t(start), c_size_t(end)))
