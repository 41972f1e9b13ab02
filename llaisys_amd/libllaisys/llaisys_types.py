"""ctypes enums; values match include/llaisys.h (reference: python/llaisys/libllaisys/llaisys_types.py:6-62)."""
import ctypes
from enum import IntEnum


class DeviceType(IntEnum):
    CPU = 0
    NVIDIA = 1
    AMD = 2
    COUNT = 3


class DataType(IntEnum):
    INVALID = 0
    BYTE = 1
    BOOL = 2
    I8 = 3
    I16 = 4
    I32 = 5
    I64 = 6
    U8 = 7
    U16 = 8
    U32 = 9
    U64 = 10
    F8 = 11
    F16 = 12
    F32 = 13
    F64 = 14
    C16 = 15
    C32 = 16
    C64 = 17
    C128 = 18
    BF16 = 19


class MemcpyKind(IntEnum):
    H2H = 0
    H2D = 1
    D2H = 2
    D2D = 3


llaisysDeviceType_t = ctypes.c_int
llaisysDataType_t = ctypes.c_int
llaisysMemcpyKind_t = ctypes.c_int
llaisysStream_t = ctypes.c_void_p

__all__ = [
    "DeviceType", "DataType", "MemcpyKind",
    "llaisysDeviceType_t", "llaisysDataType_t", "llaisysMemcpyKind_t", "llaisysStream_t",
]
