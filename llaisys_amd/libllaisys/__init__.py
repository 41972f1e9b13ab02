"""Loads libllaisys.so from this directory and declares its prototypes
(reference: python/llaisys/libllaisys/__init__.py:17-40).

The library is the HIP build for gfx950. If it has not been built, importing
this module raises: there is no CPU fallback for the kernels it carries.
"""
import ctypes
import os
import sys
from pathlib import Path

from .llaisys_types import (
    DataType,
    DeviceType,
    MemcpyKind,
    llaisysDataType_t,
    llaisysDeviceType_t,
    llaisysMemcpyKind_t,
    llaisysStream_t,
)
from .ops import load_ops
from .runtime import LlaisysRuntimeAPI, load_runtime
from .tensor import llaisysTensor_t, load_tensor

LIB_PATH = Path(__file__).resolve().parent / "libllaisys.so"


def load_shared_library():
    if not sys.platform.startswith("linux"):
        raise RuntimeError("llaisys_amd targets Linux with ROCm only")
    if not LIB_PATH.is_file():
        raise FileNotFoundError(
            f"{LIB_PATH} is missing: build it with `python -m llaisys_amd.build` "
            "(the HIP kernels have no fallback)"
        )
    return ctypes.CDLL(os.fspath(LIB_PATH))


LIB_LLAISYS = load_shared_library()
load_runtime(LIB_LLAISYS)
load_tensor(LIB_LLAISYS)
load_ops(LIB_LLAISYS)


class LlaisysError(RuntimeError):
    """A C++ check failed inside libllaisys (the message is also on stderr)."""


_ERRBUF = ctypes.create_string_buffer(4096)


def check_last_error():
    """Raise LlaisysError if the calling thread's last libllaisys call failed."""
    if LIB_LLAISYS.llaisysGetLastError(_ERRBUF, len(_ERRBUF)):
        raise LlaisysError(_ERRBUF.value.decode(errors="replace"))


__all__ = [
    "LIB_LLAISYS",
    "LIB_PATH",
    "LlaisysError",
    "check_last_error",
    "LlaisysRuntimeAPI",
    "llaisysStream_t",
    "llaisysTensor_t",
    "llaisysDataType_t",
    "DataType",
    "llaisysDeviceType_t",
    "DeviceType",
    "llaisysMemcpyKind_t",
    "MemcpyKind",
]
