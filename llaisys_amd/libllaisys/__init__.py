"""Loads libllaisys.so from this directory and declares its prototypes
(reference: python/llaisys/libllaisys/__init__.py:17-40).

The library is the HIP build for gfx950. If it has not been built, importing
this module raises: there is no CPU fallback for the kernels it carries.
"""
import ctypes
import importlib.util
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
from .kv_cache import load_kv_cache, llaisysKVBlockManager_t
from .qwen2 import LlaisysQwen2Meta, LlaisysQwen2Weights, llaisysQwen2Model_t, load_qwen2
from .ops import load_ops
from .runtime import LlaisysRuntimeAPI, load_runtime
from .serving import llaisysScheduler_t, load_serving
from .tensor import llaisysTensor_t, load_tensor
from .testing import load_testing

# LLAISYS_LIBRARY may name another build of the same library (e.g. a tuning variant).
LIB_PATH = Path(os.environ.get("LLAISYS_LIBRARY") or Path(__file__).resolve().parent / "libllaisys.so")


def _share_hip_runtime():
    """Map the HIP runtime this process should use before libllaisys.so binds it.

    libllaisys.so needs libamdhip64.so.7 (and no other ROCm library). PyTorch-ROCm
    ships its own copy under the same soname; if libllaisys.so were loaded
    first it would pull in /opt/rocm's and a later `import torch` would bring
    a second HIP runtime into the process, whose device pointers the first
    cannot use. So when torch is installed its copies are mapped first (by
    path, without importing torch), making one runtime serve both.
    LLAISYS_HIP_RUNTIME names another libamdhip64 to use instead.
    """
    path = os.environ.get("LLAISYS_HIP_RUNTIME")
    libs = [path] if path else []
    if not path:
        spec = importlib.util.find_spec("torch")
        if spec and spec.submodule_search_locations:
            torch_lib = Path(list(spec.submodule_search_locations)[0]) / "lib"
            libs = [os.fspath(torch_lib / n) for n in ("libamdhip64.so",) if (torch_lib / n).is_file()]
    for lib in libs:
        ctypes.CDLL(lib, mode=ctypes.RTLD_GLOBAL)


def load_shared_library():
    if not sys.platform.startswith("linux"):
        raise RuntimeError("llaisys_amd targets Linux with ROCm only")
    if not LIB_PATH.is_file():
        raise FileNotFoundError(
            f"{LIB_PATH} is missing: build it with `python llaisys_amd/build.py` "
            "(the HIP kernels have no fallback)"
        )
    _share_hip_runtime()
    return ctypes.CDLL(os.fspath(LIB_PATH))


LIB_LLAISYS = load_shared_library()
load_runtime(LIB_LLAISYS)
load_tensor(LIB_LLAISYS)
load_ops(LIB_LLAISYS)
load_kv_cache(LIB_LLAISYS)
load_qwen2(LIB_LLAISYS)
load_serving(LIB_LLAISYS)
load_testing(LIB_LLAISYS)


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
    "llaisysKVBlockManager_t",
    "LlaisysQwen2Meta",
    "LlaisysQwen2Weights",
    "llaisysQwen2Model_t",
    "llaisysScheduler_t",
    "llaisysDataType_t",
    "DataType",
    "llaisysDeviceType_t",
    "DeviceType",
    "llaisysMemcpyKind_t",
    "MemcpyKind",
]
