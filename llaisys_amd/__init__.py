"""llaisys_amd: the LLAISYS KV-cache attention path, native on MI355X (gfx950).

Same Python surface as the reference's `llaisys` package (RuntimeAPI,
DeviceType, DataType, MemcpyKind, Tensor, Ops) over libllaisys.so built from
HIP, plus the paged KV ops and the host-side block manager.
"""
from .libllaisys import DataType, DeviceType, LlaisysError, MemcpyKind
from .libllaisys import llaisysStream_t as Stream
from .kv_cache import KVBlockManager
from . import models
from .ops import Ops
from .serving import RequestStatus, Scheduler
from .runtime import RuntimeAPI, context_stream, device_error_flags, set_context_runtime, set_context_stream
from .tensor import Tensor

__all__ = [
    "RuntimeAPI",
    "DeviceType",
    "DataType",
    "MemcpyKind",
    "Stream",
    "Tensor",
    "Ops",
    "KVBlockManager",
    "Scheduler",
    "RequestStatus",
    "models",
    "LlaisysError",
    "set_context_runtime",
    "context_stream",
    "set_context_stream",
    "device_error_flags",
]
