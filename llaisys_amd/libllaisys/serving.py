"""Continuous-batching scheduler prototypes (include/llaisys/serving.h)."""
from ctypes import POINTER, c_int, c_int64, c_size_t, c_void_p

llaisysScheduler_t = c_void_p


def load_serving(lib):
    S = llaisysScheduler_t
    lib.llaisysQwen2SchedulerCreate.argtypes = [c_void_p, c_size_t, c_size_t, c_size_t]
    lib.llaisysQwen2SchedulerCreate.restype = S
    lib.llaisysSimSchedulerCreate.argtypes = [c_size_t, c_int64, c_size_t, c_size_t, c_size_t, c_size_t]
    lib.llaisysSimSchedulerCreate.restype = S
    lib.llaisysSchedulerDestroy.argtypes = [S]
    lib.llaisysSchedulerDestroy.restype = None
    lib.llaisysSchedulerAdd.argtypes = [S, POINTER(c_int64), c_size_t, c_size_t, c_int64]
    lib.llaisysSchedulerAdd.restype = c_int64
    lib.llaisysSchedulerStep.argtypes = [S]
    lib.llaisysSchedulerStep.restype = c_int64
    lib.llaisysSchedulerStatus.argtypes = [S, c_int64]
    lib.llaisysSchedulerStatus.restype = c_int
    lib.llaisysSchedulerTokens.argtypes = [S, c_int64, POINTER(c_int64), c_size_t]
    lib.llaisysSchedulerTokens.restype = c_int64
    lib.llaisysSchedulerRelease.argtypes = [S, c_int64]
    lib.llaisysSchedulerRelease.restype = c_int
    lib.llaisysSchedulerStats.argtypes = [S, POINTER(c_int64)]
    lib.llaisysSchedulerStats.restype = c_int
