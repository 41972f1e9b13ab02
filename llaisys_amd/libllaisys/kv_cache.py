"""Block-manager prototypes (include/llaisys/kv_cache.h)."""
from ctypes import POINTER, c_int, c_int32, c_int64, c_size_t, c_void_p

llaisysKVBlockManager_t = c_void_p


def load_kv_cache(lib):
    M = llaisysKVBlockManager_t
    lib.llaisysKVBlockManagerCreate.argtypes = [c_int]
    lib.llaisysKVBlockManagerCreate.restype = M
    lib.llaisysKVBlockManagerDestroy.argtypes = [M]
    lib.llaisysKVBlockManagerDestroy.restype = None
    lib.llaisysKVNumFreeBlocks.argtypes = [M]
    lib.llaisysKVNumFreeBlocks.restype = c_int
    lib.llaisysKVSeqCreate.argtypes = [M, c_int64, POINTER(c_int64), c_size_t]
    lib.llaisysKVSeqCreate.restype = c_int
    lib.llaisysKVSeqFork.argtypes = [M, c_int64, c_int64]
    lib.llaisysKVSeqFork.restype = c_int
    lib.llaisysKVSeqReserve.argtypes = [M, c_int64, c_int, POINTER(c_int32), c_int]
    lib.llaisysKVSeqReserve.restype = c_int
    lib.llaisysKVSeqCommit.argtypes = [M, c_int64, c_int, POINTER(c_int64)]
    lib.llaisysKVSeqCommit.restype = c_int
    lib.llaisysKVSeqFree.argtypes = [M, c_int64]
    lib.llaisysKVSeqFree.restype = c_int
    lib.llaisysKVSeqLength.argtypes = [M, c_int64]
    lib.llaisysKVSeqLength.restype = c_int
    lib.llaisysKVBuildBlockTable.argtypes = [M, POINTER(c_int64), c_size_t, POINTER(c_int32), c_size_t, POINTER(c_int32)]
    lib.llaisysKVBuildBlockTable.restype = c_int
