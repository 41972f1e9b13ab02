"""Python face of the host-side KV block manager (include/llaisys/kv_cache.h).

The manager is native (csrc/kvcache/block_manager.cpp); this class only
marshals arrays. A decode step for sequences `ids` is:

    cow = mgr.reserve(i, 1)            # per sequence; copy-on-write pairs
    Ops.paged_kv_copy_blocks(kp, vp, pairs) if any cow pairs
    table, ctx = mgr.block_table(ids)  # ctx = lengths before the append
    Ops.paged_kv_append(kp, vp, k_new, v_new, table, ctx)
    mgr.commit(i, 1, [token])          # lengths advance
    Ops.paged_attention(out, q, kp, vp, table, ctx + 1, scale)
"""
from __future__ import annotations

from ctypes import POINTER, c_int32, c_int64

import numpy as np

from .libllaisys import LIB_LLAISYS, check_last_error

BLOCK_TOKENS = 16


def _i64(a):
    if a is None:
        return None, 0
    arr = np.ascontiguousarray(np.asarray(a, dtype=np.int64))
    return arr, arr.size


def _ptr(arr, ctype):
    return None if arr is None else arr.ctypes.data_as(POINTER(ctype))


class KVBlockManager:
    def __init__(self, num_blocks: int):
        self._m = LIB_LLAISYS.llaisysKVBlockManagerCreate(int(num_blocks))
        check_last_error()
        self.num_blocks = int(num_blocks)

    def __del__(self):
        if getattr(self, "_m", None):
            LIB_LLAISYS.llaisysKVBlockManagerDestroy(self._m)
            self._m = None

    def _ret(self, r: int) -> int:
        check_last_error()
        return int(r)

    def num_free(self) -> int:
        return self._ret(LIB_LLAISYS.llaisysKVNumFreeBlocks(self._m))

    def create(self, seq_id: int, tokens=None) -> int:
        """New sequence; returns how many leading tokens the prefix cache already holds."""
        arr, n = _i64(tokens)
        return self._ret(LIB_LLAISYS.llaisysKVSeqCreate(self._m, seq_id, _ptr(arr, c_int64), n))

    def fork(self, parent: int, child: int) -> None:
        self._ret(LIB_LLAISYS.llaisysKVSeqFork(self._m, parent, child))

    def reserve(self, seq_id: int, ntokens: int) -> list[tuple[int, int]]:
        """Map blocks for ntokens more positions; returns copy-on-write (src, dst) pairs."""
        pairs = np.zeros(2, np.int32)
        n = self._ret(LIB_LLAISYS.llaisysKVSeqReserve(self._m, seq_id, int(ntokens), _ptr(pairs, c_int32), 1))
        return [(int(pairs[0]), int(pairs[1]))] if n else []

    def commit(self, seq_id: int, ntokens: int, tokens=None) -> None:
        arr, _ = _i64(tokens)
        self._ret(LIB_LLAISYS.llaisysKVSeqCommit(self._m, seq_id, int(ntokens), _ptr(arr, c_int64)))

    def free(self, seq_id: int) -> None:
        self._ret(LIB_LLAISYS.llaisysKVSeqFree(self._m, seq_id))

    def length(self, seq_id: int) -> int:
        return self._ret(LIB_LLAISYS.llaisysKVSeqLength(self._m, seq_id))

    def block_table(self, seq_ids, max_pages: int | None = None):
        """(table [B, max_pages] int32 with -1 padding, ctx_len [B] int32)."""
        ids, B = _i64(seq_ids)
        if max_pages is None:
            max_pages = max(1, self._ret(LIB_LLAISYS.llaisysKVBuildBlockTable(self._m, _ptr(ids, c_int64), B, None, 0,
                                                                               None)))
        table = np.empty((B, max_pages), np.int32)
        ctx = np.empty(B, np.int32)
        self._ret(LIB_LLAISYS.llaisysKVBuildBlockTable(self._m, _ptr(ids, c_int64), B, _ptr(table, c_int32),
                                                        max_pages, _ptr(ctx, c_int32)))
        return table, ctx
