"""Continuous-batching scheduler (include/llaisys/serving.h).

Requests queue up and every `step()` runs one mixed batch on the model:
single-token decodes of running requests plus prefill chunks of admitted
ones, with preemption (and later recomputation) when the KV pool runs short.
The reference asks for this as a serving project (README.md:421-424) and has
no code for it.

    sched = Scheduler(model, max_seqs=64, max_step_tokens=2048, prefill_chunk=512)
    rid = sched.add(prompt_ids, max_new_tokens=128)
    while sched.step():
        ...                               # sched.tokens(rid) grows as it decodes
    out = sched.tokens(rid)

`Scheduler.simulated(...)` runs the same scheduler over a host-only stand-in
model (see `sim_greedy`) for testing without a GPU.
"""
from ctypes import POINTER, c_int64
from enum import IntEnum
from typing import Dict, List, Optional, Sequence

import numpy as np

from .libllaisys import LIB_LLAISYS, check_last_error


class RequestStatus(IntEnum):
    ACTIVE = 0
    MAX_TOKENS = 1
    EOS = 2
    LENGTH = 3
    NO_CAPACITY = 4


def sim_greedy(history: Sequence[int], vocab: int) -> int:
    """The simulated model's greedy token after `history`: FNV-1a-64 over the
    int64 token values (each XORed in whole), modulo vocab."""
    h = 14695981039346656037
    for t in history:
        h ^= int(t) & 0xFFFFFFFFFFFFFFFF
        h = (h * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h % vocab


class Scheduler:
    """Continuous batching over a `llaisys_amd.models.Qwen2` model."""

    def __init__(self, model, max_seqs: int = 64, max_step_tokens: int = 2048, prefill_chunk: int = 512,
                 _handle=None):
        self._model = model  # kept alive: the scheduler uses its sequences and KV pool
        if _handle is None:
            _handle = LIB_LLAISYS.llaisysQwen2SchedulerCreate(model._model, max_seqs, max_step_tokens,
                                                              prefill_chunk)
        if not _handle:
            check_last_error()
            raise RuntimeError("llaisysQwen2SchedulerCreate failed")
        self._s = _handle

    @classmethod
    def simulated(cls, num_blocks: int, vocab: int, max_seq_len: int, max_seqs: int = 64,
                  max_step_tokens: int = 2048, prefill_chunk: int = 512) -> "Scheduler":
        """The scheduler over a host-only simulated model (no GPU): a KV pool of
        num_blocks 16-token blocks and greedy tokens given by `sim_greedy`."""
        h = LIB_LLAISYS.llaisysSimSchedulerCreate(num_blocks, vocab, max_seq_len, max_seqs, max_step_tokens,
                                                  prefill_chunk)
        if not h:
            check_last_error()
            raise RuntimeError("llaisysSimSchedulerCreate failed")
        return cls(None, _handle=h)

    def __del__(self):
        if getattr(self, "_s", None):
            LIB_LLAISYS.llaisysSchedulerDestroy(self._s)
            self._s = None

    def add(self, prompt: Sequence[int], max_new_tokens: int, eos: Optional[int] = None) -> int:
        """Queue a request; returns its id. eos: token that ends it (None: only max_new_tokens)."""
        arr = np.ascontiguousarray(prompt, dtype=np.int64)
        rid = LIB_LLAISYS.llaisysSchedulerAdd(self._s, arr.ctypes.data_as(POINTER(c_int64)), arr.size,
                                              max_new_tokens, -1 if eos is None else int(eos))
        if rid < 0:
            check_last_error()
        return int(rid)

    def step(self) -> int:
        """Run one model step; returns how many requests are unfinished."""
        n = LIB_LLAISYS.llaisysSchedulerStep(self._s)
        if n < 0:
            check_last_error()
        return int(n)

    def status(self, rid: int) -> RequestStatus:
        st = LIB_LLAISYS.llaisysSchedulerStatus(self._s, rid)
        if st < 0:
            check_last_error()
            raise KeyError(rid)
        return RequestStatus(st)

    def finished(self, rid: int) -> bool:
        return self.status(rid) != RequestStatus.ACTIVE

    def tokens(self, rid: int) -> List[int]:
        """Tokens generated so far for request rid."""
        n = LIB_LLAISYS.llaisysSchedulerTokens(self._s, rid, None, 0)
        if n < 0:
            check_last_error()
        out = np.zeros(max(int(n), 1), np.int64)
        LIB_LLAISYS.llaisysSchedulerTokens(self._s, rid, out.ctypes.data_as(POINTER(c_int64)), out.size)
        return out[:n].tolist()

    def release(self, rid: int) -> None:
        """Forget a finished request."""
        if LIB_LLAISYS.llaisysSchedulerRelease(self._s, rid) < 0:
            check_last_error()

    def stats(self) -> Dict[str, int]:
        v = (c_int64 * 5)()
        if LIB_LLAISYS.llaisysSchedulerStats(self._s, v) < 0:
            check_last_error()
        return dict(zip(("steps", "preemptions", "prefill_tokens", "decode_tokens", "finished"), list(v)))

    def run(self, max_steps: int = 1 << 30) -> int:
        """Step until every request finished (or max_steps); returns the steps run."""
        start = self.stats()["steps"]
        for _ in range(max_steps):
            if self.step() == 0:
                break
        return self.stats()["steps"] - start
