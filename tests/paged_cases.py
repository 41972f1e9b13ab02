"""Seeded paged-KV test cases: block tables over a randomly permuted pool,
logical pools (oracle layout) and their device-format copies."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

import llaisys_amd as L
import oracle
from utils import from_bits, to_llaisys


@dataclass
class PagedCase:
    ctx: np.ndarray        # [B] int32 tokens in cache
    table: np.ndarray      # [B, maxp] int32
    k_log: np.ndarray      # [nb, nkvh, 16, 128] uint16 (logical)
    v_log: np.ndarray
    nh: int
    nkvh: int

    @property
    def B(self):
        return len(self.ctx)

    def device_pools(self):
        kp = to_llaisys(from_bits(oracle.pack_pages_np(self.k_log, False)))
        vp = to_llaisys(from_bits(oracle.pack_pages_np(self.v_log, True)))
        return kp, vp

    def device_meta(self):
        return to_llaisys(torch.from_numpy(self.table)), to_llaisys(torch.from_numpy(self.ctx))


def make_case(seed: int, ctx: np.ndarray, nh: int = 12, nkvh: int = 2, spare_blocks: int = 3,
              stale_nan: bool = False, extra_pages: int = 0) -> PagedCase:
    ctx = np.asarray(ctx, np.int32)
    pages = (ctx + 15) // 16
    maxp = int(max(pages.max(initial=1), 1)) + extra_pages
    nb = int(pages.sum()) + spare_blocks
    perm = oracle.permutation(seed, nb)
    table = np.full((len(ctx), maxp), -1, np.int32)
    used = 0
    for b, p in enumerate(pages):
        table[b, :p] = perm[used:used + p]
        used += p
    k_log = oracle.f32_to_bf16(oracle.randn(seed + 1, (nb, nkvh, 16, 128)))
    v_log = oracle.f32_to_bf16(oracle.randn(seed + 2, (nb, nkvh, 16, 128)))
    if stale_nan:
        # Slots past each sequence's length (and spare blocks) hold NaN / Inf patterns.
        owned = np.zeros((nb, 16), bool)
        for b in range(len(ctx)):
            for pos in range(int(ctx[b])):
                owned[table[b, pos // 16], pos % 16] = True
        stale = ~owned
        k_log[np.broadcast_to(stale[:, None, :, None], k_log.shape)] = 0x7FC0
        v_log[np.broadcast_to(stale[:, None, :, None], v_log.shape)] = 0xFF80  # -inf
    return PagedCase(ctx, table, k_log, v_log, nh, nkvh)


def queries(seed: int, T: int, nh: int) -> np.ndarray:
    return oracle.f32_to_bf16(oracle.randn(seed, (T, nh, 128)))
