"""CPU oracle for the KV-cache attention path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker. The product (llaisys_amd) never imports it.

Contents:
  * ctypes bindings to oracle/liboracle.so (oracle.c: the C restatement of
    the reference's self_attention spec and of paged append/gather/attention);
  * numpy helpers: a splitmix64 + Box-Muller normal generator (so seeded
    inputs are reproducible without torch), exact bf16 <-> f32 conversion with
    round-to-nearest-even (reference src/utils/types.cpp:66-84), and the device
    page format written as reshape/transpose (an independent derivation of the
    index formulas in oracle.c and the HIP kernels).

Parity pins for every function live in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

PAGE = 16
HEAD_DIM = 128


def build() -> Path:
    """Compile oracle.c -> liboracle.so (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-B", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            build()
        L = ctypes.CDLL(os.fspath(LIB_PATH))
        P = ctypes.c_void_p
        i = ctypes.c_int
        L.orc_self_attention.argtypes = [P, P, P, P, i, i, i, i, i, i, ctypes.c_float, i]
        L.orc_self_attention.restype = None
        L.orc_paged_append.argtypes = [P, P, P, P, P, i, P, P, i, i, i, i]
        L.orc_paged_append.restype = i
        L.orc_paged_gather.argtypes = [P, P, P, P, P, i, P, i, i, i]
        L.orc_paged_gather.restype = i
        L.orc_pack_pages.argtypes = [P, P, ctypes.c_long, i]
        L.orc_pack_pages.restype = None
        L.orc_unpack_pages.argtypes = [P, P, ctypes.c_long, i]
        L.orc_unpack_pages.restype = None
        L.orc_paged_attention.argtypes = [P, P, P, P, P, i, P, P, i, i, i, i, ctypes.c_float, i]
        L.orc_paged_attention.restype = i
        L.orc_max_threads.argtypes = []
        L.orc_max_threads.restype = i
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- numbers


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n outputs of the splitmix64 generator started at `seed` (uint64)."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def randn(seed: int, shape) -> np.ndarray:
    """Seeded N(0,1) float32 via Box-Muller over splitmix64 uniforms."""
    n = int(np.prod(shape)) if len(shape) else 1
    m = (n + 1) // 2
    bits = splitmix64(seed, 2 * m)
    u = ((bits >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)  # (0,1)
    u1, u2 = u[:m], u[m:]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.concatenate([r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)])[:n]
    return z.astype(np.float32).reshape(shape)


def randint(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """n seeded integers uniform in [lo, hi] (inclusive)."""
    bits = splitmix64(seed, n)
    return (lo + (bits % np.uint64(hi - lo + 1)).astype(np.int64)).astype(np.int64)


def permutation(seed: int, n: int) -> np.ndarray:
    """Seeded Fisher-Yates permutation of range(n) (int32)."""
    perm = np.arange(n, dtype=np.int32)
    r = splitmix64(seed, max(n - 1, 1))
    for i in range(n - 1, 0, -1):
        j = int(r[n - 1 - i] % np.uint64(i + 1))
        perm[i], perm[j] = perm[j], perm[i]
    return perm


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (uint16); NaN stays a quiet NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


# ---------------------------------------------------------------- page format
# K page (16 t x 128 d): [16 dim-chunks of 8][16 tokens][8]
# V page: [4 (d/32)][4 (t/4)][16 (d%16)][2 ((d/16)%2)][4 (t%4)]


def pack_pages_np(logical: np.ndarray, is_v: bool) -> np.ndarray:
    """[..., 16, 128] logical pages -> device page format (same shape, permuted)."""
    lead = logical.shape[:-2]
    x = logical.reshape(-1, PAGE, HEAD_DIM)
    if not is_v:
        y = x.reshape(-1, 16, 16, 8).transpose(0, 2, 1, 3)  # [p][c][t][e]
    else:
        # t = 4*g + ti ; d = 32*b2 + 16*j + n
        y = x.reshape(-1, 4, 4, 4, 2, 16).transpose(0, 3, 1, 5, 4, 2)  # [p][b2][g][n][j][ti]
    return np.ascontiguousarray(y).reshape(*lead, PAGE, HEAD_DIM)


def unpack_pages_np(dev: np.ndarray, is_v: bool) -> np.ndarray:
    lead = dev.shape[:-2]
    x = dev.reshape(-1, PAGE * HEAD_DIM)
    if not is_v:
        y = x.reshape(-1, 16, 16, 8).transpose(0, 2, 1, 3)
    else:
        y = x.reshape(-1, 4, 4, 16, 2, 4).transpose(0, 2, 5, 1, 4, 3)  # [p][g][ti][b2][j][n]
    return np.ascontiguousarray(y).reshape(*lead, PAGE, HEAD_DIM)


def pack_pages_c(logical: np.ndarray, is_v: bool) -> np.ndarray:
    x = np.ascontiguousarray(logical, dtype=np.uint16)
    out = np.empty_like(x)
    lib().orc_pack_pages(_p(out), _p(x), x.size // (PAGE * HEAD_DIM), int(is_v))
    return out


def unpack_pages_c(dev: np.ndarray, is_v: bool) -> np.ndarray:
    x = np.ascontiguousarray(dev, dtype=np.uint16)
    out = np.empty_like(x)
    lib().orc_unpack_pages(_p(out), _p(x), x.size // (PAGE * HEAD_DIM), int(is_v))
    return out


# ---------------------------------------------------------------- ops


def self_attention(q, k, v, scale: float, nthreads: int = 1) -> np.ndarray:
    """fp32 oracle of the reference self_attention. q [L,nh,d], k [S,nkvh,d], v [S,nkvh,dv]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    L, nh, d = q.shape
    S, nkvh, _ = k.shape
    dv = v.shape[2]
    out = np.zeros((L, nh, dv), np.float32)
    lib().orc_self_attention(_p(out), _p(q), _p(k), _p(v), L, S, nh, nkvh, d, dv, float(scale), nthreads)
    return out


def paged_append(k_pool, v_pool, k_new, v_new, table, ctx, cu_new=None) -> int:
    """In place on logical uint16 pools [nb, nkvh, 16, 128]. Returns 1 on a bad mapping."""
    for a in (k_pool, v_pool):
        assert a.dtype == np.uint16 and a.flags["C_CONTIGUOUS"]
    k_new = np.ascontiguousarray(k_new, np.uint16)
    v_new = np.ascontiguousarray(v_new, np.uint16)
    table = np.ascontiguousarray(table, np.int32)
    ctx = np.ascontiguousarray(ctx, np.int32)
    cu = None if cu_new is None else np.ascontiguousarray(cu_new, np.int32)
    return lib().orc_paged_append(_p(k_pool), _p(v_pool), _p(k_new), _p(v_new), _p(table), table.shape[1], _p(ctx),
                                  _p(cu), len(ctx), k_new.shape[0], k_pool.shape[1], k_pool.shape[0])


def paged_gather(k_pool, v_pool, table, cu):
    table = np.ascontiguousarray(table, np.int32)
    cu = np.ascontiguousarray(cu, np.int32)
    T = int(cu[-1])
    nkvh = k_pool.shape[1]
    k_out = np.zeros((T, nkvh, HEAD_DIM), np.uint16)
    v_out = np.zeros((T, nkvh, HEAD_DIM), np.uint16)
    bad = lib().orc_paged_gather(_p(k_out), _p(v_out), _p(np.ascontiguousarray(k_pool)), _p(np.ascontiguousarray(v_pool)),
                                 _p(table), table.shape[1], _p(cu), len(cu) - 1, nkvh, k_pool.shape[0])
    assert bad == 0, "oracle gather hit an unmapped page"
    return k_out, v_out


def paged_attention(q_bf16, k_pool, v_pool, table, ctx, scale: float, cu_q=None, nthreads: int = 1) -> np.ndarray:
    """fp32 output [T, nh, 128]; q given as bf16 bits [T, nh, 128]; logical pools."""
    q = bf16_to_f32(q_bf16)
    T, nh, _ = q.shape
    table = np.ascontiguousarray(table, np.int32)
    ctx = np.ascontiguousarray(ctx, np.int32)
    cu = None if cu_q is None else np.ascontiguousarray(cu_q, np.int32)
    out = np.zeros((T, nh, HEAD_DIM), np.float32)
    bad = lib().orc_paged_attention(_p(out), _p(q), _p(np.ascontiguousarray(k_pool)), _p(np.ascontiguousarray(v_pool)),
                                    _p(table), table.shape[1], _p(ctx), _p(cu), len(ctx), nh, k_pool.shape[1],
                                    k_pool.shape[0], float(scale), nthreads)
    assert bad == 0, "oracle attention hit an unmapped page"
    return out


def max_threads() -> int:
    return int(lib().orc_max_threads())
