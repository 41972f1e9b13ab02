"""Op prototypes (reference: python/llaisys/libllaisys/ops.py:4-36, plus the paged KV ops)."""
from ctypes import c_float

from .tensor import llaisysTensor_t

T = llaisysTensor_t


def load_ops(lib):
    for name, args in [
        ("llaisysAdd", [T, T, T]),
        ("llaisysArgmax", [T, T, T]),
        ("llaisysEmbedding", [T, T, T]),
        ("llaisysLinear", [T, T, T, T]),
        ("llaisysRearrange", [T, T]),
        ("llaisysRmsNorm", [T, T, T, c_float]),
        ("llaisysROPE", [T, T, T, c_float]),
        ("llaisysSwiGLU", [T, T, T]),
        # attn_val, q, k, v, scale
        ("llaisysSelfAttention", [T, T, T, T, c_float]),
        # k_pool, v_pool, k_new, v_new, block_table, ctx_len, cu_new (nullable)
        ("llaisysPagedKVAppend", [T, T, T, T, T, T, T]),
        # k_pool, v_pool, pairs [P, 2] (src, dst)
        ("llaisysPagedKVCopyBlocks", [T, T, T]),
        # k_out, v_out, k_pool, v_pool, block_table, cu_seqlens
        ("llaisysPagedKVGather", [T, T, T, T, T, T]),
        # k_out, v_out, k_pool, v_pool, k_new, v_new, block_table, ctx_len, cu_seqlens
        ("llaisysPagedKVAppendGather", [T, T, T, T, T, T, T, T, T]),
        # out, q, k_pool, v_pool, block_table, ctx_len, scale
        ("llaisysLinearPackWeight", [T, T]),
        ("llaisysLinearPacked", [T, T, T, T]),
        ("llaisysPagedAttention", [T, T, T, T, T, T, c_float]),
        ("llaisysPagedAttentionNoAlloc", [T, T, T, T, T, T, c_float]),
        # out, q, k_pool, v_pool, block_table, cu_q, ctx_len, scale
        ("llaisysPagedAttentionVarlen", [T, T, T, T, T, T, T, c_float]),
    ]:
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = None
