"""Ops wrapper (reference: python/llaisys/ops.py:6-55, plus the paged KV ops).

Every method forwards to the C symbol of the same op and raises LlaisysError
if the library reported a failure.
"""
from ctypes import c_float

from .libllaisys import LIB_LLAISYS, check_last_error
from .tensor import Tensor


def _h(t):
    return None if t is None else t.lib_tensor()


class Ops:
    @staticmethod
    def add(c: Tensor, a: Tensor, b: Tensor):
        LIB_LLAISYS.llaisysAdd(_h(c), _h(a), _h(b))
        check_last_error()

    @staticmethod
    def argmax(max_idx: Tensor, max_val: Tensor, vals: Tensor):
        LIB_LLAISYS.llaisysArgmax(_h(max_idx), _h(max_val), _h(vals))
        check_last_error()

    @staticmethod
    def embedding(out: Tensor, index: Tensor, weight: Tensor):
        LIB_LLAISYS.llaisysEmbedding(_h(out), _h(index), _h(weight))
        check_last_error()

    @staticmethod
    def linear(out: Tensor, inp: Tensor, weight: Tensor, bias: Tensor):
        LIB_LLAISYS.llaisysLinear(_h(out), _h(inp), _h(weight), _h(bias))
        check_last_error()

    @staticmethod
    def linear_pack_weight(packed: Tensor, weight: Tensor):
        """Rewrite weight [N, K] into the decode GEMM's packed layout (same shape)."""
        LIB_LLAISYS.llaisysLinearPackWeight(_h(packed), _h(weight))
        check_last_error()

    @staticmethod
    def linear_packed(out: Tensor, inp: Tensor, packed: Tensor, bias: Tensor = None):
        """out = inp . W^T + bias with W given packed by linear_pack_weight, for
        decode-sized batches: bf16, M <= 128, and either K == 1536 or
        1536 < K <= 16384 with N % 128 == 0 (split over K into fp32 partials
        summed in a fixed order); the contract of llaisysLinearPacked in
        include/llaisys/ops.h."""
        LIB_LLAISYS.llaisysLinearPacked(_h(out), _h(inp), _h(packed), _h(bias))
        check_last_error()

    @staticmethod
    def rearrange(out: Tensor, inp: Tensor):
        LIB_LLAISYS.llaisysRearrange(_h(out), _h(inp))
        check_last_error()

    @staticmethod
    def rms_norm(out: Tensor, inp: Tensor, weight: Tensor, eps: float):
        LIB_LLAISYS.llaisysRmsNorm(_h(out), _h(inp), _h(weight), c_float(eps))
        check_last_error()

    @staticmethod
    def rope(out: Tensor, inp: Tensor, pos_ids: Tensor, theta: float):
        LIB_LLAISYS.llaisysROPE(_h(out), _h(inp), _h(pos_ids), c_float(theta))
        check_last_error()

    @staticmethod
    def swiglu(out: Tensor, gate: Tensor, up: Tensor):
        LIB_LLAISYS.llaisysSwiGLU(_h(out), _h(gate), _h(up))
        check_last_error()

    @staticmethod
    def self_attention(attn_val: Tensor, q: Tensor, k: Tensor, v: Tensor, scale: float):
        """Causal GQA attention over contiguous K/V (include/llaisys/ops.h)."""
        LIB_LLAISYS.llaisysSelfAttention(_h(attn_val), _h(q), _h(k), _h(v), c_float(scale))
        check_last_error()

    @staticmethod
    def paged_kv_append(k_pool: Tensor, v_pool: Tensor, k_new: Tensor, v_new: Tensor,
                        block_table: Tensor, ctx_len: Tensor, cu_new: Tensor = None):
        """Write new K/V rows at positions ctx_len[b] + i of each sequence's pages."""
        LIB_LLAISYS.llaisysPagedKVAppend(_h(k_pool), _h(v_pool), _h(k_new), _h(v_new),
                                         _h(block_table), _h(ctx_len), _h(cu_new))
        check_last_error()

    @staticmethod
    def paged_kv_gather(k_out: Tensor, v_out: Tensor, k_pool: Tensor, v_pool: Tensor,
                        block_table: Tensor, cu_seqlens: Tensor):
        """Copy each sequence's first (cu[b+1]-cu[b]) tokens out of the pool, row-major."""
        LIB_LLAISYS.llaisysPagedKVGather(_h(k_out), _h(v_out), _h(k_pool), _h(v_pool),
                                         _h(block_table), _h(cu_seqlens))
        check_last_error()

    @staticmethod
    def paged_kv_append_gather(k_out: Tensor, v_out: Tensor, k_pool: Tensor, v_pool: Tensor, k_new: Tensor,
                               v_new: Tensor, block_table: Tensor, ctx_len: Tensor, cu_seqlens: Tensor):
        """paged_kv_append of one token per sequence, then paged_kv_gather of the
        contexts including it (cu_seqlens[b+1] - cu_seqlens[b] == ctx_len[b] + 1), in one launch."""
        LIB_LLAISYS.llaisysPagedKVAppendGather(_h(k_out), _h(v_out), _h(k_pool), _h(v_pool), _h(k_new), _h(v_new),
                                               _h(block_table), _h(ctx_len), _h(cu_seqlens))
        check_last_error()

    @staticmethod
    def paged_kv_copy_blocks(k_pool: Tensor, v_pool: Tensor, pairs: Tensor):
        """Copy whole blocks (src -> dst, pairs [P, 2] I32), e.g. for copy-on-write."""
        LIB_LLAISYS.llaisysPagedKVCopyBlocks(_h(k_pool), _h(v_pool), _h(pairs))
        check_last_error()

    @staticmethod
    def paged_attention(out: Tensor, q: Tensor, k_pool: Tensor, v_pool: Tensor,
                        block_table: Tensor, ctx_len: Tensor, scale: float):
        """Batched decode attention over paged KV (one query per sequence)."""
        LIB_LLAISYS.llaisysPagedAttention(_h(out), _h(q), _h(k_pool), _h(v_pool),
                                          _h(block_table), _h(ctx_len), c_float(scale))
        check_last_error()

    @staticmethod
    def paged_attention_no_alloc(out: Tensor, q: Tensor, k_pool: Tensor, v_pool: Tensor,
                                 block_table: Tensor, ctx_len: Tensor, scale: float):
        """paged_attention with no device allocation (fixed per-GPU scratch)."""
        LIB_LLAISYS.llaisysPagedAttentionNoAlloc(_h(out), _h(q), _h(k_pool), _h(v_pool),
                                                 _h(block_table), _h(ctx_len), c_float(scale))
        check_last_error()

    @staticmethod
    def paged_attention_varlen(out: Tensor, q: Tensor, k_pool: Tensor, v_pool: Tensor,
                               block_table: Tensor, cu_q: Tensor, ctx_len: Tensor, scale: float):
        """Mixed chunked-prefill + decode attention over paged KV."""
        LIB_LLAISYS.llaisysPagedAttentionVarlen(_h(out), _h(q), _h(k_pool), _h(v_pool),
                                                _h(block_table), _h(cu_q), _h(ctx_len), c_float(scale))
        check_last_error()
