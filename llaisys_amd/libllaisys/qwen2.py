"""Qwen2 model prototypes (include/llaisys/models/qwen2.h; the first four as
the reference declares them, qwen2.h:7-40)."""
from ctypes import POINTER, Structure, c_float, c_int, c_int64, c_size_t, c_void_p

from .llaisys_types import llaisysDataType_t, llaisysDeviceType_t
from .tensor import llaisysTensor_t


class LlaisysQwen2Meta(Structure):
    _fields_ = [
        ("dtype", llaisysDataType_t),
        ("nlayer", c_size_t),
        ("hs", c_size_t),
        ("nh", c_size_t),
        ("nkvh", c_size_t),
        ("dh", c_size_t),
        ("di", c_size_t),
        ("maxseq", c_size_t),
        ("voc", c_size_t),
        ("epsilon", c_float),
        ("theta", c_float),
        ("end_token", c_int64),
    ]


class LlaisysQwen2Weights(Structure):
    _fields_ = [
        ("in_embed", llaisysTensor_t),
        ("out_embed", llaisysTensor_t),
        ("out_norm_w", llaisysTensor_t),
        ("attn_norm_w", POINTER(llaisysTensor_t)),
        ("attn_q_w", POINTER(llaisysTensor_t)),
        ("attn_q_b", POINTER(llaisysTensor_t)),
        ("attn_k_w", POINTER(llaisysTensor_t)),
        ("attn_k_b", POINTER(llaisysTensor_t)),
        ("attn_v_w", POINTER(llaisysTensor_t)),
        ("attn_v_b", POINTER(llaisysTensor_t)),
        ("attn_o_w", POINTER(llaisysTensor_t)),
        ("mlp_norm_w", POINTER(llaisysTensor_t)),
        ("mlp_gate_w", POINTER(llaisysTensor_t)),
        ("mlp_up_w", POINTER(llaisysTensor_t)),
        ("mlp_down_w", POINTER(llaisysTensor_t)),
    ]


llaisysQwen2Model_t = c_void_p


def load_qwen2(lib):
    M = llaisysQwen2Model_t
    lib.llaisysQwen2ModelCreate.argtypes = [POINTER(LlaisysQwen2Meta), llaisysDeviceType_t, POINTER(c_int), c_int]
    lib.llaisysQwen2ModelCreate.restype = M
    lib.llaisysQwen2ModelCreatePaged.argtypes = [POINTER(LlaisysQwen2Meta), llaisysDeviceType_t, POINTER(c_int), c_int,
                                                 c_size_t]
    lib.llaisysQwen2ModelCreatePaged.restype = M
    lib.llaisysQwen2ModelDestroy.argtypes = [M]
    lib.llaisysQwen2ModelDestroy.restype = None
    lib.llaisysQwen2ModelWeights.argtypes = [M]
    lib.llaisysQwen2ModelWeights.restype = POINTER(LlaisysQwen2Weights)
    lib.llaisysQwen2ModelInfer.argtypes = [M, POINTER(c_int64), c_size_t]
    lib.llaisysQwen2ModelInfer.restype = c_int64
    lib.llaisysQwen2SeqCreate.argtypes = [M, POINTER(c_int64), c_size_t, POINTER(c_size_t)]
    lib.llaisysQwen2SeqCreate.restype = c_int64
    lib.llaisysQwen2SeqFork.argtypes = [M, c_int64]
    lib.llaisysQwen2SeqFork.restype = c_int64
    lib.llaisysQwen2SeqFree.argtypes = [M, c_int64]
    lib.llaisysQwen2SeqFree.restype = c_int
    lib.llaisysQwen2SeqLength.argtypes = [M, c_int64]
    lib.llaisysQwen2SeqLength.restype = c_int64
    lib.llaisysQwen2NumFreeBlocks.argtypes = [M]
    lib.llaisysQwen2NumFreeBlocks.restype = c_int64
    lib.llaisysQwen2ModelStep.argtypes = [M, POINTER(c_int64), c_size_t, POINTER(c_int64), POINTER(c_size_t),
                                          POINTER(c_int64)]
    lib.llaisysQwen2ModelStep.restype = c_int
    lib.llaisysQwen2ModelDecode.argtypes = [M, POINTER(c_int64), c_size_t, POINTER(c_int64), c_size_t,
                                            POINTER(c_int64)]
    lib.llaisysQwen2ModelDecode.restype = c_int
    lib.llaisysQwen2ModelLogits.argtypes = [M]
    lib.llaisysQwen2ModelLogits.restype = llaisysTensor_t
