"""Prototypes of the test hooks (include/llaisys/testing.h): the decode step's
fused kernels called alone on device pointers."""
from ctypes import c_float, c_int, c_void_p


def load_testing(lib):
    P, I, F = c_void_p, c_int, c_float
    for name, args in [
        ("llaisysTestPackWeight", [P, P, P, I, I]),
        ("llaisysTestPackWeightGateUp", [P, P, I, I]),
        ("llaisysTestPackedXGemm", [P, P, P, I, I, I, I, P]),
        ("llaisysTestQkvRopeGemm", [P, P, P, P, P, P, P, P, I, I, I, I, I, I, F, F]),
        ("llaisysTestGateUpSwiglu", [P, P, P, I, I, I, F, I]),
        ("llaisysTestSplitKPackedGemm", [P, P, P, I, I, I, I, P]),
        ("llaisysTestSwigluInterleave", [P, P, I, I]),
        ("llaisysTestLinearSwiglu", [P, P, P, I, I, I]),
    ]:
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = None
