// Cross-lane exchanges by the gfx950 lane swaps: plain VALU, no LDS round
// trip as a ds_bpermute shuffle takes.
//
// v_permlane32_swap_b32 a, b exchanges lanes 32-63 of a with lanes 0-31 of b
// (v_permlane16_swap_b32 likewise rows 1 and 3 of a with rows 0 and 2 of b,
// rows being 16-lane groups). Both registers are results. They are written
// here as inline assembly with two in/out operands: the compiler's builtins
// for these instructions hand back the first register as both results (its
// second result reads the same value), so a reduction over the pair through
// them silently drops half the lanes. The s_nop pads keep the VALU write ->
// swap read distance that the instruction needs, whatever the compiler
// scheduled around the statement.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace llaisys::kernels {

__device__ __forceinline__ void laneSwap32(uint32_t &a, uint32_t &b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

__device__ __forceinline__ void laneSwap16(uint32_t &a, uint32_t &b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// The value lane l ^ 32 holds.
__device__ __forceinline__ float partner32(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    laneSwap32(a, b); // a: lanes 0-31 of x in both halves, b: lanes 32-63 in both
    return __builtin_bit_cast(float, (threadIdx.x & 32) ? a : b);
}

// Sum (Max) over lanes l, l ^ 16, l ^ 32, l ^ 48, the same value in all four:
// first the two halves (32 apart), then the two rows of each half.
__device__ __forceinline__ float sumOverGroups(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    laneSwap32(a, b);
    const float y = __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
    uint32_t c = __builtin_bit_cast(uint32_t, y), d = c;
    laneSwap16(c, d);
    return __builtin_bit_cast(float, c) + __builtin_bit_cast(float, d);
}

__device__ __forceinline__ float maxOverGroups(float x) {
    uint32_t a = __builtin_bit_cast(uint32_t, x), b = a;
    laneSwap32(a, b);
    const float y = fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
    uint32_t c = __builtin_bit_cast(uint32_t, y), d = c;
    laneSwap16(c, d);
    return fmaxf(__builtin_bit_cast(float, c), __builtin_bit_cast(float, d));
}

} // namespace llaisys::kernels
