/*
 * LLAISYS C-ABI base types, MI355X build.
 *
 * Same enums, values and export macro as the reference's include/llaisys.h:1-66
 * so that the reference's ctypes layer (python/llaisys/libllaisys/llaisys_types.py)
 * binds unchanged. One addition: LLAISYS_DEVICE_AMD = 2, appended after NVIDIA as
 * the reference asks device numbers to stay consecutive (include/llaisys.h:25).
 */
#ifndef LLAISYS_H
#define LLAISYS_H

#if defined(__GNUC__)
#define __export __attribute__((visibility("default")))
#else
#define __export
#endif

#ifdef __cplusplus
#define __C extern "C"
#include <cstddef>
#include <cstdint>
#else
#define __C
#include <stddef.h>
#include <stdint.h>
#endif

typedef enum {
    LLAISYS_DEVICE_CPU = 0,
    LLAISYS_DEVICE_NVIDIA = 1, /* kept so numbering matches; always reports 0 devices here */
    LLAISYS_DEVICE_AMD = 2,    /* MI355X (gfx950) through HIP */
    LLAISYS_DEVICE_TYPE_COUNT
} llaisysDeviceType_t;

typedef enum {
    LLAISYS_DTYPE_INVALID = 0,
    LLAISYS_DTYPE_BYTE = 1,
    LLAISYS_DTYPE_BOOL = 2,
    LLAISYS_DTYPE_I8 = 3,
    LLAISYS_DTYPE_I16 = 4,
    LLAISYS_DTYPE_I32 = 5,
    LLAISYS_DTYPE_I64 = 6,
    LLAISYS_DTYPE_U8 = 7,
    LLAISYS_DTYPE_U16 = 8,
    LLAISYS_DTYPE_U32 = 9,
    LLAISYS_DTYPE_U64 = 10,
    LLAISYS_DTYPE_F8 = 11,
    LLAISYS_DTYPE_F16 = 12,
    LLAISYS_DTYPE_F32 = 13,
    LLAISYS_DTYPE_F64 = 14,
    LLAISYS_DTYPE_C16 = 15,
    LLAISYS_DTYPE_C32 = 16,
    LLAISYS_DTYPE_C64 = 17,
    LLAISYS_DTYPE_C128 = 18,
    LLAISYS_DTYPE_BF16 = 19,
} llaisysDataType_t;

typedef void *llaisysStream_t;

typedef enum {
    LLAISYS_MEMCPY_H2H = 0,
    LLAISYS_MEMCPY_H2D = 1,
    LLAISYS_MEMCPY_D2H = 2,
    LLAISYS_MEMCPY_D2D = 3,
} llaisysMemcpyKind_t;

#endif /* LLAISYS_H */
