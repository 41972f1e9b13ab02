#pragma once

#include "../common.hpp"

#include <hip/hip_runtime.h>

#define HIP_CHECK(expr)                                                                   \
    do {                                                                                  \
        hipError_t e__ = (expr);                                                          \
        if (e__ != hipSuccess) LLAISYS_RAISE("HIP error " << hipGetErrorName(e__) << " (" \
                                             << hipGetErrorString(e__) << ") from " #expr); \
    } while (0)
