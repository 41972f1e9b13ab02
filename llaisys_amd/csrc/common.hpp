// Error reporting and dtype helpers shared by every translation unit.
//
// Error convention follows the reference's src/utils/check.hpp:4-88: a failed
// check prints "[ERROR] <message> at <file>:<line>" to stderr and throws. The
// C-ABI layer (capi.cpp) catches the exception, so a ctypes caller gets the
// stderr line plus llaisysGetLastError() instead of a process abort.
#pragma once

#include "llaisys.h"

#include <cstdint>
#include <cstring>
#include <sstream>
#include <stdexcept>
#include <string>

namespace llaisys {

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void raise(const std::string &msg, const char *file, int line);

const char *dtypeName(llaisysDataType_t dt);
const char *deviceName(llaisysDeviceType_t dev);
size_t dsize(llaisysDataType_t dt);

// bf16 <-> f32. Widening is exact (bits << 16). Narrowing is round to nearest
// even, as src/utils/types.cpp:74-84, with NaN kept quiet.
inline float bf16ToF32(uint16_t h) {
    uint32_t u = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
inline uint16_t f32ToBf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
}
float f16ToF32(uint16_t h);

} // namespace llaisys

#define LLAISYS_RAISE(msg)                                   \
    do {                                                     \
        std::ostringstream os__;                             \
        os__ << msg;                                         \
        ::llaisys::raise(os__.str(), __FILE__, __LINE__);    \
    } while (0)

#define LLAISYS_CHECK(cond, msg)                                        \
    do {                                                                \
        if (!(cond)) LLAISYS_RAISE(msg << " [check: " #cond "]");       \
    } while (0)
