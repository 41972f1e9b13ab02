#include "common.hpp"

#include <iostream>

namespace llaisys {

void raise(const std::string &msg, const char *file, int line) {
    std::ostringstream os;
    os << msg << " at " << file << ":" << line;
    std::cerr << "[ERROR] " << os.str() << std::endl;
    throw Error(os.str());
}

const char *dtypeName(llaisysDataType_t dt) {
    switch (dt) {
    case LLAISYS_DTYPE_BYTE: return "byte";
    case LLAISYS_DTYPE_BOOL: return "bool";
    case LLAISYS_DTYPE_I8: return "i8";
    case LLAISYS_DTYPE_I16: return "i16";
    case LLAISYS_DTYPE_I32: return "i32";
    case LLAISYS_DTYPE_I64: return "i64";
    case LLAISYS_DTYPE_U8: return "u8";
    case LLAISYS_DTYPE_U16: return "u16";
    case LLAISYS_DTYPE_U32: return "u32";
    case LLAISYS_DTYPE_U64: return "u64";
    case LLAISYS_DTYPE_F8: return "f8";
    case LLAISYS_DTYPE_F16: return "f16";
    case LLAISYS_DTYPE_F32: return "f32";
    case LLAISYS_DTYPE_F64: return "f64";
    case LLAISYS_DTYPE_C16: return "c16";
    case LLAISYS_DTYPE_C32: return "c32";
    case LLAISYS_DTYPE_C64: return "c64";
    case LLAISYS_DTYPE_C128: return "c128";
    case LLAISYS_DTYPE_BF16: return "bf16";
    default: return "invalid";
    }
}

const char *deviceName(llaisysDeviceType_t dev) {
    switch (dev) {
    case LLAISYS_DEVICE_CPU: return "cpu";
    case LLAISYS_DEVICE_NVIDIA: return "nvidia";
    case LLAISYS_DEVICE_AMD: return "amd";
    default: return "unknown";
    }
}

// Element sizes as src/utils/types.hpp:18-62.
size_t dsize(llaisysDataType_t dt) {
    switch (dt) {
    case LLAISYS_DTYPE_BYTE:
    case LLAISYS_DTYPE_BOOL:
    case LLAISYS_DTYPE_I8:
    case LLAISYS_DTYPE_U8:
    case LLAISYS_DTYPE_F8: return 1;
    case LLAISYS_DTYPE_I16:
    case LLAISYS_DTYPE_U16:
    case LLAISYS_DTYPE_F16:
    case LLAISYS_DTYPE_BF16:
    case LLAISYS_DTYPE_C16: return 2;
    case LLAISYS_DTYPE_I32:
    case LLAISYS_DTYPE_U32:
    case LLAISYS_DTYPE_F32:
    case LLAISYS_DTYPE_C32: return 4;
    case LLAISYS_DTYPE_I64:
    case LLAISYS_DTYPE_U64:
    case LLAISYS_DTYPE_F64:
    case LLAISYS_DTYPE_C64: return 8;
    case LLAISYS_DTYPE_C128: return 16;
    default: LLAISYS_RAISE("unsupported data type " << int(dt));
    }
}

// IEEE binary16 -> binary32, exact (subnormals renormalised).
float f16ToF32(uint16_t h) {
    uint32_t sign = uint32_t(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do {
                man <<= 1;
                ++e;
            } while ((man & 0x400u) == 0);
            bits = sign | uint32_t(127 - 15 - e) << 23 | ((man & 0x3ffu) << 13);
        }
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

} // namespace llaisys
