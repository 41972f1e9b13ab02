#include "runtime_api.hpp"

#include "../common.hpp"

#include <cstdlib>

namespace llaisys::device {

// ---- CPU: plain malloc/memcpy, null stream (src/device/cpu/cpu_runtime_api.cpp:9-73).
namespace cpu {
int count() { return 1; }
void setDev(int) {}
void sync() {}
llaisysStream_t mkStream() { return nullptr; }
void rmStream(llaisysStream_t) {}
void syncStream(llaisysStream_t) {}
void *alloc(size_t n) { return std::malloc(n ? n : 1); }
void release(void *p) { std::free(p); }
void copy(void *dst, const void *src, size_t n, llaisysMemcpyKind_t) { std::memcpy(dst, src, n); }
void copyAsync(void *dst, const void *src, size_t n, llaisysMemcpyKind_t k, llaisysStream_t) { copy(dst, src, n, k); }
const LlaisysRuntimeAPI TABLE = {count, setDev, sync, mkStream, rmStream, syncStream,
                                 alloc, release, alloc, release, copy, copyAsync};
} // namespace cpu

// ---- Devices this build has no runtime for: zero devices, everything else raises
// (src/device/runtime_api.cpp:5-71).
namespace none {
int count() { return 0; }
[[noreturn]] void fail() { LLAISYS_RAISE("device type not supported by this build"); }
void setDev(int) { fail(); }
void sync() { fail(); }
llaisysStream_t mkStream() { fail(); }
void rmStream(llaisysStream_t) { fail(); }
void syncStream(llaisysStream_t) { fail(); }
void *alloc(size_t) { fail(); }
void release(void *) { fail(); }
void copy(void *, const void *, size_t, llaisysMemcpyKind_t) { fail(); }
void copyAsync(void *, const void *, size_t, llaisysMemcpyKind_t, llaisysStream_t) { fail(); }
const LlaisysRuntimeAPI TABLE = {count, setDev, sync, mkStream, rmStream, syncStream,
                                 alloc, release, alloc, release, copy, copyAsync};
} // namespace none

const LlaisysRuntimeAPI *cpuRuntimeAPI() { return &cpu::TABLE; }
const LlaisysRuntimeAPI *unsupportedRuntimeAPI() { return &none::TABLE; }

const LlaisysRuntimeAPI *getRuntimeAPI(llaisysDeviceType_t type) {
    switch (type) {
    case LLAISYS_DEVICE_CPU: return cpuRuntimeAPI();
    case LLAISYS_DEVICE_NVIDIA: return unsupportedRuntimeAPI();
    case LLAISYS_DEVICE_AMD: return hipRuntimeAPI();
    default: LLAISYS_RAISE("unknown device type " << int(type));
    }
}

} // namespace llaisys::device
