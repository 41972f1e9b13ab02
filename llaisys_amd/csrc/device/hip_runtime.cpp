// HIP runtime for LLAISYS_DEVICE_AMD: fills the 12-entry LlaisysRuntimeAPI
// (include/llaisys/runtime.h:25-38) the reference's CPU table
// (src/device/cpu/cpu_runtime_api.cpp:56-68) shows the shape of.
//
// Host memory is pinned (hipHostMalloc) so H2D/D2H copies run at full PCIe
// rate. memcpy_sync waits for the whole device first: the reference's tests
// copy results out straight after an op with no explicit sync
// (test/test_utils.py:143-149), so a synchronous copy must order after every
// kernel already queued on any stream.
#include "hip_check.hpp"
#include "runtime_api.hpp"

namespace llaisys::device {
namespace hip {

int count() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}
void setDev(int id) { HIP_CHECK(hipSetDevice(id)); }
void sync() { HIP_CHECK(hipDeviceSynchronize()); }
llaisysStream_t mkStream() {
    hipStream_t s = nullptr;
    HIP_CHECK(hipStreamCreate(&s));
    return s;
}
void rmStream(llaisysStream_t s) {
    if (s) HIP_CHECK(hipStreamDestroy(static_cast<hipStream_t>(s)));
}
void syncStream(llaisysStream_t s) { HIP_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(s))); }
void *allocDevice(size_t n) {
    void *p = nullptr;
    HIP_CHECK(hipMalloc(&p, n ? n : 1));
    return p;
}
void freeDevice(void *p) {
    if (p) HIP_CHECK(hipFree(p));
}
void *allocHost(size_t n) {
    void *p = nullptr;
    HIP_CHECK(hipHostMalloc(&p, n ? n : 1, hipHostMallocDefault));
    return p;
}
void freeHost(void *p) {
    if (p) HIP_CHECK(hipHostFree(p));
}
hipMemcpyKind kindOf(llaisysMemcpyKind_t k) {
    switch (k) {
    case LLAISYS_MEMCPY_H2H: return hipMemcpyHostToHost;
    case LLAISYS_MEMCPY_H2D: return hipMemcpyHostToDevice;
    case LLAISYS_MEMCPY_D2H: return hipMemcpyDeviceToHost;
    case LLAISYS_MEMCPY_D2D: return hipMemcpyDeviceToDevice;
    }
    LLAISYS_RAISE("bad memcpy kind " << int(k));
}
void copy(void *dst, const void *src, size_t n, llaisysMemcpyKind_t k) {
    HIP_CHECK(hipDeviceSynchronize());
    if (n) HIP_CHECK(hipMemcpy(dst, src, n, kindOf(k)));
}
void copyAsync(void *dst, const void *src, size_t n, llaisysMemcpyKind_t k, llaisysStream_t s) {
    if (n) HIP_CHECK(hipMemcpyAsync(dst, src, n, kindOf(k), static_cast<hipStream_t>(s)));
}

const LlaisysRuntimeAPI TABLE = {count, setDev, sync, mkStream, rmStream, syncStream,
                                 allocDevice, freeDevice, allocHost, freeHost, copy, copyAsync};
} // namespace hip

const LlaisysRuntimeAPI *hipRuntimeAPI() { return &hip::TABLE; }

} // namespace llaisys::device
