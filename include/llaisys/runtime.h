/*
 * Device runtime function table. Layout and order are the reference's
 * include/llaisys/runtime.h:25-38 (12 function pointers) so that
 * python/llaisys/libllaisys/runtime.py:24-38 reads it unchanged.
 * For LLAISYS_DEVICE_AMD the table is filled by the HIP runtime.
 */
#ifndef LLAISYS_RUNTIME_H
#define LLAISYS_RUNTIME_H

#include "../llaisys.h"

__C {
    typedef int (*get_device_count_api)(void);
    typedef void (*set_device_api)(int);
    typedef void (*device_synchronize_api)(void);
    typedef llaisysStream_t (*create_stream_api)(void);
    typedef void (*destroy_stream_api)(llaisysStream_t);
    typedef void (*stream_synchronize_api)(llaisysStream_t);
    typedef void *(*malloc_device_api)(size_t);
    typedef void (*free_device_api)(void *);
    typedef void *(*malloc_host_api)(size_t);
    typedef void (*free_host_api)(void *);
    typedef void (*memcpy_sync_api)(void *, const void *, size_t, llaisysMemcpyKind_t);
    typedef void (*memcpy_async_api)(void *, const void *, size_t, llaisysMemcpyKind_t, llaisysStream_t);

    struct LlaisysRuntimeAPI {
        get_device_count_api get_device_count;
        set_device_api set_device;
        device_synchronize_api device_synchronize;
        create_stream_api create_stream;
        destroy_stream_api destroy_stream;
        stream_synchronize_api stream_synchronize;
        malloc_device_api malloc_device;
        free_device_api free_device;
        malloc_host_api malloc_host;
        free_host_api free_host;
        memcpy_sync_api memcpy_sync;
        memcpy_async_api memcpy_async;
    };

    /* Replaces include/llaisys/runtime.h:41. */
    __export const struct LlaisysRuntimeAPI *llaisysGetRuntimeAPI(llaisysDeviceType_t);

    /* Replaces include/llaisys/runtime.h:44. */
    __export void llaisysSetContextRuntime(llaisysDeviceType_t, int);

    /* New (no reference counterpart): the stream the calling thread's active
     * runtime launches kernels on, so callers can order their own work and
     * time kernels with events on it. */
    __export llaisysStream_t llaisysGetContextStream(void);

    /* New (no reference counterpart): make the calling thread's active runtime
     * launch on `stream` (NULL restores the runtime's own stream). */
    __export void llaisysSetContextStream(llaisysStream_t stream);

    /* New (no reference counterpart). The reference lets C++ exceptions escape
     * its extern "C" functions, which aborts a ctypes caller. Here every entry
     * point catches them, prints the same "[ERROR] ..." line to stderr and
     * records the message; this returns 1 and copies the message (clearing it)
     * if the calling thread's last call failed, else 0. */
    __export int llaisysGetLastError(char *buf, size_t buf_size);

    /* New (no reference counterpart): OR of the kernel-side error bits the
     * active AMD runtime has recorded (1 = block id outside the pool,
     * 2 = context longer than the block table), clearing them. Synchronises
     * the runtime's stream. 0 on CPU. */
    __export int llaisysGetDeviceErrorFlags(void);
}

#endif /* LLAISYS_RUNTIME_H */
