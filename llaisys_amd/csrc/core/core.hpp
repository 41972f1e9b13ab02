// Storage, per-device Runtime and the thread-local Context.
//
// Behaviour follows the reference's src/core/{storage,runtime,context}:
//  * a Storage owns one buffer and frees it through the runtime table that
//    allocated it (storage.cpp:9-11);
//  * a Runtime is one (device type, id): its table, one stream, allocation
//    (runtime.cpp:7-12, :49-55);
//  * the Context is thread-local and activates the first non-CPU device found,
//    else CPU (context.cpp:7-32, :74-77).
// Two reference hazards are avoided: the current-runtime pointer starts null
// (context.hpp:16 leaves it uninitialised) and lazily created runtimes are
// stored back into the map (context.cpp:55-62 mutates a copy).
//
// The AMD runtime also owns the device workspace the attention kernels use:
// split-KV partial results and an error word.
#pragma once

#include <atomic>

#include "llaisys/runtime.h"

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <vector>

namespace llaisys::core {

class Storage {
public:
    Storage(std::byte *mem, size_t size, const LlaisysRuntimeAPI *api, llaisysDeviceType_t type, int id,
            bool is_host);
    ~Storage();
    Storage(const Storage &) = delete;
    Storage &operator=(const Storage &) = delete;

    std::byte *memory() const { return mem_; }
    size_t size() const { return size_; }
    bool isHost() const { return is_host_; }
    // Host storage reports CPU/0, as storage.cpp:21-35.
    llaisysDeviceType_t deviceType() const { return is_host_ ? LLAISYS_DEVICE_CPU : type_; }
    int deviceId() const { return is_host_ ? 0 : id_; }
    // Write generation: bumped by every write the library cannot see (a load
    // from the host, a raw data pointer handed out through the C-API), so
    // copies derived from the bytes (folded model weights) know to refresh.
    uint64_t version() const { return version_.load(std::memory_order_relaxed); }
    void touch() { version_.fetch_add(1, std::memory_order_relaxed); }

private:
    std::atomic<uint64_t> version_{0};
    std::byte *mem_;
    size_t size_;
    const LlaisysRuntimeAPI *api_;
    llaisysDeviceType_t type_;
    int id_;
    bool is_host_;
};
using storage_t = std::shared_ptr<Storage>;

class Runtime {
public:
    Runtime(llaisysDeviceType_t type, int id);
    ~Runtime();
    Runtime(const Runtime &) = delete;
    Runtime &operator=(const Runtime &) = delete;

    llaisysDeviceType_t deviceType() const { return type_; }
    int deviceId() const { return id_; }
    const LlaisysRuntimeAPI *api() const { return api_; }

    // Stream ops launch on: the override if one is set, else the runtime's own.
    llaisysStream_t stream() const { return override_stream_ ? override_stream_ : stream_; }
    void setStreamOverride(llaisysStream_t s) { override_stream_ = s; }

    storage_t allocateDeviceStorage(size_t size);
    storage_t allocateHostStorage(size_t size);

    // Device workspace (AMD only). Grow-only; growing waits for the device.
    void *scratch(size_t bytes);
    // Persistent device buffers of the decode attention's per-unit record
    // slots: the headers (at least header_ints int32, zeroed when allocated;
    // kernels leave them at zero after every call) and the records (at least
    // record_bytes). Separate allocations, so records never land on headers
    // whatever the batch shape of a call. Grow-only.
    int *decodeSlotHeaders(size_t header_ints);
    void *decodeSlotRecords(size_t record_bytes);
    // Bumped whenever scratch() or the slot buffers move: captured graphs that
    // baked the old addresses in must be re-captured.
    uint64_t workspaceGeneration() const { return ws_gen_; }
    // One int32 of kernel-side error bits (device memory on AMD; on CPU a host
    // word the host ops raise bits in, read and cleared the same way).
    int *errorWord();
    // Two int32 work-queue counters for persistent kernels, zeroed once; the
    // kernels return them to zero before they end.
    int *queueCounters();
    // Bits raised since the last call (llaisysGetDeviceErrorFlags), then zero.
    int takeErrorFlags();
    // For callers that check their own launches' bits (the model): first move
    // the bits raised so far into a host-side pending word (waits for the
    // stream), then, after their launches, read and clear the device word
    // alone. The pending bits stay for takeErrorFlags().
    void stashErrorFlags();
    int takeDeviceErrorFlags();
    // The same split without waiting (AMD runtimes): flagSnapshotAsync(i)
    // enqueues on the stream a copy of the device word into pinned host slot
    // i (of 2) and the word's clearing; once the caller has synchronised the
    // stream, flagSnapshot(i) holds the bits. addPendingErrorFlags keeps bits
    // for takeErrorFlags(), as stashErrorFlags does.
    void flagSnapshotAsync(int slot);
    int flagSnapshot(int slot) const;
    void addPendingErrorFlags(int bits) { pending_error_flags_ |= bits; }

    void activate();

private:
    llaisysDeviceType_t type_;
    int id_;
    const LlaisysRuntimeAPI *api_;
    llaisysStream_t stream_ = nullptr;
    llaisysStream_t override_stream_ = nullptr;
    void *scratch_ = nullptr;
    size_t scratch_bytes_ = 0;
    int *error_word_ = nullptr;
    int *queue_counters_ = nullptr;
    int host_error_word_ = 0;
    int pending_error_flags_ = 0; // stashed by stashErrorFlags(), returned by takeErrorFlags()
    int *flag_slots_ = nullptr;   // pinned host, 2 ints (flagSnapshotAsync)
    int *slot_hdr_ = nullptr;
    size_t slot_hdr_ints_ = 0;
    void *slot_rec_ = nullptr;
    size_t slot_rec_bytes_ = 0;
    uint64_t ws_gen_ = 0;
};

class Context {
public:
    Context();
    ~Context();
    void setDevice(llaisysDeviceType_t type, int id);
    Runtime &runtime();

private:
    std::map<llaisysDeviceType_t, std::vector<std::unique_ptr<Runtime>>> runtimes_;
    Runtime *current_ = nullptr;
};

Context &context();

} // namespace llaisys::core
