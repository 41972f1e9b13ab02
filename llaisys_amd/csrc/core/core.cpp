#include "core.hpp"

#include "../common.hpp"
#include "../device/runtime_api.hpp"
#include "../kernels/launch.hpp"

#include <hip/hip_runtime.h>

namespace llaisys::core {

Storage::Storage(std::byte *mem, size_t size, const LlaisysRuntimeAPI *api, llaisysDeviceType_t type, int id,
                 bool is_host)
    : mem_(mem), size_(size), api_(api), type_(type), id_(id), is_host_(is_host) {}

Storage::~Storage() {
    try {
        if (is_host_) {
            api_->free_host(mem_);
        } else {
            api_->set_device(id_);
            api_->free_device(mem_);
        }
    } catch (...) {
        // Destructors must not throw; the error line is already on stderr.
    }
}

Runtime::Runtime(llaisysDeviceType_t type, int id) : type_(type), id_(id), api_(device::getRuntimeAPI(type)) {
    api_->set_device(id_);
    stream_ = api_->create_stream();
    if (type_ == LLAISYS_DEVICE_AMD) {
        // Per-device set-up: the error word exists from here on (entry points
        // never allocate it), and the allocation-free decode finds its scratch.
        errorWord();
        kernels::noAllocInit();
    }
}

Runtime::~Runtime() {
    try {
        api_->set_device(id_);
        if (type_ != LLAISYS_DEVICE_CPU) api_->device_synchronize();
        if (scratch_) api_->free_device(scratch_);
        if (slot_hdr_) api_->free_device(slot_hdr_);
        if (slot_rec_) api_->free_device(slot_rec_);
        if (error_word_) api_->free_device(error_word_);
        if (queue_counters_) api_->free_device(queue_counters_);
        if (flag_slots_) api_->free_host(flag_slots_);
        api_->destroy_stream(stream_);
    } catch (...) {
    }
}

void Runtime::activate() { api_->set_device(id_); }

storage_t Runtime::allocateDeviceStorage(size_t size) {
    auto *mem = static_cast<std::byte *>(api_->malloc_device(size));
    return std::make_shared<Storage>(mem, size, api_, type_, id_, false);
}

storage_t Runtime::allocateHostStorage(size_t size) {
    auto *mem = static_cast<std::byte *>(api_->malloc_host(size));
    return std::make_shared<Storage>(mem, size, api_, type_, id_, true);
}

void *Runtime::scratch(size_t bytes) {
    LLAISYS_CHECK(type_ == LLAISYS_DEVICE_AMD, "device workspace exists on AMD runtimes only");
    if (bytes > scratch_bytes_) {
        api_->device_synchronize();
        if (scratch_) api_->free_device(scratch_);
        size_t grown = std::max(bytes, scratch_bytes_ * 2);
        scratch_ = api_->malloc_device(grown);
        scratch_bytes_ = grown;
        ++ws_gen_;
    }
    return scratch_;
}

int *Runtime::decodeSlotHeaders(size_t header_ints) {
    LLAISYS_CHECK(type_ == LLAISYS_DEVICE_AMD, "device workspace exists on AMD runtimes only");
    if (header_ints > slot_hdr_ints_) {
        api_->device_synchronize();
        if (slot_hdr_) api_->free_device(slot_hdr_);
        const size_t grown = std::max(header_ints, slot_hdr_ints_ * 2);
        slot_hdr_ = static_cast<int *>(api_->malloc_device(grown * sizeof(int)));
        if (hipMemset(slot_hdr_, 0, grown * sizeof(int)) != hipSuccess) LLAISYS_RAISE("hipMemset failed");
        api_->device_synchronize();
        slot_hdr_ints_ = grown;
        ++ws_gen_;
    }
    return slot_hdr_;
}

void *Runtime::decodeSlotRecords(size_t record_bytes) {
    LLAISYS_CHECK(type_ == LLAISYS_DEVICE_AMD, "device workspace exists on AMD runtimes only");
    if (record_bytes > slot_rec_bytes_) {
        api_->device_synchronize();
        if (slot_rec_) api_->free_device(slot_rec_);
        const size_t grown = std::max(record_bytes, slot_rec_bytes_ * 2);
        slot_rec_ = api_->malloc_device(grown);
        slot_rec_bytes_ = grown;
        ++ws_gen_;
    }
    return slot_rec_;
}

int *Runtime::errorWord() {
    if (type_ == LLAISYS_DEVICE_CPU) return &host_error_word_;
    LLAISYS_CHECK(type_ == LLAISYS_DEVICE_AMD, "device workspace exists on AMD runtimes only");
    if (!error_word_) {
        error_word_ = static_cast<int *>(api_->malloc_device(sizeof(int)));
        if (hipMemset(error_word_, 0, sizeof(int)) != hipSuccess) LLAISYS_RAISE("hipMemset failed");
        api_->device_synchronize();
    }
    return error_word_;
}

int *Runtime::queueCounters() {
    LLAISYS_CHECK(type_ == LLAISYS_DEVICE_AMD, "device workspace exists on AMD runtimes only");
    if (!queue_counters_) {
        queue_counters_ = static_cast<int *>(api_->malloc_device(2 * sizeof(int)));
        if (hipMemset(queue_counters_, 0, 2 * sizeof(int)) != hipSuccess) LLAISYS_RAISE("hipMemset failed");
        api_->device_synchronize();
    }
    return queue_counters_;
}

int Runtime::takeErrorFlags() {
    const int pending = pending_error_flags_;
    pending_error_flags_ = 0;
    return pending | takeDeviceErrorFlags();
}

void Runtime::stashErrorFlags() { pending_error_flags_ |= takeDeviceErrorFlags(); }

void Runtime::flagSnapshotAsync(int slot) {
    LLAISYS_CHECK(type_ == LLAISYS_DEVICE_AMD && slot >= 0 && slot < 2, "flag snapshots: AMD runtimes, slots 0 and 1");
    int *word = errorWord();
    if (!flag_slots_) {
        flag_slots_ = static_cast<int *>(api_->malloc_host(2 * sizeof(int)));
        flag_slots_[0] = flag_slots_[1] = 0;
    }
    api_->memcpy_async(flag_slots_ + slot, word, sizeof(int), LLAISYS_MEMCPY_D2H, stream());
    if (hipMemsetAsync(word, 0, sizeof(int), static_cast<hipStream_t>(stream())) != hipSuccess)
        LLAISYS_RAISE("hipMemsetAsync failed");
}

int Runtime::flagSnapshot(int slot) const { return flag_slots_ && slot >= 0 && slot < 2 ? flag_slots_[slot] : 0; }

int Runtime::takeDeviceErrorFlags() {
    if (type_ == LLAISYS_DEVICE_CPU) return __atomic_exchange_n(&host_error_word_, 0, __ATOMIC_RELAXED);
    if (type_ != LLAISYS_DEVICE_AMD || !error_word_) return 0;
    int flags = 0;
    api_->stream_synchronize(stream());
    api_->memcpy_sync(&flags, error_word_, sizeof(int), LLAISYS_MEMCPY_D2H);
    if (flags) {
        int zero = 0;
        api_->memcpy_sync(error_word_, &zero, sizeof(int), LLAISYS_MEMCPY_H2D);
    }
    return flags;
}

Context::Context() {
    // Non-CPU device types first, CPU last; activate the first device found.
    std::vector<llaisysDeviceType_t> order;
    for (int t = 1; t < LLAISYS_DEVICE_TYPE_COUNT; ++t) order.push_back(static_cast<llaisysDeviceType_t>(t));
    order.push_back(LLAISYS_DEVICE_CPU);
    for (auto t : order) {
        int n = device::getRuntimeAPI(t)->get_device_count();
        runtimes_[t].resize(size_t(n > 0 ? n : 0));
        if (!current_ && n > 0) {
            runtimes_[t][0] = std::make_unique<Runtime>(t, 0);
            current_ = runtimes_[t][0].get();
        }
    }
}

Context::~Context() {
    current_ = nullptr;
    runtimes_.clear();
}

void Context::setDevice(llaisysDeviceType_t type, int id) {
    if (current_ && current_->deviceType() == type && current_->deviceId() == id) {
        current_->activate();
        return;
    }
    auto it = runtimes_.find(type);
    LLAISYS_CHECK(it != runtimes_.end(), "unknown device type " << int(type));
    auto &slots = it->second;
    LLAISYS_CHECK(id >= 0 && size_t(id) < slots.size(),
                  "invalid device id " << id << " for " << deviceName(type) << " (" << slots.size() << " present)");
    if (!slots[id]) slots[id] = std::make_unique<Runtime>(type, id);
    slots[id]->activate();
    current_ = slots[id].get();
}

Runtime &Context::runtime() {
    LLAISYS_CHECK(current_ != nullptr, "no runtime is active; call setDevice first");
    return *current_;
}

// Deliberately never destroyed: tearing down HIP streams from a thread-exit
// destructor can run after the HIP runtime itself has shut down.
Context &context() {
    thread_local Context *ctx = new Context();
    return *ctx;
}

} // namespace llaisys::core
