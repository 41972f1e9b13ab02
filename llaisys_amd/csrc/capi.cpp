// extern "C" glue: handle boxes around shared_ptr<Tensor> and one-line
// forwards (reference: src/llaisys/{tensor,runtime,ops}.cc,
// src/llaisys/llaisys_tensor.hpp:7-9). Every entry point catches exceptions:
// the message is already on stderr, is kept for llaisysGetLastError(), and the
// function returns its neutral value (NULL / 0 / nothing).
#include "llaisys/kv_cache.h"
#include "llaisys/ops.h"
#include "llaisys/runtime.h"
#include "llaisys/tensor.h"

#include "common.hpp"
#include "core/core.hpp"
#include "device/runtime_api.hpp"
#include "kvcache/block_manager.hpp"
#include "ops/ops.hpp"
#include "tensor/tensor.hpp"

#include <algorithm>
#include <string>

struct LlaisysTensor {
    llaisys::tensor_t tensor;
};

struct LlaisysKVBlockManager {
    llaisys::kvcache::BlockManager impl;
};

namespace {

thread_local std::string g_last_error;

template <typename F> auto guarded(F &&f, decltype(f()) fallback) -> decltype(f()) {
    try {
        return f();
    } catch (const std::exception &e) {
        g_last_error = e.what();
    } catch (...) {
        g_last_error = "unknown C++ exception";
    }
    return fallback;
}

template <typename F> void guardedVoid(F &&f) {
    try {
        f();
    } catch (const std::exception &e) {
        g_last_error = e.what();
    } catch (...) {
        g_last_error = "unknown C++ exception";
    }
}

llaisys::tensor_t unbox(llaisysTensor_t t, const char *what) {
    if (!t) LLAISYS_RAISE(what << ": null tensor handle");
    return t->tensor;
}
llaisys::tensor_t unboxOpt(llaisysTensor_t t) { return t ? t->tensor : nullptr; }

} // namespace

__C {

// ---------------- runtime.h
const LlaisysRuntimeAPI *llaisysGetRuntimeAPI(llaisysDeviceType_t type) {
    return guarded([&] { return llaisys::device::getRuntimeAPI(type); },
                   llaisys::device::unsupportedRuntimeAPI());
}

void llaisysSetContextRuntime(llaisysDeviceType_t type, int id) {
    guardedVoid([&] { llaisys::core::context().setDevice(type, id); });
}

llaisysStream_t llaisysGetContextStream(void) {
    return guarded([&] { return llaisys::core::context().runtime().stream(); }, llaisysStream_t(nullptr));
}

void llaisysSetContextStream(llaisysStream_t stream) {
    guardedVoid([&] { llaisys::core::context().runtime().setStreamOverride(stream); });
}

int llaisysGetLastError(char *buf, size_t buf_size) {
    if (g_last_error.empty()) return 0;
    if (buf && buf_size) {
        size_t n = std::min(buf_size - 1, g_last_error.size());
        std::memcpy(buf, g_last_error.data(), n);
        buf[n] = '\0';
    }
    g_last_error.clear();
    return 1;
}

int llaisysGetDeviceErrorFlags(void) {
    return guarded([&] { return llaisys::core::context().runtime().takeErrorFlags(); }, -1);
}

// ---------------- tensor.h
llaisysTensor_t tensorCreate(size_t *shape, size_t ndim, llaisysDataType_t dtype, llaisysDeviceType_t device_type,
                             int device_id) {
    return guarded(
        [&]() -> llaisysTensor_t {
            std::vector<size_t> s(shape, shape + ndim);
            return new LlaisysTensor{llaisys::Tensor::create(s, dtype, device_type, device_id)};
        },
        nullptr);
}

void tensorDestroy(llaisysTensor_t tensor) { delete tensor; }

void *tensorGetData(llaisysTensor_t t) {
    return guarded([&]() -> void * { return unbox(t, "tensorGetData")->data(); }, nullptr);
}

size_t tensorGetNdim(llaisysTensor_t t) {
    return guarded([&] { return unbox(t, "tensorGetNdim")->ndim(); }, size_t(0));
}

void tensorGetShape(llaisysTensor_t t, size_t *shape) {
    guardedVoid([&] {
        auto &s = unbox(t, "tensorGetShape")->shape();
        std::copy(s.begin(), s.end(), shape);
    });
}

void tensorGetStrides(llaisysTensor_t t, ptrdiff_t *strides) {
    guardedVoid([&] {
        auto &s = unbox(t, "tensorGetStrides")->strides();
        std::copy(s.begin(), s.end(), strides);
    });
}

llaisysDataType_t tensorGetDataType(llaisysTensor_t t) {
    return guarded([&] { return unbox(t, "tensorGetDataType")->dtype(); }, LLAISYS_DTYPE_INVALID);
}

llaisysDeviceType_t tensorGetDeviceType(llaisysTensor_t t) {
    return guarded([&] { return unbox(t, "tensorGetDeviceType")->deviceType(); }, LLAISYS_DEVICE_CPU);
}

int tensorGetDeviceId(llaisysTensor_t t) {
    return guarded([&] { return unbox(t, "tensorGetDeviceId")->deviceId(); }, -1);
}

void tensorDebug(llaisysTensor_t t) {
    guardedVoid([&] { unbox(t, "tensorDebug")->debug(); });
}

uint8_t tensorIsContiguous(llaisysTensor_t t) {
    return guarded([&] { return uint8_t(unbox(t, "tensorIsContiguous")->isContiguous()); }, uint8_t(0));
}

void tensorLoad(llaisysTensor_t t, const void *data) {
    guardedVoid([&] { unbox(t, "tensorLoad")->load(data); });
}

llaisysTensor_t tensorView(llaisysTensor_t t, size_t *shape, size_t ndim) {
    return guarded(
        [&]() -> llaisysTensor_t {
            std::vector<size_t> s(shape, shape + ndim);
            return new LlaisysTensor{unbox(t, "tensorView")->view(s)};
        },
        nullptr);
}

llaisysTensor_t tensorPermute(llaisysTensor_t t, size_t *order) {
    return guarded(
        [&]() -> llaisysTensor_t {
            auto tt = unbox(t, "tensorPermute");
            std::vector<size_t> o(order, order + tt->ndim());
            return new LlaisysTensor{tt->permute(o)};
        },
        nullptr);
}

llaisysTensor_t tensorSlice(llaisysTensor_t t, size_t dim, size_t start, size_t end) {
    return guarded([&]() -> llaisysTensor_t { return new LlaisysTensor{unbox(t, "tensorSlice")->slice(dim, start, end)}; },
                   nullptr);
}

// ---------------- ops.h
void llaisysAdd(llaisysTensor_t c, llaisysTensor_t a, llaisysTensor_t b) {
    guardedVoid([&] { llaisys::ops::add(unbox(c, "add"), unbox(a, "add"), unbox(b, "add")); });
}
void llaisysArgmax(llaisysTensor_t max_idx, llaisysTensor_t max_val, llaisysTensor_t vals) {
    guardedVoid([&] { llaisys::ops::argmax(unbox(max_idx, "argmax"), unboxOpt(max_val), unbox(vals, "argmax")); });
}
void llaisysEmbedding(llaisysTensor_t out, llaisysTensor_t index, llaisysTensor_t weight) {
    guardedVoid([&] {
        llaisys::ops::embedding(unbox(out, "embedding"), unbox(index, "embedding"), unbox(weight, "embedding"));
    });
}
void llaisysLinear(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t weight, llaisysTensor_t bias) {
    guardedVoid([&] {
        llaisys::ops::linear(unbox(out, "linear"), unbox(in, "linear"), unbox(weight, "linear"), unboxOpt(bias));
    });
}
void llaisysRearrange(llaisysTensor_t out, llaisysTensor_t in) {
    guardedVoid([&] { llaisys::ops::rearrange(unbox(out, "rearrange"), unbox(in, "rearrange")); });
}
void llaisysRmsNorm(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t weight, float eps) {
    guardedVoid([&] {
        llaisys::ops::rmsNorm(unbox(out, "rms_norm"), unbox(in, "rms_norm"), unbox(weight, "rms_norm"), eps);
    });
}
void llaisysROPE(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t pos_ids, float theta) {
    guardedVoid([&] { llaisys::ops::rope(unbox(out, "rope"), unbox(in, "rope"), unbox(pos_ids, "rope"), theta); });
}
void llaisysSwiGLU(llaisysTensor_t out, llaisysTensor_t gate, llaisysTensor_t up) {
    guardedVoid([&] { llaisys::ops::swiglu(unbox(out, "swiglu"), unbox(gate, "swiglu"), unbox(up, "swiglu")); });
}

void llaisysSelfAttention(llaisysTensor_t attn_val, llaisysTensor_t q, llaisysTensor_t k, llaisysTensor_t v,
                          float scale) {
    guardedVoid([&] {
        llaisys::ops::selfAttention(unbox(attn_val, "self_attention"), unbox(q, "self_attention"),
                                    unbox(k, "self_attention"), unbox(v, "self_attention"), scale);
    });
}

void llaisysPagedKVAppend(llaisysTensor_t k_pool, llaisysTensor_t v_pool, llaisysTensor_t k_new, llaisysTensor_t v_new,
                          llaisysTensor_t block_table, llaisysTensor_t ctx_len, llaisysTensor_t cu_new) {
    guardedVoid([&] {
        const char *w = "paged_kv_append";
        llaisys::ops::pagedKVAppend(unbox(k_pool, w), unbox(v_pool, w), unbox(k_new, w), unbox(v_new, w),
                                    unbox(block_table, w), unbox(ctx_len, w), unboxOpt(cu_new));
    });
}

void llaisysPagedKVGather(llaisysTensor_t k_out, llaisysTensor_t v_out, llaisysTensor_t k_pool, llaisysTensor_t v_pool,
                          llaisysTensor_t block_table, llaisysTensor_t cu_seqlens) {
    guardedVoid([&] {
        const char *w = "paged_kv_gather";
        llaisys::ops::pagedKVGather(unbox(k_out, w), unbox(v_out, w), unbox(k_pool, w), unbox(v_pool, w),
                                    unbox(block_table, w), unbox(cu_seqlens, w));
    });
}

void llaisysPagedAttention(llaisysTensor_t out, llaisysTensor_t q, llaisysTensor_t k_pool, llaisysTensor_t v_pool,
                           llaisysTensor_t block_table, llaisysTensor_t ctx_len, float scale) {
    guardedVoid([&] {
        const char *w = "paged_attention";
        llaisys::ops::pagedAttention(unbox(out, w), unbox(q, w), unbox(k_pool, w), unbox(v_pool, w),
                                     unbox(block_table, w), unbox(ctx_len, w), nullptr, scale);
    });
}

void llaisysPagedAttentionVarlen(llaisysTensor_t out, llaisysTensor_t q, llaisysTensor_t k_pool,
                                 llaisysTensor_t v_pool, llaisysTensor_t block_table, llaisysTensor_t cu_q,
                                 llaisysTensor_t ctx_len, float scale) {
    guardedVoid([&] {
        const char *w = "paged_attention_varlen";
        llaisys::ops::pagedAttention(unbox(out, w), unbox(q, w), unbox(k_pool, w), unbox(v_pool, w),
                                     unbox(block_table, w), unbox(ctx_len, w), unbox(cu_q, w), scale);
    });
}

void llaisysPagedKVCopyBlocks(llaisysTensor_t k_pool, llaisysTensor_t v_pool, llaisysTensor_t pairs) {
    guardedVoid([&] {
        const char *w = "paged_kv_copy_blocks";
        llaisys::ops::pagedKVCopyBlocks(unbox(k_pool, w), unbox(v_pool, w), unbox(pairs, w));
    });
}

// ---------------- kv_cache.h
namespace {
llaisys::kvcache::BlockManager &mgr(llaisysKVBlockManager_t m) {
    if (!m) LLAISYS_RAISE("kv block manager: null handle");
    return m->impl;
}
} // namespace

llaisysKVBlockManager_t llaisysKVBlockManagerCreate(int num_blocks) {
    return guarded([&]() -> llaisysKVBlockManager_t { return new LlaisysKVBlockManager{llaisys::kvcache::BlockManager(num_blocks)}; },
                   nullptr);
}

void llaisysKVBlockManagerDestroy(llaisysKVBlockManager_t m) { delete m; }

int llaisysKVNumFreeBlocks(llaisysKVBlockManager_t m) {
    return guarded([&] { return mgr(m).numFree(); }, -1);
}

int llaisysKVSeqCreate(llaisysKVBlockManager_t m, int64_t seq_id, const int64_t *tokens, size_t ntokens) {
    return guarded([&] { return mgr(m).create(seq_id, tokens, ntokens); }, -1);
}

int llaisysKVSeqFork(llaisysKVBlockManager_t m, int64_t parent, int64_t child) {
    return guarded([&] { mgr(m).fork(parent, child); return 0; }, -1);
}

int llaisysKVSeqReserve(llaisysKVBlockManager_t m, int64_t seq_id, int ntokens, int32_t *cow_pairs, int cow_capacity) {
    return guarded([&] { return mgr(m).reserve(seq_id, ntokens, cow_pairs, cow_capacity); }, -1);
}

int llaisysKVSeqCommit(llaisysKVBlockManager_t m, int64_t seq_id, int ntokens, const int64_t *tokens) {
    return guarded([&] { mgr(m).commit(seq_id, ntokens, tokens); return 0; }, -1);
}

int llaisysKVSeqFree(llaisysKVBlockManager_t m, int64_t seq_id) {
    return guarded([&] { mgr(m).release(seq_id); return 0; }, -1);
}

int llaisysKVSeqLength(llaisysKVBlockManager_t m, int64_t seq_id) {
    return guarded([&] { return mgr(m).length(seq_id); }, -1);
}

int llaisysKVBuildBlockTable(llaisysKVBlockManager_t m, const int64_t *seq_ids, size_t B, int32_t *table,
                             size_t max_pages, int32_t *ctx_len) {
    return guarded([&] { return mgr(m).buildTable(seq_ids, B, table, max_pages, ctx_len); }, -1);
}

} // extern "C"
