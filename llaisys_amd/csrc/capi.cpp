// extern "C" glue: handle boxes around shared_ptr<Tensor> and one-line
// forwards (reference: src/llaisys/{tensor,runtime,ops}.cc,
// src/llaisys/llaisys_tensor.hpp:7-9). Every entry point catches exceptions:
// the message is already on stderr, is kept for llaisysGetLastError(), and the
// function returns its neutral value (NULL / 0 / nothing).
#include "llaisys/kv_cache.h"
#include "llaisys/models/qwen2.h"
#include "llaisys/ops.h"
#include "llaisys/runtime.h"
#include "llaisys/serving.h"
#include "llaisys/tensor.h"
#include "llaisys/testing.h"

#include "common.hpp"
#include "device/hip_check.hpp"
#include "kernels/launch.hpp"
#include "core/core.hpp"
#include "device/runtime_api.hpp"
#include "kvcache/block_manager.hpp"
#include "models/qwen2.hpp"
#include "ops/ops.hpp"
#include "serving/scheduler.hpp"
#include "tensor/tensor.hpp"

#include <algorithm>
#include <memory>
#include <string>
#include <vector>

struct LlaisysTensor {
    llaisys::tensor_t tensor;
};

struct LlaisysKVBlockManager {
    llaisys::kvcache::BlockManager impl;
};

// The model plus the handle boxes of its weights. `orig` keeps the boxes the
// model handed out, so handles a caller swapped into `w` can be detected and
// copied into the model's own tensors.
struct LlaisysScheduler {
    std::unique_ptr<llaisys::serving::Backend> backend;
    std::unique_ptr<llaisys::serving::Scheduler> sched; // destroyed first
    ~LlaisysScheduler() { sched.reset(); }
};

struct LlaisysQwen2Model {
    std::unique_ptr<llaisys::models::Qwen2Model> impl;
    LlaisysQwen2Weights w{};
    LlaisysQwen2Weights orig{};
    std::vector<std::unique_ptr<LlaisysTensor>> owned;
    std::vector<std::vector<llaisysTensor_t>> arrays, orig_arrays; // 12 per-layer arrays
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

// Per-layer weight slots of LlaisysQwen2Weights in declaration order.
constexpr int kQwen2LayerSlots = 12;
llaisysTensor_t *&layerSlot(LlaisysQwen2Weights &w, int k) {
    llaisysTensor_t **slots[kQwen2LayerSlots] = {&w.attn_norm_w, &w.attn_q_w, &w.attn_q_b,  &w.attn_k_w,
                                                 &w.attn_k_b,    &w.attn_v_w, &w.attn_v_b,  &w.attn_o_w,
                                                 &w.mlp_norm_w,  &w.mlp_gate_w, &w.mlp_up_w, &w.mlp_down_w};
    return *slots[k];
}

llaisys::tensor_t layerTensor(const llaisys::models::Qwen2LayerWeights &L, int k) {
    const llaisys::tensor_t *t[kQwen2LayerSlots] = {&L.attn_norm, &L.q_w, &L.q_b, &L.k_w, &L.k_b, &L.v_w,
                                                    &L.v_b,       &L.o_w, &L.mlp_norm, &L.gate_w, &L.up_w, &L.down_w};
    return *t[k];
}

LlaisysQwen2Model *createQwen2(const LlaisysQwen2Meta *meta, llaisysDeviceType_t device, const int *device_ids,
                               int ndevice, size_t num_blocks) {
    LLAISYS_CHECK(meta, "qwen2: null meta");
    LLAISYS_CHECK(device == LLAISYS_DEVICE_AMD, "qwen2: llaisys_amd runs the model on LLAISYS_DEVICE_AMD only");
    LLAISYS_CHECK(ndevice == 1, "qwen2: one device per model (got " << ndevice << ")");
    const int id = device_ids ? device_ids[0] : 0;
    llaisys::models::Qwen2Config cfg{meta->dtype, meta->nlayer, meta->hs,     meta->nh,    meta->nkvh, meta->dh,
                                     meta->di,    meta->maxseq, meta->voc,    meta->epsilon, meta->theta,
                                     meta->end_token};
    if (num_blocks == 0) num_blocks = (meta->maxseq + 15) / 16 + 1;
    auto m = std::make_unique<LlaisysQwen2Model>();
    m->impl = std::make_unique<llaisys::models::Qwen2Model>(cfg, id, num_blocks);
    auto box = [&](const llaisys::tensor_t &t) {
        m->owned.push_back(std::make_unique<LlaisysTensor>(LlaisysTensor{t}));
        return m->owned.back().get();
    };
    m->w.in_embed = box(m->impl->inEmbed());
    m->w.out_embed = box(m->impl->outEmbed());
    m->w.out_norm_w = box(m->impl->outNorm());
    m->arrays.assign(kQwen2LayerSlots, std::vector<llaisysTensor_t>(cfg.nlayer));
    for (int k = 0; k < kQwen2LayerSlots; ++k) {
        for (size_t l = 0; l < cfg.nlayer; ++l) m->arrays[k][l] = box(layerTensor(m->impl->layer(l), k));
        layerSlot(m->w, k) = m->arrays[k].data();
    }
    m->orig = m->w;
    m->orig_arrays = m->arrays;
    return m.release();
}

// Copy a caller-supplied tensor into the model's own and restore the slot.
void adopt(llaisysTensor_t &slot, llaisysTensor_t own) {
    if (slot == own || slot == nullptr) {
        slot = own;
        return;
    }
    const auto &src = slot->tensor;
    const auto &dst = own->tensor;
    LLAISYS_CHECK(src->shape() == dst->shape() && src->dtype() == dst->dtype(),
                  "qwen2: replaced weight " << src->info() << " does not match " << dst->info());
    LLAISYS_CHECK(src->isContiguous(), "qwen2: replaced weight must be contiguous");
    auto &ctx = llaisys::core::context();
    ctx.setDevice(dst->deviceType(), dst->deviceId());
    const size_t bytes = dst->numel() * dst->elementSize();
    const auto kind = src->deviceType() == LLAISYS_DEVICE_CPU ? LLAISYS_MEMCPY_H2D : LLAISYS_MEMCPY_D2D;
    if (bytes) ctx.runtime().api()->memcpy_sync(dst->data(), src->data(), bytes, kind);
    slot = own;
}

void syncWeights(LlaisysQwen2Model &m) {
    adopt(m.w.in_embed, m.orig.in_embed);
    adopt(m.w.out_embed, m.orig.out_embed);
    adopt(m.w.out_norm_w, m.orig.out_norm_w);
    for (int k = 0; k < kQwen2LayerSlots; ++k) {
        llaisysTensor_t *arr = layerSlot(m.w, k);
        if (arr != m.arrays[k].data()) { // caller swapped the whole array
            for (size_t l = 0; l < m.arrays[k].size(); ++l) m.arrays[k][l] = arr[l];
            layerSlot(m.w, k) = m.arrays[k].data();
        }
        for (size_t l = 0; l < m.arrays[k].size(); ++l) adopt(m.arrays[k][l], m.orig_arrays[k][l]);
    }
}

llaisys::models::Qwen2Model &model(LlaisysQwen2Model *m) {
    LLAISYS_CHECK(m && m->impl, "qwen2: null model");
    return *m->impl;
}

// The scheduler's view of a Qwen2 model: its sequences, KV pool and step
// (weights replaced by the caller are copied in first, as in ModelStep).
class Qwen2Backend : public llaisys::serving::Backend {
public:
    explicit Qwen2Backend(LlaisysQwen2Model *m) : m_(m) {}
    int64_t seqCreate(const int64_t *tokens, size_t n, size_t *reused) override {
        return model(m_).seqCreate(tokens, n, reused);
    }
    void seqFree(int64_t id) override { model(m_).seqFree(id); }
    int64_t numFreeBlocks() override { return int64_t(model(m_).numFreeBlocks()); }
    size_t maxSeqLen() override { return model(m_).config().maxseq; }
    void step(const int64_t *ids, size_t nseq, const int64_t *tokens, const size_t *ntokens, int64_t *next) override {
        syncWeights(*m_);
        model(m_).step(ids, nseq, tokens, ntokens, next);
    }

private:
    LlaisysQwen2Model *m_;
};

} // namespace

// ---- test hooks' plumbing (testing.h)
namespace {
// The AMD runtime of the current HIP device, its stream, and a sync after the launch.
template <typename F> void testHook(F &&f) {
    guardedVoid([&] {
        int dev = 0;
        HIP_CHECK(hipGetDevice(&dev));
        auto &ctx = llaisys::core::context();
        ctx.setDevice(LLAISYS_DEVICE_AMD, dev);
        void *stream = ctx.runtime().stream();
        f(stream, ctx.runtime());
        HIP_CHECK(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    });
}
uint16_t *w16(void *p) { return static_cast<uint16_t *>(p); }
const uint16_t *r16(const void *p) { return static_cast<const uint16_t *>(p); }
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
    // The caller may write through the pointer: count it as a write.
    return guarded(
        [&]() -> void * {
            const auto &x = unbox(t, "tensorGetData");
            x->touch();
            return x->data();
        },
        nullptr);
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

void llaisysLinearPackWeight(llaisysTensor_t packed, llaisysTensor_t weight) {
    guardedVoid([&] {
        const char *w = "linear_pack_weight";
        llaisys::ops::linearPackWeight(unbox(packed, w), unbox(weight, w));
    });
}

void llaisysLinearPacked(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t packed, llaisysTensor_t bias) {
    guardedVoid([&] {
        const char *w = "linear_packed";
        llaisys::ops::linearPacked(unbox(out, w), unbox(in, w), unbox(packed, w), bias ? unbox(bias, w) : nullptr);
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

void llaisysPagedKVAppendGather(llaisysTensor_t k_out, llaisysTensor_t v_out, llaisysTensor_t k_pool,
                                llaisysTensor_t v_pool, llaisysTensor_t k_new, llaisysTensor_t v_new,
                                llaisysTensor_t block_table, llaisysTensor_t ctx_len, llaisysTensor_t cu_seqlens) {
    guardedVoid([&] {
        const char *w = "paged_kv_append_gather";
        llaisys::ops::pagedKVAppendGather(unbox(k_out, w), unbox(v_out, w), unbox(k_pool, w), unbox(v_pool, w),
                                          unbox(k_new, w), unbox(v_new, w), unbox(block_table, w),
                                          unbox(ctx_len, w), unbox(cu_seqlens, w));
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

void llaisysPagedAttentionNoAlloc(llaisysTensor_t out, llaisysTensor_t q, llaisysTensor_t k_pool,
                                  llaisysTensor_t v_pool, llaisysTensor_t block_table, llaisysTensor_t ctx_len,
                                  float scale) {
    guardedVoid([&] {
        const char *w = "paged_attention_no_alloc";
        llaisys::ops::pagedAttentionNoAlloc(unbox(out, w), unbox(q, w), unbox(k_pool, w), unbox(v_pool, w),
                                            unbox(block_table, w), unbox(ctx_len, w), scale);
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

// ---------------- models/qwen2.h
LlaisysQwen2Model *llaisysQwen2ModelCreate(const LlaisysQwen2Meta *meta, llaisysDeviceType_t device, int *device_ids,
                                           int ndevice) {
    return guarded([&] { return createQwen2(meta, device, device_ids, ndevice, 0); },
                   static_cast<LlaisysQwen2Model *>(nullptr));
}

LlaisysQwen2Model *llaisysQwen2ModelCreatePaged(const LlaisysQwen2Meta *meta, llaisysDeviceType_t device,
                                                int *device_ids, int ndevice, size_t num_blocks) {
    return guarded(
        [&] {
            LLAISYS_CHECK(num_blocks > 0, "qwen2: num_blocks must be positive");
            return createQwen2(meta, device, device_ids, ndevice, num_blocks);
        },
        static_cast<LlaisysQwen2Model *>(nullptr));
}

void llaisysQwen2ModelDestroy(LlaisysQwen2Model *m) {
    guardedVoid([&] { delete m; });
}

LlaisysQwen2Weights *llaisysQwen2ModelWeights(LlaisysQwen2Model *m) {
    return guarded([&] { model(m); return &m->w; }, static_cast<LlaisysQwen2Weights *>(nullptr));
}

int64_t llaisysQwen2ModelInfer(LlaisysQwen2Model *m, int64_t *token_ids, size_t ntoken) {
    return guarded([&] { auto &impl = model(m); syncWeights(*m); return impl.infer(token_ids, ntoken); }, int64_t(-1));
}

int64_t llaisysQwen2SeqCreate(LlaisysQwen2Model *m, const int64_t *tokens, size_t ntokens, size_t *reused) {
    return guarded([&] { return model(m).seqCreate(tokens, ntokens, reused); }, int64_t(-1));
}

int64_t llaisysQwen2SeqFork(LlaisysQwen2Model *m, int64_t parent) {
    return guarded([&] { return model(m).seqFork(parent); }, int64_t(-1));
}

int llaisysQwen2SeqFree(LlaisysQwen2Model *m, int64_t seq_id) {
    return guarded([&] { model(m).seqFree(seq_id); return 0; }, -1);
}

int64_t llaisysQwen2SeqLength(LlaisysQwen2Model *m, int64_t seq_id) {
    return guarded([&] { return int64_t(model(m).seqLength(seq_id)); }, int64_t(-1));
}

int64_t llaisysQwen2NumFreeBlocks(LlaisysQwen2Model *m) {
    return guarded([&] { return int64_t(model(m).numFreeBlocks()); }, int64_t(-1));
}

int llaisysQwen2ModelStep(LlaisysQwen2Model *m, const int64_t *seq_ids, size_t nseq, const int64_t *token_ids,
                          const size_t *ntokens, int64_t *next_tokens) {
    return guarded(
        [&] {
            auto &impl = model(m);
            syncWeights(*m);
            impl.step(seq_ids, nseq, token_ids, ntokens, next_tokens);
            return 0;
        },
        -1);
}

int llaisysQwen2ModelDecode(LlaisysQwen2Model *m, const int64_t *seq_ids, size_t nseq, const int64_t *first_tokens,
                            size_t nsteps, int64_t *out_tokens) {
    return guarded(
        [&] {
            auto &impl = model(m);
            syncWeights(*m);
            impl.decode(seq_ids, nseq, first_tokens, nsteps, out_tokens);
            return 0;
        },
        -1);
}

llaisysTensor_t llaisysQwen2ModelLogits(LlaisysQwen2Model *m) {
    return guarded([&] { return new LlaisysTensor{model(m).lastLogits()}; }, static_cast<llaisysTensor_t>(nullptr));
}


// ---------------------------------------------------------------- scheduler

namespace {
llaisys::serving::Scheduler &sched(LlaisysScheduler *s) {
    if (!s || !s->sched) LLAISYS_RAISE("scheduler: null handle");
    return *s->sched;
}
llaisys::serving::SchedulerConfig schedConfig(size_t max_seqs, size_t max_step_tokens, size_t prefill_chunk) {
    llaisys::serving::SchedulerConfig c;
    c.max_seqs = max_seqs;
    c.max_step_tokens = max_step_tokens;
    c.prefill_chunk = prefill_chunk;
    return c;
}
} // namespace

LlaisysScheduler *llaisysQwen2SchedulerCreate(LlaisysQwen2Model *m, size_t max_seqs, size_t max_step_tokens,
                                              size_t prefill_chunk) {
    return guarded(
        [&] {
            model(m);
            auto s = std::make_unique<LlaisysScheduler>();
            s->backend = std::make_unique<Qwen2Backend>(m);
            s->sched = std::make_unique<llaisys::serving::Scheduler>(
                *s->backend, schedConfig(max_seqs, max_step_tokens, prefill_chunk));
            return s.release();
        },
        static_cast<LlaisysScheduler *>(nullptr));
}

LlaisysScheduler *llaisysSimSchedulerCreate(size_t num_blocks, int64_t vocab, size_t max_seq_len, size_t max_seqs,
                                            size_t max_step_tokens, size_t prefill_chunk) {
    return guarded(
        [&] {
            LLAISYS_CHECK(num_blocks <= size_t(1) << 30, "sim scheduler: num_blocks too large");
            auto s = std::make_unique<LlaisysScheduler>();
            s->backend = std::make_unique<llaisys::serving::SimBackend>(int(num_blocks), vocab, max_seq_len);
            s->sched = std::make_unique<llaisys::serving::Scheduler>(
                *s->backend, schedConfig(max_seqs, max_step_tokens, prefill_chunk));
            return s.release();
        },
        static_cast<LlaisysScheduler *>(nullptr));
}

void llaisysSchedulerDestroy(LlaisysScheduler *s) {
    guardedVoid([&] { delete s; });
}

int64_t llaisysSchedulerAdd(LlaisysScheduler *s, const int64_t *prompt, size_t nprompt, size_t max_new_tokens,
                            int64_t eos) {
    return guarded([&] { return sched(s).add(prompt, nprompt, max_new_tokens, eos); }, int64_t(-1));
}

int64_t llaisysSchedulerStep(LlaisysScheduler *s) {
    return guarded([&] { return int64_t(sched(s).step()); }, int64_t(-1));
}

int llaisysSchedulerStatus(LlaisysScheduler *s, int64_t request) {
    return guarded(
        [&] {
            auto &sc = sched(s);
            if (!sc.known(request)) return -1;
            return sc.finished(request) ? int(sc.reason(request)) : int(LLAISYS_REQUEST_ACTIVE);
        },
        -1);
}

int64_t llaisysSchedulerTokens(LlaisysScheduler *s, int64_t request, int64_t *out, size_t capacity) {
    return guarded(
        [&] {
            const auto &t = sched(s).generated(request);
            if (out) std::copy_n(t.begin(), std::min(capacity, t.size()), out);
            return int64_t(t.size());
        },
        int64_t(-1));
}

int llaisysSchedulerRelease(LlaisysScheduler *s, int64_t request) {
    return guarded([&] { sched(s).release(request); return 0; }, -1);
}

int llaisysSchedulerStats(LlaisysScheduler *s, int64_t *out) {
    return guarded(
        [&] {
            LLAISYS_CHECK(out, "scheduler stats: null output");
            const auto &st = sched(s).stats();
            const int64_t v[5] = {st.steps, st.preemptions, st.prefill_tokens, st.decode_tokens, st.finished};
            std::copy_n(v, 5, out);
            return 0;
        },
        -1);
}

// ---------------- testing.h (the decode step's kernels called alone)

void llaisysTestPackWeight(void *packed, const void *w, const void *fold_g, int N, int K) {
    testHook([&](void *s, auto &) { llaisys::kernels::packWeight(w16(packed), r16(w), r16(fold_g), N, K, s); });
}

void llaisysTestPackWeightGateUp(void *packed, const void *w, int di, int K) {
    testHook([&](void *s, auto &) { llaisys::kernels::packWeightGateUp(w16(packed), r16(w), di, K, s); });
}

void llaisysTestPackedXGemm(void *y, const void *x_packed, const void *w_packed, int M, int N, int K, int accumulate,
                            void *y_packed) {
    testHook([&](void *s, auto &) {
        llaisys::kernels::packedXGemm(w16(y), r16(x_packed), r16(w_packed), M, N, K, accumulate != 0, s,
                                      w16(y_packed));
    });
}

void llaisysTestQkvRopeGemm(void *q, void *k_pool, void *v_pool, const void *x_packed, const void *w_packed,
                            const void *bias, const int32_t *table, const int32_t *ctx, int M, int nh, int nkvh,
                            int K, int max_pages, int num_blocks, float eps, float theta) {
    testHook([&](void *s, auto &rt) {
        llaisys::kernels::qkvRopeGemm(w16(q), w16(k_pool), w16(v_pool), r16(x_packed), r16(w_packed), r16(bias),
                                      table, ctx, M, nh, nkvh, K, max_pages, num_blocks, eps, theta, rt.errorWord(),
                                      s);
    });
}

void llaisysTestGateUpSwiglu(void *act, const void *x_packed, const void *w_packed, int M, int di, int K, float eps,
                             int act_packed) {
    testHook([&](void *s, auto &) {
        llaisys::kernels::gateUpSwiglu(w16(act), r16(x_packed), r16(w_packed), M, di, K, eps, s, act_packed != 0);
    });
}

void llaisysTestSwigluInterleave(void *out, const void *w, int di, int K) {
    testHook([&](void *s, auto &) { llaisys::kernels::swigluInterleave(w16(out), r16(w), di, K, s); });
}

void llaisysTestLinearSwiglu(void *act, const void *x, const void *w_interleaved, int M, int di, int K) {
    testHook([&](void *s, auto &) {
        llaisys::kernels::linearSwiglu(act, x, w_interleaved, llaisys::kernels::ElemType::BF16, M, di, K, s);
    });
}

void llaisysTestSplitKPackedGemm(void *y, const void *x_packed, const void *w_packed, int M, int N, int K,
                                 int accumulate, void *y_packed) {
    testHook([&](void *s, auto &rt) {
        auto *part = static_cast<float *>(rt.scratch(llaisys::kernels::splitKPackedWorkspaceBytes(M, N, K)));
        llaisys::kernels::splitKPackedGemm(w16(y), r16(x_packed), r16(w_packed), M, N, K, accumulate != 0, part, s,
                                           w16(y_packed));
    });
}

} // extern "C"
