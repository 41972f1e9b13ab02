#include "ops.hpp"

#include "../common.hpp"
#include "../kernels/launch.hpp"
#include "cpu/cpu_kernels.hpp"

#include <algorithm>

namespace llaisys::ops {

namespace {

namespace K = llaisys::kernels;

std::string shapeStr(const tensor_t &t) {
    std::ostringstream os;
    os << "[";
    for (size_t i = 0; i < t->ndim(); ++i) os << (i ? "," : "") << t->shape()[i];
    os << "]";
    return os.str();
}

void requireContiguous(const tensor_t &t, const char *op, const char *name) {
    LLAISYS_CHECK(t->isContiguous(), op << ": " << name << " must be contiguous");
}

void requireDtype(const tensor_t &t, llaisysDataType_t dt, const char *op, const char *name) {
    LLAISYS_CHECK(t->dtype() == dt, op << ": " << name << " must be " << dtypeName(dt) << ", got "
                                       << dtypeName(t->dtype()));
}

void requireShape(const tensor_t &t, std::initializer_list<size_t> shape, const char *op, const char *name) {
    std::vector<size_t> want(shape);
    LLAISYS_CHECK(t->shape() == want, op << ": " << name << " has shape " << shapeStr(t) << ", expected a different shape");
}

// Every tensor of an op must live on one device: the AMD GPU (HIP kernels) or
// the host (the CPU implementations), as the reference dispatches on the
// tensor's device (src/ops/add/op.cpp:16-33). Returns true for the host.
bool onHost(const char *op, std::initializer_list<const tensor_t *> ts) {
    const tensor_t &first = **ts.begin();
    const auto dev = first->deviceType();
    LLAISYS_CHECK(dev == LLAISYS_DEVICE_AMD || dev == LLAISYS_DEVICE_CPU,
                  op << ": no implementation for device " << deviceName(dev));
    for (auto *t : ts) {
        if (!*t) continue;
        LLAISYS_CHECK((*t)->deviceType() == dev && (*t)->deviceId() == first->deviceId(),
                      op << ": tensors are on different devices (" << deviceName(dev) << " and "
                         << deviceName((*t)->deviceType()) << ")");
    }
    core::context().setDevice(dev, first->deviceId());
    return dev == LLAISYS_DEVICE_CPU;
}

K::ElemType elemType(llaisysDataType_t dt, const char *op) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return K::ElemType::F32;
    case LLAISYS_DTYPE_F16: return K::ElemType::F16;
    case LLAISYS_DTYPE_BF16: return K::ElemType::BF16;
    default: LLAISYS_RAISE(op << ": unsupported dtype " << dtypeName(dt));
    }
}

// Pool: [num_blocks, nkvh, 16, 128] bf16 contiguous.
void checkPool(const tensor_t &kp, const tensor_t &vp, const char *op) {
    for (auto *t : {&kp, &vp}) {
        LLAISYS_CHECK((*t)->ndim() == 4 && (*t)->shape()[2] == size_t(K::kPageTokens) &&
                          (*t)->shape()[3] == size_t(K::kHeadDim),
                      op << ": pool must be [num_blocks, nkvh, 16, 128], got " << shapeStr(*t));
        requireDtype(*t, LLAISYS_DTYPE_BF16, op, "pool");
        requireContiguous(*t, op, "pool");
    }
    LLAISYS_CHECK(kp->shape() == vp->shape(), op << ": K and V pools differ in shape");
    LLAISYS_CHECK(kp->shape()[0] < size_t(1) << 31, op << ": too many blocks");
}

void checkTable(const tensor_t &table, size_t B, const char *op) {
    LLAISYS_CHECK(table->ndim() == 2 && table->shape()[0] == B,
                  op << ": block_table must be [B=" << B << ", max_pages], got " << shapeStr(table));
    requireDtype(table, LLAISYS_DTYPE_I32, op, "block_table");
    requireContiguous(table, op, "block_table");
}

void checkI32Vec(const tensor_t &t, size_t n, const char *op, const char *name) {
    LLAISYS_CHECK(t->ndim() == 1 && t->shape()[0] == n,
                  op << ": " << name << " must be [" << n << "], got " << shapeStr(t));
    requireDtype(t, LLAISYS_DTYPE_I32, op, name);
    requireContiguous(t, op, name);
}

void *streamOf() { return core::context().runtime().stream(); }
namespace C = llaisys::cpu;
int *errWord() { return core::context().runtime().errorWord(); }

} // namespace

// README.md:244-266: attn_val [L, nh, dv], q [L, nh, d], k [S, nkvh, d], v [S, nkvh, dv].
void selfAttention(const tensor_t &out, const tensor_t &q, const tensor_t &k, const tensor_t &v, float scale) {
    const char *op = "self_attention";
    LLAISYS_CHECK(out && q && k && v, op << ": null tensor");
    LLAISYS_CHECK(q->ndim() == 3 && k->ndim() == 3 && v->ndim() == 3 && out->ndim() == 3,
                  op << ": q, k, v and attn_val must be 3-D");
    const size_t L = q->shape()[0], nh = q->shape()[1], d = q->shape()[2];
    const size_t S = k->shape()[0], nkvh = k->shape()[1], dv = v->shape()[2];
    LLAISYS_CHECK(k->shape()[2] == d, op << ": k head dim " << k->shape()[2] << " != q head dim " << d);
    LLAISYS_CHECK(v->shape()[0] == S && v->shape()[1] == nkvh, op << ": v shape " << shapeStr(v) << " does not match k " << shapeStr(k));
    requireShape(out, {L, nh, dv}, op, "attn_val");
    LLAISYS_CHECK(nkvh > 0 && nh % nkvh == 0, op << ": nh=" << nh << " is not a multiple of nkvh=" << nkvh);
    LLAISYS_CHECK(S >= L, op << ": total_len " << S << " < seqlen " << L);
    LLAISYS_CHECK(q->dtype() == k->dtype() && q->dtype() == v->dtype() && q->dtype() == out->dtype(),
                  op << ": q, k, v, attn_val must share one dtype");
    for (auto *t : {&out, &q, &k, &v}) requireContiguous(*t, op, "every tensor");
    const bool host = onHost(op, {&out, &q, &k, &v});
    if (L == 0) return;
    LLAISYS_CHECK(S > 0, op << ": empty key set");
    if (host)
        return C::selfAttention(out->data(), q->data(), k->data(), v->data(), elemType(q->dtype(), op), int(L),
                                int(S), int(nh), int(nkvh), int(d), int(dv), scale);
    void *ws = core::context().runtime().scratch(K::selfAttentionWorkspaceBytes(int(L), int(S), int(nh), int(dv)));
    K::selfAttention(out->data(), q->data(), k->data(), v->data(), elemType(q->dtype(), op), int(L), int(S),
                     int(nh), int(nkvh), int(d), int(dv), scale, streamOf(), ws);
}

void pagedKVAppend(const tensor_t &k_pool, const tensor_t &v_pool, const tensor_t &k_new, const tensor_t &v_new,
                   const tensor_t &block_table, const tensor_t &ctx_len, const tensor_t &cu_new) {
    const char *op = "paged_kv_append";
    LLAISYS_CHECK(k_pool && v_pool && k_new && v_new && block_table && ctx_len, op << ": null tensor");
    checkPool(k_pool, v_pool, op);
    const size_t nkvh = k_pool->shape()[1];
    LLAISYS_CHECK(k_new->ndim() == 3 && k_new->shape()[1] == nkvh && k_new->shape()[2] == size_t(K::kHeadDim),
                  op << ": k_new must be [T, nkvh=" << nkvh << ", 128], got " << shapeStr(k_new));
    LLAISYS_CHECK(v_new->shape() == k_new->shape(), op << ": v_new shape differs from k_new");
    requireDtype(k_new, LLAISYS_DTYPE_BF16, op, "k_new");
    requireDtype(v_new, LLAISYS_DTYPE_BF16, op, "v_new");
    requireContiguous(k_new, op, "k_new");
    requireContiguous(v_new, op, "v_new");
    const size_t T = k_new->shape()[0];
    const size_t B = ctx_len->ndim() == 1 ? ctx_len->shape()[0] : 0;
    checkI32Vec(ctx_len, B, op, "ctx_len");
    checkTable(block_table, B, op);
    if (cu_new) {
        checkI32Vec(cu_new, B + 1, op, "cu_new");
    } else {
        LLAISYS_CHECK(T == B, op << ": without cu_new, k_new must hold one token per sequence (T=" << T << ", B=" << B << ")");
    }
    const bool host = onHost(op, {&k_pool, &v_pool, &k_new, &v_new, &block_table, &ctx_len, &cu_new});
    if (T == 0) return;
    LLAISYS_CHECK(B > 0, op << ": tokens given for zero sequences");
    auto *kp = reinterpret_cast<uint16_t *>(k_pool->data());
    auto *vp = reinterpret_cast<uint16_t *>(v_pool->data());
    const auto *kn = reinterpret_cast<const uint16_t *>(k_new->data());
    const auto *vn = reinterpret_cast<const uint16_t *>(v_new->data());
    const auto *tab = reinterpret_cast<const int32_t *>(block_table->data());
    const auto *ctx = reinterpret_cast<const int32_t *>(ctx_len->data());
    const auto *cu = cu_new ? reinterpret_cast<const int32_t *>(cu_new->data()) : nullptr;
    const int maxp = int(block_table->shape()[1]), nb = int(k_pool->shape()[0]);
    if (host)
        C::pagedAppend(kp, vp, kn, vn, tab, ctx, cu, int(T), int(B), int(nkvh), maxp, nb, errWord());
    else
        K::pagedAppend(kp, vp, kn, vn, tab, ctx, cu, int(T), int(B), int(nkvh), maxp, nb, errWord(), streamOf());
}

void pagedKVGather(const tensor_t &k_out, const tensor_t &v_out, const tensor_t &k_pool, const tensor_t &v_pool,
                   const tensor_t &block_table, const tensor_t &cu_seqlens) {
    const char *op = "paged_kv_gather";
    LLAISYS_CHECK(k_out && v_out && k_pool && v_pool && block_table && cu_seqlens, op << ": null tensor");
    checkPool(k_pool, v_pool, op);
    const size_t nkvh = k_pool->shape()[1];
    LLAISYS_CHECK(k_out->ndim() == 3 && k_out->shape()[1] == nkvh && k_out->shape()[2] == size_t(K::kHeadDim),
                  op << ": k_out must be [T, nkvh=" << nkvh << ", 128], got " << shapeStr(k_out));
    LLAISYS_CHECK(v_out->shape() == k_out->shape(), op << ": v_out shape differs from k_out");
    requireDtype(k_out, LLAISYS_DTYPE_BF16, op, "k_out");
    requireDtype(v_out, LLAISYS_DTYPE_BF16, op, "v_out");
    requireContiguous(k_out, op, "k_out");
    requireContiguous(v_out, op, "v_out");
    LLAISYS_CHECK(cu_seqlens->ndim() == 1 && cu_seqlens->shape()[0] >= 1, op << ": cu_seqlens must be [B+1]");
    const size_t B = cu_seqlens->shape()[0] - 1;
    checkI32Vec(cu_seqlens, B + 1, op, "cu_seqlens");
    checkTable(block_table, B, op);
    const bool host = onHost(op, {&k_out, &v_out, &k_pool, &v_pool, &block_table, &cu_seqlens});
    auto *ko = reinterpret_cast<uint16_t *>(k_out->data());
    auto *vo = reinterpret_cast<uint16_t *>(v_out->data());
    const auto *kp = reinterpret_cast<const uint16_t *>(k_pool->data());
    const auto *vp = reinterpret_cast<const uint16_t *>(v_pool->data());
    const auto *tab = reinterpret_cast<const int32_t *>(block_table->data());
    const auto *cu = reinterpret_cast<const int32_t *>(cu_seqlens->data());
    const int T = int(k_out->shape()[0]), maxp = int(block_table->shape()[1]), nb = int(k_pool->shape()[0]);
    if (host)
        C::pagedGather(ko, vo, kp, vp, tab, cu, T, int(B), int(nkvh), maxp, nb, errWord());
    else
        K::pagedGather(ko, vo, kp, vp, tab, cu, T, int(B), int(nkvh), maxp, nb, errWord(), streamOf());
}

void pagedKVAppendGather(const tensor_t &k_out, const tensor_t &v_out, const tensor_t &k_pool, const tensor_t &v_pool,
                         const tensor_t &k_new, const tensor_t &v_new, const tensor_t &block_table,
                         const tensor_t &ctx_len, const tensor_t &cu_seqlens) {
    const char *op = "paged_kv_append_gather";
    LLAISYS_CHECK(k_out && v_out && k_pool && v_pool && k_new && v_new && block_table && ctx_len && cu_seqlens,
                  op << ": null tensor");
    checkPool(k_pool, v_pool, op);
    const size_t nkvh = k_pool->shape()[1];
    for (const auto *t : {&k_out, &k_new}) {
        const char *name = t == &k_out ? "k_out" : "k_new";
        LLAISYS_CHECK((*t)->ndim() == 3 && (*t)->shape()[1] == nkvh && (*t)->shape()[2] == size_t(K::kHeadDim),
                      op << ": " << name << " must be [rows, nkvh=" << nkvh << ", 128], got " << shapeStr(*t));
    }
    LLAISYS_CHECK(v_out->shape() == k_out->shape(), op << ": v_out shape differs from k_out");
    LLAISYS_CHECK(v_new->shape() == k_new->shape(), op << ": v_new shape differs from k_new");
    for (const auto *t : {&k_out, &v_out, &k_new, &v_new}) {
        requireDtype(*t, LLAISYS_DTYPE_BF16, op, "k_out, v_out, k_new and v_new");
        requireContiguous(*t, op, "k_out, v_out, k_new and v_new");
    }
    LLAISYS_CHECK(cu_seqlens->ndim() == 1 && cu_seqlens->shape()[0] >= 1, op << ": cu_seqlens must be [B+1]");
    const size_t B = cu_seqlens->shape()[0] - 1;
    checkI32Vec(cu_seqlens, B + 1, op, "cu_seqlens");
    checkI32Vec(ctx_len, B, op, "ctx_len");
    checkTable(block_table, B, op);
    LLAISYS_CHECK(k_new->shape()[0] == B, op << ": k_new must hold one token per sequence (rows=" << k_new->shape()[0]
                                             << ", B=" << B << ")");
    const bool host = onHost(op, {&k_out, &v_out, &k_pool, &v_pool, &k_new, &v_new, &block_table, &ctx_len, &cu_seqlens});
    auto *ko = reinterpret_cast<uint16_t *>(k_out->data());
    auto *vo = reinterpret_cast<uint16_t *>(v_out->data());
    auto *kp = reinterpret_cast<uint16_t *>(k_pool->data());
    auto *vp = reinterpret_cast<uint16_t *>(v_pool->data());
    const auto *kn = reinterpret_cast<const uint16_t *>(k_new->data());
    const auto *vn = reinterpret_cast<const uint16_t *>(v_new->data());
    const auto *tab = reinterpret_cast<const int32_t *>(block_table->data());
    const auto *ctx = reinterpret_cast<const int32_t *>(ctx_len->data());
    const auto *cu = reinterpret_cast<const int32_t *>(cu_seqlens->data());
    const int T = int(k_out->shape()[0]), maxp = int(block_table->shape()[1]), nb = int(k_pool->shape()[0]);
    if (host)
        C::pagedAppendGather(ko, vo, kp, vp, kn, vn, tab, ctx, cu, T, int(B), int(nkvh), maxp, nb, errWord());
    else
        K::pagedAppendGather(ko, vo, kp, vp, kn, vn, tab, ctx, cu, T, int(B), int(nkvh), maxp, nb, errWord(),
                             streamOf());
}

void pagedKVCopyBlocks(const tensor_t &k_pool, const tensor_t &v_pool, const tensor_t &pairs) {
    const char *op = "paged_kv_copy_blocks";
    LLAISYS_CHECK(k_pool && v_pool && pairs, op << ": null tensor");
    checkPool(k_pool, v_pool, op);
    LLAISYS_CHECK(pairs->ndim() == 2 && pairs->shape()[1] == 2, op << ": pairs must be [P, 2], got " << shapeStr(pairs));
    requireDtype(pairs, LLAISYS_DTYPE_I32, op, "pairs");
    requireContiguous(pairs, op, "pairs");
    const bool host = onHost(op, {&k_pool, &v_pool, &pairs});
    auto *kp = reinterpret_cast<uint16_t *>(k_pool->data());
    auto *vp = reinterpret_cast<uint16_t *>(v_pool->data());
    const auto *pr = reinterpret_cast<const int32_t *>(pairs->data());
    const int P = int(pairs->shape()[0]), nkvh = int(k_pool->shape()[1]), nb = int(k_pool->shape()[0]);
    if (host)
        C::pagedCopyBlocks(kp, vp, pr, P, nkvh, nb, errWord());
    else
        K::pagedCopyBlocks(kp, vp, pr, P, nkvh, nb, errWord(), streamOf());
}

namespace {

// Shapes, dtypes and layouts of a paged attention call (decode when cu_q is
// null); returns {T, nh, nkvh, B}.
struct AttnDims {
    size_t T, nh, nkvh, B;
};
AttnDims checkAttention(const char *op, const tensor_t &out, const tensor_t &q, const tensor_t &k_pool,
                        const tensor_t &v_pool, const tensor_t &block_table, const tensor_t &ctx_len,
                        const tensor_t &cu_q) {
    LLAISYS_CHECK(out && q && k_pool && v_pool && block_table && ctx_len, op << ": null tensor");
    checkPool(k_pool, v_pool, op);
    const size_t nkvh = k_pool->shape()[1];
    LLAISYS_CHECK(q->ndim() == 3 && q->shape()[2] == size_t(K::kHeadDim),
                  op << ": q must be [T, nh, 128], got " << shapeStr(q));
    const size_t T = q->shape()[0], nh = q->shape()[1];
    LLAISYS_CHECK(nkvh > 0 && nh % nkvh == 0 && nh / nkvh <= 16,
                  op << ": need nh % nkvh == 0 and nh / nkvh <= 16 (nh=" << nh << ", nkvh=" << nkvh << ")");
    requireDtype(q, LLAISYS_DTYPE_BF16, op, "q");
    requireContiguous(q, op, "q");
    requireShape(out, {T, nh, size_t(K::kHeadDim)}, op, "out");
    LLAISYS_CHECK(out->dtype() == LLAISYS_DTYPE_BF16 || out->dtype() == LLAISYS_DTYPE_F32,
                  op << ": out must be bf16 or f32");
    requireContiguous(out, op, "out");
    LLAISYS_CHECK(ctx_len->ndim() == 1, op << ": ctx_len must be [B]");
    const size_t B = ctx_len->shape()[0];
    checkI32Vec(ctx_len, B, op, "ctx_len");
    checkTable(block_table, B, op);
    if (cu_q) {
        checkI32Vec(cu_q, B + 1, op, "cu_q");
    } else {
        LLAISYS_CHECK(T == B, op << ": q must hold one query per sequence (T=" << T << ", B=" << B << ")");
    }
    return {T, nh, nkvh, B};
}

} // namespace

void pagedAttention(const tensor_t &out, const tensor_t &q, const tensor_t &k_pool, const tensor_t &v_pool,
                    const tensor_t &block_table, const tensor_t &ctx_len, const tensor_t &cu_q, float scale) {
    const char *op = cu_q ? "paged_attention_varlen" : "paged_attention";
    const auto [T, nh, nkvh, B] = checkAttention(op, out, q, k_pool, v_pool, block_table, ctx_len, cu_q);
    const bool host = onHost(op, {&out, &q, &k_pool, &v_pool, &block_table, &ctx_len, &cu_q});
    if (T == 0 || B == 0) return;
    const int max_pages = int(block_table->shape()[1]);
    LLAISYS_CHECK(max_pages > 0, op << ": block_table has no pages");
    if (host)
        return C::pagedAttention(out->data(), out->dtype() == LLAISYS_DTYPE_F32,
                                 reinterpret_cast<const uint16_t *>(q->data()),
                                 reinterpret_cast<const uint16_t *>(k_pool->data()),
                                 reinterpret_cast<const uint16_t *>(v_pool->data()),
                                 reinterpret_cast<const int32_t *>(block_table->data()),
                                 reinterpret_cast<const int32_t *>(ctx_len->data()),
                                 cu_q ? reinterpret_cast<const int32_t *>(cu_q->data()) : nullptr, int(B), int(T),
                                 int(nh), int(nkvh), max_pages, int(k_pool->shape()[0]), scale, errWord());
    auto &rt = core::context().runtime();
    const int G = int(nh / nkvh);
    const bool f32 = out->dtype() == LLAISYS_DTYPE_F32;
    const auto *qp = reinterpret_cast<const uint16_t *>(q->data());
    const auto *kp = reinterpret_cast<const uint16_t *>(k_pool->data());
    const auto *vp = reinterpret_cast<const uint16_t *>(v_pool->data());
    const auto *tab = reinterpret_cast<const int32_t *>(block_table->data());
    const auto *ctx = reinterpret_cast<const int32_t *>(ctx_len->data());
    const int nb = int(k_pool->shape()[0]);
    if (!cu_q) {
        // Decode: sequences are independent, so large batches run in chunks
        // whose length prefix fits the kernel's LDS.
        for (size_t b0 = 0; b0 < B; b0 += K::kDecodeMaxBatch) {
            const int Bc = int(std::min<size_t>(K::kDecodeMaxBatch, B - b0));
            auto plan = K::planDecode(Bc, int(nkvh), G, max_pages);
            float *records = static_cast<float *>(rt.scratch(plan.record_bytes));
            const size_t esz = f32 ? 4 : 2;
            K::pagedDecode(static_cast<std::byte *>(out->data()) + b0 * nh * K::kHeadDim * esz, f32,
                           qp + b0 * nh * K::kHeadDim, kp, vp, tab + b0 * size_t(max_pages), ctx + b0, nullptr, Bc,
                           Bc, int(nh), int(nkvh), max_pages, nb, scale, plan, records, rt.errorWord(),
                           plan.slot_headers ? rt.decodeSlotHeaders(plan.slot_headers) : nullptr,
                           plan.slot_headers ? rt.decodeSlotRecords(plan.slot_record_bytes) : nullptr, rt.stream());
        }
        return;
    }
    // Varlen: single-query sequences through the decode kernel, the rest
    // through the prefill kernel; both read the same cu_q and skip the other's.
    LLAISYS_CHECK(B <= size_t(K::kDecodeMaxBatch),
                  op << ": at most " << K::kDecodeMaxBatch << " sequences per varlen call");
    const auto *cu = reinterpret_cast<const int32_t *>(cu_q->data());
    auto dplan = K::planDecode(int(B), int(nkvh), G, max_pages);
    auto pplan = K::planPrefill(int(B), int(T), int(nkvh), G, max_pages);
    float *records = static_cast<float *>(rt.scratch(std::max(dplan.record_bytes, pplan.partial_bytes)));
    int *queue = rt.queueCounters();
    // The persistent prefill kernel takes the single-query sequences too
    // when it runs (their HBM-bound work then overlaps the prefill's MFMA
    // work); otherwise the decode kernel does.
    if (!K::prefillTakesDecode(int(B), int(T), pplan, queue)) {
        int *slot_hdr = dplan.slot_headers ? rt.decodeSlotHeaders(dplan.slot_headers) : nullptr;
        void *slot_rec = dplan.slot_headers ? rt.decodeSlotRecords(dplan.slot_record_bytes) : nullptr;
        K::pagedDecode(out->data(), f32, qp, kp, vp, tab, ctx, cu, int(B), int(T), int(nh), int(nkvh), max_pages, nb,
                       scale, dplan, records, rt.errorWord(), slot_hdr, slot_rec, rt.stream());
    }
    K::pagedPrefill(out->data(), f32, qp, kp, vp, tab, ctx, cu, int(B), int(T), int(nh), int(nkvh), max_pages, nb,
                    scale, pplan, records, rt.errorWord(), queue, rt.stream());
}

// No counterpart in the reference: the decode above for callers that cannot
// allocate device memory (graph capture, fixed-memory serving loops).
void pagedAttentionNoAlloc(const tensor_t &out, const tensor_t &q, const tensor_t &k_pool, const tensor_t &v_pool,
                           const tensor_t &block_table, const tensor_t &ctx_len, float scale) {
    const char *op = "paged_attention_no_alloc";
    const auto [T, nh, nkvh, B] = checkAttention(op, out, q, k_pool, v_pool, block_table, ctx_len, nullptr);
    LLAISYS_CHECK(!onHost(op, {&out, &q, &k_pool, &v_pool, &block_table, &ctx_len}),
                  op << ": AMD device tensors only (host tensors use llaisysPagedAttention)");
    if (T == 0 || B == 0) return;
    const int max_pages = int(block_table->shape()[1]);
    LLAISYS_CHECK(max_pages > 0, op << ": block_table has no pages");
    K::pagedDecodeNoAlloc(out->data(), out->dtype() == LLAISYS_DTYPE_F32, reinterpret_cast<const uint16_t *>(q->data()),
                          reinterpret_cast<const uint16_t *>(k_pool->data()),
                          reinterpret_cast<const uint16_t *>(v_pool->data()),
                          reinterpret_cast<const int32_t *>(block_table->data()),
                          reinterpret_cast<const int32_t *>(ctx_len->data()), int(B), int(nh), int(nkvh), max_pages,
                          int(k_pool->shape()[0]), scale, errWord(), streamOf());
}

} // namespace llaisys::ops
