// The reference's model ops on the AMD device and the host (README.md:145-292), as used
// by the Qwen2 decode step. Shape/dtype contracts follow the reference
// README and test/ops/*.py; all tensors contiguous unless stated.
#include "ops.hpp"

#include "../common.hpp"
#include "../kernels/launch.hpp"
#include "cpu/cpu_kernels.hpp"

namespace llaisys::ops {

namespace {

namespace K = llaisys::kernels;
namespace C = llaisys::cpu;

std::string shapeOf(const tensor_t &t) {
    std::ostringstream os;
    os << "[";
    for (size_t i = 0; i < t->ndim(); ++i) os << (i ? "," : "") << t->shape()[i];
    os << "]";
    return os.str();
}

K::ElemType floatType(const tensor_t &t, const char *op) {
    switch (t->dtype()) {
    case LLAISYS_DTYPE_F32: return K::ElemType::F32;
    case LLAISYS_DTYPE_F16: return K::ElemType::F16;
    case LLAISYS_DTYPE_BF16: return K::ElemType::BF16;
    default: LLAISYS_RAISE(op << ": dtype " << dtypeName(t->dtype()) << " not supported (f32, f16, bf16)");
    }
}

// All tensors on one device, AMD (HIP kernels) or the host (CPU
// implementations), dispatched as src/ops/add/op.cpp:16-33 does. Returns true
// for the host.
bool onHost(const char *op, std::initializer_list<const tensor_t *> ts, bool contiguous = true) {
    const tensor_t *first = nullptr;
    for (auto *t : ts) {
        if (!*t) continue;
        if (!first) {
            first = t;
            const auto dev = (*t)->deviceType();
            LLAISYS_CHECK(dev == LLAISYS_DEVICE_AMD || dev == LLAISYS_DEVICE_CPU,
                          op << ": no implementation for device " << deviceName(dev));
        }
        LLAISYS_CHECK((*t)->deviceType() == (*first)->deviceType() && (*t)->deviceId() == (*first)->deviceId(),
                      op << ": tensors are on different devices");
        if (contiguous) LLAISYS_CHECK((*t)->isContiguous(), op << ": tensors must be contiguous");
    }
    core::context().setDevice((*first)->deviceType(), (*first)->deviceId());
    return (*first)->deviceType() == LLAISYS_DEVICE_CPU;
}

void sameDtype(const char *op, std::initializer_list<const tensor_t *> ts) {
    const auto dt = (**ts.begin())->dtype();
    for (auto *t : ts)
        if (*t) LLAISYS_CHECK((*t)->dtype() == dt, op << ": tensors must share one dtype");
}

void *stream() { return core::context().runtime().stream(); }

} // namespace

void add(const tensor_t &c, const tensor_t &a, const tensor_t &b) {
    const char *op = "add";
    LLAISYS_CHECK(c && a && b, op << ": null tensor");
    LLAISYS_CHECK(c->shape() == a->shape() && c->shape() == b->shape(), op << ": shapes differ");
    sameDtype(op, {&c, &a, &b});
    if (onHost(op, {&c, &a, &b})) return C::add(c->data(), a->data(), b->data(), floatType(c, op), c->numel());
    K::add(c->data(), a->data(), b->data(), floatType(c, op), c->numel(), stream());
}

void argmax(const tensor_t &max_idx, const tensor_t &max_val, const tensor_t &vals) {
    const char *op = "argmax";
    LLAISYS_CHECK(max_idx && vals, op << ": null tensor");
    LLAISYS_CHECK(vals->ndim() >= 1 && vals->shape().back() > 0, op << ": vals must be non-empty");
    const size_t n = vals->shape().back();
    const size_t rows = vals->numel() / n;
    LLAISYS_CHECK(max_idx->numel() == rows && max_idx->dtype() == LLAISYS_DTYPE_I64,
                  op << ": max_idx must be I64 with one element per row (" << rows << ")");
    if (max_val) {
        LLAISYS_CHECK(max_val->numel() == rows && max_val->dtype() == vals->dtype(),
                      op << ": max_val must match vals' dtype with one element per row");
    }
    if (onHost(op, {&max_idx, &max_val, &vals}))
        return C::argmax(reinterpret_cast<int64_t *>(max_idx->data()), max_val ? max_val->data() : nullptr,
                         vals->data(), floatType(vals, op), rows, int64_t(n));
    void *ws = core::context().runtime().scratch(K::argmaxWorkspaceBytes(rows, int64_t(n)));
    K::argmax(reinterpret_cast<int64_t *>(max_idx->data()), max_val ? max_val->data() : nullptr, vals->data(),
              floatType(vals, op), rows, int64_t(n), ws, stream());
}

void embedding(const tensor_t &out, const tensor_t &index, const tensor_t &weight) {
    const char *op = "embedding";
    LLAISYS_CHECK(out && index && weight, op << ": null tensor");
    LLAISYS_CHECK(index->ndim() == 1 && index->dtype() == LLAISYS_DTYPE_I64, op << ": index must be 1-D I64");
    LLAISYS_CHECK(weight->ndim() == 2, op << ": weight must be 2-D");
    LLAISYS_CHECK(out->ndim() == 2 && out->shape()[0] == index->shape()[0] && out->shape()[1] == weight->shape()[1],
                  op << ": out must be [" << index->shape()[0] << ", " << weight->shape()[1] << "], got " << shapeOf(out));
    sameDtype(op, {&out, &weight});
    if (onHost(op, {&out, &index, &weight}))
        return C::embedding(out->data(), reinterpret_cast<const int64_t *>(index->data()), weight->data(),
                            floatType(out, op), index->shape()[0], int64_t(weight->shape()[0]),
                            int(weight->shape()[1]), core::context().runtime().errorWord());
    K::embedding(out->data(), reinterpret_cast<const int64_t *>(index->data()), weight->data(), floatType(out, op),
                 index->shape()[0], int64_t(weight->shape()[0]), int(weight->shape()[1]),
                 core::context().runtime().errorWord(), stream());
}

void linear(const tensor_t &out, const tensor_t &in, const tensor_t &weight, const tensor_t &bias) {
    const char *op = "linear";
    LLAISYS_CHECK(out && in && weight, op << ": null tensor");
    LLAISYS_CHECK(in->ndim() == 2 && weight->ndim() == 2 && out->ndim() == 2, op << ": in, weight, out must be 2-D");
    const size_t M = in->shape()[0], Kd = in->shape()[1], N = weight->shape()[0];
    LLAISYS_CHECK(weight->shape()[1] == Kd, op << ": weight " << shapeOf(weight) << " does not match in " << shapeOf(in));
    LLAISYS_CHECK(out->shape()[0] == M && out->shape()[1] == N, op << ": out must be [" << M << ", " << N << "]");
    if (bias) LLAISYS_CHECK(bias->ndim() == 1 && bias->shape()[0] == N, op << ": bias must be [" << N << "]");
    sameDtype(op, {&out, &in, &weight, &bias});
    if (onHost(op, {&out, &in, &weight, &bias}))
        return C::linear(out->data(), in->data(), weight->data(), bias ? bias->data() : nullptr, floatType(out, op),
                         int(M), int(N), int(Kd));
    const auto t = floatType(out, op);
    void *ws = core::context().runtime().scratch(K::linearWorkspaceBytes(t, int(M), int(N), int(Kd)));
    K::linear(out->data(), in->data(), weight->data(), bias ? bias->data() : nullptr, t, int(M), int(N), int(Kd),
              stream(), false, ws);
}

void linearPackWeight(const tensor_t &packed, const tensor_t &weight) {
    const char *op = "linear_pack_weight";
    LLAISYS_CHECK(packed && weight, op << ": null tensor");
    LLAISYS_CHECK(weight->ndim() == 2 && packed->shape() == weight->shape(),
                  op << ": packed must have the weight's shape [N, K], got " << shapeOf(packed) << " for "
                     << shapeOf(weight));
    LLAISYS_CHECK(weight->dtype() == LLAISYS_DTYPE_BF16 && packed->dtype() == LLAISYS_DTYPE_BF16, op << ": bf16 only");
    const int N = int(weight->shape()[0]), Kd = int(weight->shape()[1]);
    LLAISYS_CHECK(N % 16 == 0 && Kd % 32 == 0, op << ": needs N % 16 == 0 and K % 32 == 0");
    LLAISYS_CHECK(!onHost(op, {&packed, &weight}), op << ": AMD device tensors only");
    LLAISYS_CHECK(packed->isContiguous() && weight->isContiguous(), op << ": contiguous tensors only");
    {
        // The kernel reads W while it writes the tiled copy: overlapping
        // storage (e.g. packing in place) would corrupt both.
        const auto *p = static_cast<const std::byte *>(packed->data());
        const auto *w = static_cast<const std::byte *>(weight->data());
        const size_t bytes = size_t(N) * size_t(Kd) * 2;
        LLAISYS_CHECK(p + bytes <= w || w + bytes <= p, op << ": packed and weight must not overlap");
    }
    K::packWeight(reinterpret_cast<uint16_t *>(packed->data()), reinterpret_cast<const uint16_t *>(weight->data()),
                  nullptr, N, Kd, stream());
}

void linearPacked(const tensor_t &out, const tensor_t &in, const tensor_t &packed, const tensor_t &bias) {
    const char *op = "linear_packed";
    LLAISYS_CHECK(out && in && packed, op << ": null tensor");
    LLAISYS_CHECK(in->ndim() == 2 && packed->ndim() == 2 && out->ndim() == 2, op << ": in, packed, out must be 2-D");
    const int M = int(in->shape()[0]), Kd = int(in->shape()[1]), N = int(packed->shape()[0]);
    LLAISYS_CHECK(int(packed->shape()[1]) == Kd, op << ": packed " << shapeOf(packed) << " does not match in " << shapeOf(in));
    LLAISYS_CHECK(int(out->shape()[0]) == M && int(out->shape()[1]) == N, op << ": out must be [" << M << ", " << N << "]");
    if (bias) LLAISYS_CHECK(bias->ndim() == 1 && int(bias->shape()[0]) == N, op << ": bias must be [" << N << "]");
    for (auto *t : {&out, &in, &packed, &bias})
        if (*t) LLAISYS_CHECK((*t)->dtype() == LLAISYS_DTYPE_BF16, op << ": bf16 only");
    const bool split = !K::decodeGemmSupported(M, N, Kd) && K::splitKGemmSupported(M, N, Kd);
    LLAISYS_CHECK(K::decodeGemmSupported(M, N, Kd) || split,
                  op << ": needs 1 <= M <= " << K::kDecodeGemmMaxM << " and either K == " << K::kDecodeGemmK
                     << ", N % 16 == 0, or " << K::kDecodeGemmK << " < K <= " << K::kSplitKMaxK
                     << ", K % 32 == 0, N % 128 == 0 (M=" << M << ", N=" << N << ", K=" << Kd
                     << "); use llaisysLinear");
    LLAISYS_CHECK(!onHost(op, {&out, &in, &packed, &bias}), op << ": AMD device tensors only");
    auto *y = reinterpret_cast<uint16_t *>(out->data());
    const auto *x = reinterpret_cast<const uint16_t *>(in->data());
    const auto *w = reinterpret_cast<const uint16_t *>(packed->data());
    if (bias) K::fillRows(y, bias->data(), K::ElemType::BF16, size_t(M), size_t(N), stream());
    if (split) {
        auto *part = static_cast<float *>(core::context().runtime().scratch(K::splitKWorkspaceBytes(M, N, Kd)));
        K::splitKGemm(y, x, w, M, N, Kd, bias != nullptr, part, stream());
    } else {
        K::decodeGemm(y, x, w, M, N, Kd, bias != nullptr, stream());
    }
}

void rearrange(const tensor_t &out, const tensor_t &in) {
    const char *op = "rearrange";
    LLAISYS_CHECK(out && in, op << ": null tensor");
    LLAISYS_CHECK(out->shape() == in->shape(), op << ": shapes differ");
    sameDtype(op, {&out, &in});
    const bool host = onHost(op, {&out, &in}, false);
    std::vector<int64_t> shape(out->ndim()), os(out->ndim()), is(out->ndim());
    for (size_t k = 0; k < out->ndim(); ++k) {
        shape[k] = int64_t(out->shape()[k]);
        os[k] = out->strides()[k];
        is[k] = in->strides()[k];
    }
    if (host)
        return C::rearrange(out->data(), in->data(), out->elementSize(), int(out->ndim()), shape.data(), os.data(),
                            is.data());
    K::rearrange(out->data(), in->data(), out->elementSize(), int(out->ndim()), shape.data(), os.data(), is.data(),
                 stream());
}

void rmsNorm(const tensor_t &out, const tensor_t &in, const tensor_t &weight, float eps) {
    const char *op = "rms_norm";
    LLAISYS_CHECK(out && in && weight, op << ": null tensor");
    LLAISYS_CHECK(in->ndim() >= 1 && out->shape() == in->shape(), op << ": out and in must share a shape");
    const size_t d = in->shape().back();
    LLAISYS_CHECK(weight->ndim() == 1 && weight->shape()[0] == d, op << ": weight must be [" << d << "]");
    sameDtype(op, {&out, &in, &weight});
    if (onHost(op, {&out, &in, &weight}))
        return C::rmsNorm(out->data(), in->data(), weight->data(), floatType(out, op), in->numel() / d, int(d), eps);
    K::rmsNorm(out->data(), in->data(), weight->data(), floatType(out, op), in->numel() / d, int(d), eps, stream());
}

void rope(const tensor_t &out, const tensor_t &in, const tensor_t &pos_ids, float theta) {
    const char *op = "rope";
    LLAISYS_CHECK(out && in && pos_ids, op << ": null tensor");
    LLAISYS_CHECK(in->ndim() == 3 && out->shape() == in->shape(), op << ": in/out must be [seqlen, nhead, d]");
    LLAISYS_CHECK(in->shape()[2] % 2 == 0, op << ": head dim must be even");
    LLAISYS_CHECK(pos_ids->ndim() == 1 && pos_ids->shape()[0] == in->shape()[0] && pos_ids->dtype() == LLAISYS_DTYPE_I64,
                  op << ": pos_ids must be I64 [" << in->shape()[0] << "]");
    sameDtype(op, {&out, &in});
    if (onHost(op, {&out, &in, &pos_ids}))
        return C::rope(out->data(), in->data(), reinterpret_cast<const int64_t *>(pos_ids->data()), floatType(out, op),
                       in->shape()[0], int(in->shape()[1]), int(in->shape()[2]), theta);
    K::rope(out->data(), in->data(), reinterpret_cast<const int64_t *>(pos_ids->data()), floatType(out, op),
            in->shape()[0], int(in->shape()[1]), int(in->shape()[2]), theta, stream());
}

void swiglu(const tensor_t &out, const tensor_t &gate, const tensor_t &up) {
    const char *op = "swiglu";
    LLAISYS_CHECK(out && gate && up, op << ": null tensor");
    LLAISYS_CHECK(out->shape() == gate->shape() && out->shape() == up->shape(), op << ": shapes differ");
    sameDtype(op, {&out, &gate, &up});
    if (onHost(op, {&out, &gate, &up}))
        return C::swiglu(out->data(), gate->data(), up->data(), floatType(out, op), out->numel());
    K::swiglu(out->data(), gate->data(), up->data(), floatType(out, op), out->numel(), stream());
}

} // namespace llaisys::ops
