#include "tensor.hpp"

#include "../common.hpp"

#include <iostream>
#include <numeric>

namespace llaisys {

namespace {
std::vector<ptrdiff_t> rowMajorStrides(const std::vector<size_t> &shape) {
    std::vector<ptrdiff_t> st(shape.size());
    ptrdiff_t s = 1;
    for (size_t i = shape.size(); i-- > 0;) {
        st[i] = s;
        s *= ptrdiff_t(shape[i]);
    }
    return st;
}
size_t product(const std::vector<size_t> &v) {
    return std::accumulate(v.begin(), v.end(), size_t(1), std::multiplies<size_t>());
}
} // namespace

// A CPU tensor created while a device runtime is active gets that runtime's
// (pinned) host storage, as tensor.cpp:29-31; otherwise the target device's
// runtime is activated and allocates.
tensor_t Tensor::create(const std::vector<size_t> &shape, llaisysDataType_t dtype, llaisysDeviceType_t device_type,
                        int device_id) {
    size_t bytes = product(shape) * dsize(dtype);
    auto &ctx = core::context();
    core::storage_t st;
    if (device_type == LLAISYS_DEVICE_CPU && ctx.runtime().deviceType() != LLAISYS_DEVICE_CPU) {
        st = ctx.runtime().allocateHostStorage(bytes);
    } else {
        ctx.setDevice(device_type, device_id);
        st = ctx.runtime().allocateDeviceStorage(bytes);
    }
    return tensor_t(new Tensor(dtype, shape, rowMajorStrides(shape), std::move(st), 0));
}

size_t Tensor::numel() const { return product(shape_); }
size_t Tensor::elementSize() const { return dsize(dtype_); }

std::string Tensor::info() const {
    std::ostringstream os;
    os << "Tensor: shape[ ";
    for (auto s : shape_) os << s << " ";
    os << "] strides[ ";
    for (auto s : strides_) os << s << " ";
    os << "] dtype=" << int(dtype_);
    return os.str();
}

namespace {
double elementAsDouble(const std::byte *p, llaisysDataType_t dt) {
    switch (dt) {
    case LLAISYS_DTYPE_BOOL: return double(*reinterpret_cast<const bool *>(p));
    case LLAISYS_DTYPE_I8: return *reinterpret_cast<const int8_t *>(p);
    case LLAISYS_DTYPE_I16: return *reinterpret_cast<const int16_t *>(p);
    case LLAISYS_DTYPE_I32: return *reinterpret_cast<const int32_t *>(p);
    case LLAISYS_DTYPE_I64: return double(*reinterpret_cast<const int64_t *>(p));
    case LLAISYS_DTYPE_BYTE:
    case LLAISYS_DTYPE_U8: return *reinterpret_cast<const uint8_t *>(p);
    case LLAISYS_DTYPE_U16: return *reinterpret_cast<const uint16_t *>(p);
    case LLAISYS_DTYPE_U32: return *reinterpret_cast<const uint32_t *>(p);
    case LLAISYS_DTYPE_U64: return double(*reinterpret_cast<const uint64_t *>(p));
    case LLAISYS_DTYPE_F16: return f16ToF32(*reinterpret_cast<const uint16_t *>(p));
    case LLAISYS_DTYPE_BF16: return bf16ToF32(*reinterpret_cast<const uint16_t *>(p));
    case LLAISYS_DTYPE_F32: return *reinterpret_cast<const float *>(p);
    case LLAISYS_DTYPE_F64: return *reinterpret_cast<const double *>(p);
    default: LLAISYS_RAISE("debug print: unsupported dtype " << dtypeName(dt));
    }
}
void printRec(const std::byte *base, const std::vector<size_t> &shape, const std::vector<ptrdiff_t> &strides,
              size_t dim, size_t esz, llaisysDataType_t dt) {
    if (shape.empty()) {
        std::cout << elementAsDouble(base, dt) << std::endl;
        return;
    }
    if (dim + 1 == shape.size()) {
        for (size_t i = 0; i < shape[dim]; ++i) std::cout << elementAsDouble(base + i * strides[dim] * esz, dt) << " ";
        std::cout << std::endl;
        return;
    }
    for (size_t i = 0; i < shape[dim]; ++i) printRec(base + i * strides[dim] * esz, shape, strides, dim + 1, esz, dt);
}
// Bytes from data() to one past the last element reachable through the strides.
size_t footprint(const std::vector<size_t> &shape, const std::vector<ptrdiff_t> &strides, size_t esz) {
    size_t last = 0;
    for (size_t i = 0; i < shape.size(); ++i) {
        if (shape[i] == 0) return 0;
        last += size_t(strides[i]) * (shape[i] - 1);
    }
    return (last + 1) * esz;
}
} // namespace

// Prints the tensor like tensor.cpp:149-164 (device data is copied to the host first).
void Tensor::debug() const {
    auto &ctx = core::context();
    ctx.setDevice(storage_->isHost() ? ctx.runtime().deviceType() : deviceType(),
                  storage_->isHost() ? ctx.runtime().deviceId() : deviceId());
    ctx.runtime().api()->device_synchronize();
    std::cout << info() << std::endl;
    size_t esz = elementSize();
    if (deviceType() == LLAISYS_DEVICE_CPU) {
        printRec(data(), shape_, strides_, 0, esz, dtype_);
        return;
    }
    size_t bytes = footprint(shape_, strides_, esz);
    std::vector<std::byte> host(bytes);
    if (bytes) ctx.runtime().api()->memcpy_sync(host.data(), data(), bytes, LLAISYS_MEMCPY_D2H);
    printRec(host.data(), shape_, strides_, 0, esz, dtype_);
}

bool Tensor::isContiguous() const {
    ptrdiff_t expect = 1;
    for (size_t i = shape_.size(); i-- > 0;) {
        if (shape_[i] == 1) continue;
        if (strides_[i] != expect) return false;
        expect *= ptrdiff_t(shape_[i]);
    }
    return true;
}

tensor_t Tensor::permute(const std::vector<size_t> &order) const {
    LLAISYS_CHECK(order.size() == ndim(), "permute: order has " << order.size() << " entries for " << ndim() << " dims");
    std::vector<bool> seen(ndim(), false);
    std::vector<size_t> shape(ndim());
    std::vector<ptrdiff_t> strides(ndim());
    for (size_t i = 0; i < order.size(); ++i) {
        LLAISYS_CHECK(order[i] < ndim() && !seen[order[i]], "permute: order is not a permutation");
        seen[order[i]] = true;
        shape[i] = shape_[order[i]];
        strides[i] = strides_[order[i]];
    }
    return tensor_t(new Tensor(dtype_, shape, strides, storage_, offset_));
}

tensor_t Tensor::slice(size_t dim, size_t start, size_t end) const {
    LLAISYS_CHECK(dim < ndim(), "slice: dim " << dim << " out of range");
    LLAISYS_CHECK(start <= end && end <= shape_[dim], "slice: [" << start << ", " << end << ") out of [0, "
                                                               << shape_[dim] << ")");
    auto shape = shape_;
    shape[dim] = end - start;
    size_t off = offset_ + start * size_t(strides_[dim]) * elementSize();
    return tensor_t(new Tensor(dtype_, shape, strides_, storage_, off));
}

// Reshape without moving data. Non-unit old dims are grouped into runs that
// are laid out contiguously with each other; each run must be covered exactly
// by consecutive non-unit new dims, otherwise no strided view exists and this
// raises (README.md:112-118). Unit new dims get the row-major stride.
tensor_t Tensor::view(const std::vector<size_t> &shape) const {
    LLAISYS_CHECK(product(shape) == numel(),
                  "view: " << product(shape) << " elements requested, tensor has " << numel());
    std::vector<size_t> osz;
    std::vector<ptrdiff_t> ost;
    for (size_t i = 0; i < ndim(); ++i)
        if (shape_[i] != 1) {
            osz.push_back(shape_[i]);
            ost.push_back(strides_[i]);
        }
    std::vector<ptrdiff_t> out(shape.size(), 0);
    size_t ni = 0;
    size_t oi = 0;
    while (oi < osz.size()) {
        size_t run_end = oi;
        size_t run_elems = osz[oi];
        while (run_end + 1 < osz.size() && ost[run_end] == ost[run_end + 1] * ptrdiff_t(osz[run_end + 1])) {
            ++run_end;
            run_elems *= osz[run_end];
        }
        std::vector<size_t> group;
        size_t acc = 1;
        while (acc < run_elems && ni < shape.size()) {
            if (shape[ni] != 1) {
                acc *= shape[ni];
                group.push_back(ni);
            }
            ++ni;
        }
        LLAISYS_CHECK(acc == run_elems, "view: shape is not compatible with the tensor's strides");
        ptrdiff_t s = ost[run_end];
        for (size_t k = group.size(); k-- > 0;) {
            out[group[k]] = s;
            s *= ptrdiff_t(shape[group[k]]);
        }
        oi = run_end + 1;
    }
    for (size_t k = shape.size(); k-- > 0;)
        if (shape[k] == 1) out[k] = (k + 1 < shape.size()) ? out[k + 1] * ptrdiff_t(shape[k + 1]) : 1;
    return tensor_t(new Tensor(dtype_, shape, out, storage_, offset_));
}

// Copy numel*elsize bytes of host memory into the tensor (README.md:90-96).
void Tensor::load(const void *host_src) {
    LLAISYS_CHECK(isContiguous(), "load: tensor must be contiguous");
    size_t bytes = numel() * elementSize();
    if (!bytes) return;
    touch();
    auto &ctx = core::context();
    if (deviceType() == LLAISYS_DEVICE_CPU) {
        std::memcpy(data(), host_src, bytes);
        return;
    }
    ctx.setDevice(deviceType(), deviceId());
    ctx.runtime().api()->memcpy_sync(data(), host_src, bytes, LLAISYS_MEMCPY_H2D);
}

} // namespace llaisys
