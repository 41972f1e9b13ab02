// Strided tensor = dtype/shape/strides + shared Storage + byte offset
// (reference: src/tensor/tensor.hpp:9-58). Shapes are size_t, strides are in
// elements, the offset is in bytes (tensor.cpp:39-41).
#pragma once

#include "../core/core.hpp"

#include <memory>
#include <string>
#include <vector>

namespace llaisys {

class Tensor;
using tensor_t = std::shared_ptr<Tensor>;

class Tensor {
public:
    static tensor_t create(const std::vector<size_t> &shape, llaisysDataType_t dtype,
                           llaisysDeviceType_t device_type = LLAISYS_DEVICE_CPU, int device_id = 0);

    std::byte *data() const { return storage_->memory() + offset_; }
    size_t ndim() const { return shape_.size(); }
    const std::vector<size_t> &shape() const { return shape_; }
    const std::vector<ptrdiff_t> &strides() const { return strides_; }
    llaisysDataType_t dtype() const { return dtype_; }
    llaisysDeviceType_t deviceType() const { return storage_->deviceType(); }
    int deviceId() const { return storage_->deviceId(); }
    size_t numel() const;
    size_t elementSize() const;

    std::string info() const;
    void debug() const;
    bool isContiguous() const;

    tensor_t permute(const std::vector<size_t> &order) const;
    tensor_t slice(size_t dim, size_t start, size_t end) const;
    tensor_t view(const std::vector<size_t> &shape) const;
    void load(const void *host_src);
    // Write generation of the underlying storage (shared by views and slices).
    uint64_t version() const { return storage_->version(); }
    void touch() const { storage_->touch(); }

private:
    Tensor(llaisysDataType_t dtype, std::vector<size_t> shape, std::vector<ptrdiff_t> strides,
           core::storage_t storage, size_t offset)
        : dtype_(dtype), shape_(std::move(shape)), strides_(std::move(strides)), storage_(std::move(storage)),
          offset_(offset) {}

    llaisysDataType_t dtype_;
    std::vector<size_t> shape_;
    std::vector<ptrdiff_t> strides_;
    core::storage_t storage_;
    size_t offset_;
};

} // namespace llaisys
