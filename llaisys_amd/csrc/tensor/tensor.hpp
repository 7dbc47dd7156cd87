// Tensor = dtype + shape + strides (elements) + byte offset over a shared Storage.
//
// Semantics follow the reference Tensor (src/tensor/tensor.hpp:9-58,
// src/tensor/tensor.cpp:17-342).  One deliberate difference: view() and permute() keep
// the byte offset of the source tensor, where the reference resets it to 0
// (tensor.cpp:210,239), so a view of a slice addresses the slice's data.
#pragma once

#include "../core/core.hpp"

#include "llaisys.h"

#include <memory>
#include <string>
#include <vector>

namespace llaisys {

class Tensor;
using tensor_t = std::shared_ptr<Tensor>;

class Tensor {
public:
    static tensor_t create(const std::vector<size_t> &shape, llaisysDataType_t dtype,
                           llaisysDeviceType_t device_type = LLAISYS_DEVICE_CPU,
                           int device = 0);

    std::byte *data() const { return _storage->memory() + _offset; }
    size_t ndim() const { return _shape.size(); }
    const std::vector<size_t> &shape() const { return _shape; }
    const std::vector<ptrdiff_t> &strides() const { return _strides; }
    llaisysDataType_t dtype() const { return _dtype; }
    llaisysDeviceType_t deviceType() const { return _storage->deviceType(); }
    int deviceId() const { return _storage->deviceId(); }
    size_t numel() const;
    size_t elementSize() const;
    bool isContiguous() const;

    std::string info() const;
    void debug() const;

    tensor_t permute(const std::vector<size_t> &order) const;
    tensor_t slice(size_t dim, size_t start, size_t end) const;
    tensor_t view(const std::vector<size_t> &shape) const;

    // Synchronous copy of numel() * elementSize() bytes from host memory.
    void load(const void *src);

    // Reference tensor.hpp:55-57 (stubs there, tensor.cpp:344-357).
    // contiguous(): this tensor when already contiguous (shared storage), else a new
    // contiguous tensor on the same device holding a copy (a GPU rearrange on AMD devices).
    tensor_t contiguous() const;
    // reshape(): a view when contiguous, else a view of contiguous().
    tensor_t reshape(const std::vector<size_t> &shape) const;
    // to(): this tensor when already on (device_type, device), else a contiguous copy there.
    // device < 0 means this tensor's device id for the same device type, else 0.
    tensor_t to(llaisysDeviceType_t device_type, int device = -1) const;
    // Element-by-element copy into `out` (same shape and dtype, same device).
    void copyInto(const tensor_t &out) const;

private:
    Tensor(llaisysDataType_t dt, std::vector<size_t> shape, std::vector<ptrdiff_t> strides,
           core::storage_t storage, size_t offset)
        : _dtype(dt), _shape(std::move(shape)), _strides(std::move(strides)),
          _storage(std::move(storage)), _offset(offset) {}

    llaisysDataType_t _dtype;
    std::vector<size_t> _shape;
    std::vector<ptrdiff_t> _strides;
    core::storage_t _storage;
    size_t _offset;
};

} // namespace llaisys
