#include "tensor.hpp"

#include "../device/runtime_api.hpp"
#include "../kernels/launch.hpp"
#include "../utils/check.hpp"
#include "../utils/types.hpp"

#include <cstring>
#include <iostream>
#include <sstream>

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

size_t product(const std::vector<size_t> &shape) {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    return n;
}
} // namespace

tensor_t Tensor::create(const std::vector<size_t> &shape, llaisysDataType_t dtype,
                        llaisysDeviceType_t device_type, int device) {
    const size_t bytes = product(shape) * utils::dsize(dtype);
    auto &ctx = core::context();
    core::storage_t storage;
    // A CPU tensor made while a GPU runtime is current gets pinned host memory from that
    // runtime (reference tensor.cpp:32-34); otherwise the target device allocates.
    if (device_type == LLAISYS_DEVICE_CPU && ctx.runtime().deviceType() != LLAISYS_DEVICE_CPU) {
        storage = ctx.runtime().allocateHostStorage(bytes);
    } else {
        ctx.setDevice(device_type, device);
        storage = ctx.runtime().allocateDeviceStorage(bytes);
    }
    return tensor_t(new Tensor(dtype, shape, rowMajorStrides(shape), std::move(storage), 0));
}

size_t Tensor::numel() const { return product(_shape); }

size_t Tensor::elementSize() const { return utils::dsize(_dtype); }

bool Tensor::isContiguous() const {
    ptrdiff_t expect = 1;
    for (size_t i = _shape.size(); i-- > 0;) {
        if (_strides[i] != expect) return false;
        expect *= ptrdiff_t(_shape[i]);
    }
    return true;
}

std::string Tensor::info() const {
    std::ostringstream os;
    os << "Tensor: shape[ ";
    for (auto s : _shape) os << s << " ";
    os << "] strides[ ";
    for (auto s : _strides) os << s << " ";
    os << "] dtype=" << _dtype;
    return os.str();
}

namespace {
template <typename T, typename F>
void printRows(const std::byte *base, const std::vector<size_t> &shape,
               const std::vector<ptrdiff_t> &strides, size_t dim, F widen) {
    const T *p = reinterpret_cast<const T *>(base);
    if (dim + 1 == shape.size()) {
        for (size_t i = 0; i < shape[dim]; i++) std::cout << widen(p[i * strides[dim]]) << " ";
        std::cout << std::endl;
        return;
    }
    for (size_t i = 0; i < shape[dim]; i++)
        printRows<T>(base + i * strides[dim] * sizeof(T), shape, strides, dim + 1, widen);
}

void printTensor(const std::byte *p, const std::vector<size_t> &shape,
                 const std::vector<ptrdiff_t> &strides, llaisysDataType_t dt) {
    if (shape.empty()) return;
    auto same = [](auto v) { return v; };
    auto asInt = [](auto v) { return int(v); };
    switch (dt) {
    case LLAISYS_DTYPE_BYTE:
    case LLAISYS_DTYPE_I8: return printRows<int8_t>(p, shape, strides, 0, asInt);
    case LLAISYS_DTYPE_BOOL:
    case LLAISYS_DTYPE_U8: return printRows<uint8_t>(p, shape, strides, 0, asInt);
    case LLAISYS_DTYPE_I16: return printRows<int16_t>(p, shape, strides, 0, same);
    case LLAISYS_DTYPE_U16: return printRows<uint16_t>(p, shape, strides, 0, same);
    case LLAISYS_DTYPE_I32: return printRows<int32_t>(p, shape, strides, 0, same);
    case LLAISYS_DTYPE_U32: return printRows<uint32_t>(p, shape, strides, 0, same);
    case LLAISYS_DTYPE_I64: return printRows<int64_t>(p, shape, strides, 0, same);
    case LLAISYS_DTYPE_U64: return printRows<uint64_t>(p, shape, strides, 0, same);
    case LLAISYS_DTYPE_F32: return printRows<float>(p, shape, strides, 0, same);
    case LLAISYS_DTYPE_F64: return printRows<double>(p, shape, strides, 0, same);
    case LLAISYS_DTYPE_BF16:
        return printRows<uint16_t>(p, shape, strides, 0, utils::bf16_bits_to_f32);
    case LLAISYS_DTYPE_F16:
        return printRows<uint16_t>(p, shape, strides, 0, utils::f16_bits_to_f32);
    default: EXCEPTION_UNSUPPORTED_DATATYPE(dt);
    }
}

// Span in elements from the first to one past the last addressed element.
size_t extent(const std::vector<size_t> &shape, const std::vector<ptrdiff_t> &strides) {
    size_t e = 1;
    for (size_t i = 0; i < shape.size(); i++) {
        if (shape[i] == 0) return 0;
        e += size_t(strides[i]) * (shape[i] - 1);
    }
    return e;
}
} // namespace

void Tensor::debug() const {
    auto &ctx = core::context();
    ctx.setDevice(deviceType(), deviceId());
    ctx.runtime().api()->device_synchronize();
    std::cout << info() << std::endl;
    if (deviceType() == LLAISYS_DEVICE_CPU) {
        printTensor(data(), _shape, _strides, _dtype);
        return;
    }
    const size_t bytes = extent(_shape, _strides) * elementSize();
    std::vector<std::byte> host(bytes);
    ctx.runtime().api()->memcpy_sync(host.data(), data(), bytes, LLAISYS_MEMCPY_D2H);
    printTensor(host.data(), _shape, _strides, _dtype);
}

tensor_t Tensor::permute(const std::vector<size_t> &order) const {
    if (order.size() != _shape.size()) throw std::runtime_error("Permute dimensions mismatch.");
    std::vector<size_t> shape(order.size());
    std::vector<ptrdiff_t> strides(order.size());
    std::vector<bool> seen(order.size(), false);
    for (size_t i = 0; i < order.size(); i++) {
        const size_t d = order[i];
        if (d >= _shape.size() || seen[d]) throw std::runtime_error("Permute dimensions mismatch.");
        seen[d] = true;
        shape[i] = _shape[d];
        strides[i] = _strides[d];
    }
    return tensor_t(new Tensor(_dtype, shape, strides, _storage, _offset));
}

tensor_t Tensor::view(const std::vector<size_t> &shape) const {
    if (product(shape) != numel())
        throw std::runtime_error("View shape mismatch: numel must be the same.");
    if (!isContiguous())
        throw std::runtime_error("View on non-contiguous tensor is not supported yet.");
    return tensor_t(new Tensor(_dtype, shape, rowMajorStrides(shape), _storage, _offset));
}

tensor_t Tensor::slice(size_t dim, size_t start, size_t end) const {
    if (dim >= _shape.size()) throw std::runtime_error("Slice dimesion out of range.\n");
    if (start >= end || end > _shape[dim])
        throw std::runtime_error("Slice : Argument start or end out of range.\n");
    std::vector<size_t> shape = _shape;
    shape[dim] = end - start;
    const size_t off = _offset + start * size_t(_strides[dim]) * elementSize();
    return tensor_t(new Tensor(_dtype, shape, _strides, _storage, off));
}

void Tensor::load(const void *src) {
    const size_t bytes = numel() * elementSize();
    device::getRuntimeAPI(_storage->deviceType())
        ->memcpy_sync(data(), src, bytes, LLAISYS_MEMCPY_H2D);
}

namespace {
// host strided copy of one element at a time (host tensors only: data movement, not compute)
void hostCopy(std::byte *dst, const std::vector<ptrdiff_t> &sdst, const std::byte *src,
              const std::vector<ptrdiff_t> &ssrc, const std::vector<size_t> &shape, size_t dim,
              size_t esize) {
    if (dim == shape.size()) {
        std::memcpy(dst, src, esize);
        return;
    }
    for (size_t i = 0; i < shape[dim]; i++)
        hostCopy(dst + ptrdiff_t(i) * sdst[dim] * ptrdiff_t(esize), sdst,
                 src + ptrdiff_t(i) * ssrc[dim] * ptrdiff_t(esize), ssrc, shape, dim + 1, esize);
}
} // namespace

void Tensor::copyInto(const tensor_t &out) const {
    CHECK_ARGUMENT(out->shape() == _shape, "copy: shapes differ");
    CHECK_ARGUMENT(out->dtype() == _dtype, "copy: dtypes differ");
    CHECK_ARGUMENT(out->deviceType() == deviceType() && out->deviceId() == deviceId(),
                   "copy: tensors on different devices");
    CHECK_ARGUMENT(_shape.size() <= 8, "copy: at most 8 dimensions");
    if (numel() == 0) return;
    if (deviceType() == LLAISYS_DEVICE_CPU) {
        hostCopy(out->data(), out->strides(), data(), _strides, _shape, 0, elementSize());
        return;
    }
    auto &ctx = core::context();
    ctx.setDevice(deviceType(), deviceId());
    auto s = static_cast<hipStream_t>(ctx.runtime().stream());
    kernels::rearrange(out->data(), data(), _shape.size(), _shape.data(), _strides.data(),
                       out->strides().data(), elementSize(), s);
    device::amd::check(hipGetLastError(), "rearrange");
}

tensor_t Tensor::contiguous() const {
    if (isContiguous()) return tensor_t(new Tensor(_dtype, _shape, _strides, _storage, _offset));
    tensor_t out = create(_shape, _dtype, deviceType(), deviceId());
    copyInto(out);
    return out;
}

tensor_t Tensor::reshape(const std::vector<size_t> &shape) const {
    if (product(shape) != numel())
        throw std::runtime_error("Reshape shape mismatch: numel must be the same.");
    return contiguous()->view(shape);
}

tensor_t Tensor::to(llaisysDeviceType_t device_type, int device) const {
    if (device < 0) device = device_type == deviceType() ? deviceId() : 0;
    if (device_type == deviceType() && device == deviceId())
        return tensor_t(new Tensor(_dtype, _shape, _strides, _storage, _offset));
    const tensor_t src = contiguous();
    tensor_t dst = create(_shape, _dtype, device_type, device);
    const size_t bytes = numel() * elementSize();
    if (bytes == 0) return dst;
    auto &ctx = core::context();
    const bool fromGpu = deviceType() != LLAISYS_DEVICE_CPU, toGpu = device_type != LLAISYS_DEVICE_CPU;
    if (fromGpu) { // the source may still be written by work queued on its stream
        ctx.setDevice(deviceType(), deviceId());
        ctx.runtime().api()->device_synchronize();
    }
    if (!fromGpu && !toGpu) {
        std::memcpy(dst->data(), src->data(), bytes);
        return dst;
    }
    const llaisysMemcpyKind_t kind = fromGpu && toGpu ? LLAISYS_MEMCPY_D2D
                                     : fromGpu         ? LLAISYS_MEMCPY_D2H
                                                       : LLAISYS_MEMCPY_H2D;
    ctx.setDevice(toGpu ? device_type : deviceType(), toGpu ? device : deviceId());
    ctx.runtime().api()->memcpy_sync(dst->data(), src->data(), bytes, kind);
    return dst;
}

} // namespace llaisys
