#include "core.hpp"

#include "../device/runtime_api.hpp"
#include "../utils/check.hpp"

namespace llaisys::core {

// ---- Storage -------------------------------------------------------------------------

Storage::~Storage() { _rt.release(this); }

llaisysDeviceType_t Storage::deviceType() const {
    return _host ? LLAISYS_DEVICE_CPU : _rt.deviceType();
}

int Storage::deviceId() const { return _host ? 0 : _rt.deviceId(); }

// ---- Runtime -------------------------------------------------------------------------

Runtime::Runtime(llaisysDeviceType_t type, int id)
    : _type(type), _id(id), _api(device::getRuntimeAPI(type)), _stream(nullptr) {
    _api->set_device(_id);
    _stream = _api->create_stream();
}

Runtime::~Runtime() {
    _api->set_device(_id);
    _api->destroy_stream(_stream);
}

void Runtime::activate() const { _api->set_device(_id); }

storage_t Runtime::allocateDeviceStorage(size_t bytes) {
    auto *mem = static_cast<std::byte *>(_api->malloc_device(bytes));
    return storage_t(new Storage(mem, bytes, *this, false));
}

storage_t Runtime::allocateHostStorage(size_t bytes) {
    auto *mem = static_cast<std::byte *>(_api->malloc_host(bytes));
    return storage_t(new Storage(mem, bytes, *this, true));
}

void Runtime::release(Storage *s) {
    if (s->isHost())
        _api->free_host(s->memory());
    else
        _api->free_device(s->memory());
}

void Runtime::synchronize() const { _api->stream_synchronize(_stream); }

// ---- Context -------------------------------------------------------------------------

Context::Context() {
    // GPU device types first, the CPU last; the first device found becomes current.
    std::vector<llaisysDeviceType_t> order;
    for (int t = 1; t < LLAISYS_DEVICE_TYPE_COUNT; ++t)
        order.push_back(static_cast<llaisysDeviceType_t>(t));
    order.push_back(LLAISYS_DEVICE_CPU);
    for (auto t : order) {
        const int n = device::getRuntimeAPI(t)->get_device_count();
        auto &slots = _runtimes[t];
        slots.resize(n > 0 ? size_t(n) : 0);
        if (!_current && n > 0) {
            slots[0].reset(new Runtime(t, 0));
            _current = slots[0].get();
        }
    }
}

Context::~Context() {
    // Runtimes (streams) are deliberately kept until the process ends: tensors that
    // outlive the thread still free through them, and at process exit the HIP runtime
    // may already be torn down when thread-local destructors run.
    for (auto &kv : _runtimes)
        for (auto &rt : kv.second) (void)rt.release();
    _current = nullptr;
}

void Context::setDevice(llaisysDeviceType_t type, int id) {
    if (_current && _current->deviceType() == type && _current->deviceId() == id) return;
    auto &slots = _runtimes[type];
    CHECK_ARGUMENT(id >= 0 && size_t(id) < slots.size(), "invalid device id");
    if (!slots[id]) slots[id].reset(new Runtime(type, id));
    slots[id]->activate();
    _current = slots[id].get();
}

Runtime &Context::runtime() {
    ASSERT(_current != nullptr, "No runtime is activated, please call setDevice() first.");
    return *_current;
}

Context &context() {
    thread_local Context ctx;
    return ctx;
}

} // namespace llaisys::core
