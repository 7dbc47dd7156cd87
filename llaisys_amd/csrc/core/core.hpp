// Per-thread device context, per-device runtime (stream + allocator) and storage blocks.
//
// Same structure and semantics as the reference core (src/core/context/context.cpp:7-99,
// src/core/runtime/runtime.cpp:9-108, src/core/storage/storage.cpp:6-39): one
// thread-local Context; on first use it activates the first GPU found (non-CPU device
// types are probed first, CPU last); each (device type, id) gets one Runtime with one
// stream, created on first use; a Storage frees itself through the Runtime that made it.
#pragma once

#include "llaisys/runtime.h"

#include <cstddef>
#include <memory>
#include <unordered_map>
#include <vector>

namespace llaisys::core {

class Runtime;

class Storage {
public:
    ~Storage();
    std::byte *memory() const { return _mem; }
    size_t size() const { return _size; }
    bool isHost() const { return _host; }
    llaisysDeviceType_t deviceType() const;
    int deviceId() const;

private:
    friend class Runtime;
    Storage(std::byte *mem, size_t size, Runtime &rt, bool host)
        : _mem(mem), _size(size), _rt(rt), _host(host) {}
    std::byte *_mem;
    size_t _size;
    Runtime &_rt;
    bool _host;
};
using storage_t = std::shared_ptr<Storage>;

class Runtime {
public:
    ~Runtime();
    Runtime(const Runtime &) = delete;
    Runtime &operator=(const Runtime &) = delete;

    llaisysDeviceType_t deviceType() const { return _type; }
    int deviceId() const { return _id; }
    const LlaisysRuntimeAPI *api() const { return _api; }
    llaisysStream_t stream() const { return _stream; }

    storage_t allocateDeviceStorage(size_t bytes);
    storage_t allocateHostStorage(size_t bytes);
    void release(Storage *s);
    void synchronize() const;

private:
    friend class Context;
    Runtime(llaisysDeviceType_t type, int id);
    void activate() const;

    llaisysDeviceType_t _type;
    int _id;
    const LlaisysRuntimeAPI *_api;
    llaisysStream_t _stream;
};

class Context {
public:
    ~Context();
    Context(const Context &) = delete;
    Context &operator=(const Context &) = delete;

    // Makes (type, id) current, creating its Runtime on first use; throws
    // "invalid device id" for an id the device type does not have.
    void setDevice(llaisysDeviceType_t type, int id);
    Runtime &runtime();

private:
    friend Context &context();
    Context();
    std::unordered_map<int, std::vector<std::unique_ptr<Runtime>>> _runtimes;
    Runtime *_current = nullptr;
};

Context &context();

} // namespace llaisys::core
