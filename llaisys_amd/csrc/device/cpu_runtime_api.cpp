// Host "device": plain malloc and memcpy, no streams (reference
// src/device/cpu/cpu_runtime_api.cpp:10-53 has the same behaviour).
#include "runtime_api.hpp"

#include <cstdlib>
#include <cstring>

namespace llaisys::device::cpu {

namespace {
int count() { return 1; }
void setDevice(int) {}
void sync() {}
llaisysStream_t createStream() { return nullptr; }
void destroyStream(llaisysStream_t) {}
void streamSync(llaisysStream_t) {}
void *alloc(size_t n) { return std::malloc(n); }
void release(void *p) { std::free(p); }
void copy(void *dst, const void *src, size_t n, llaisysMemcpyKind_t) { std::memcpy(dst, src, n); }
void copyAsync(void *dst, const void *src, size_t n, llaisysMemcpyKind_t k, llaisysStream_t) {
    copy(dst, src, n, k);
}

const LlaisysRuntimeAPI kTable = {&count,  &setDevice,     &sync,  &createStream,
                                  &destroyStream, &streamSync, &alloc, &release,
                                  &alloc,  &release,      &copy,  &copyAsync};
} // namespace

const LlaisysRuntimeAPI *getRuntimeAPI() { return &kTable; }

} // namespace llaisys::device::cpu
