#include "runtime_api.hpp"

#include "../utils/check.hpp"

namespace llaisys::device {

namespace {
// Table of a device type that is not built in: no devices; anything else is an error.
int noDevices() { return 0; }
void noSetDevice(int) { EXCEPTION_UNSUPPORTED_DEVICE; }
void noSync() { EXCEPTION_UNSUPPORTED_DEVICE; }
llaisysStream_t noCreateStream() { EXCEPTION_UNSUPPORTED_DEVICE; }
void noStream(llaisysStream_t) { EXCEPTION_UNSUPPORTED_DEVICE; }
void *noMalloc(size_t) { EXCEPTION_UNSUPPORTED_DEVICE; }
void noFree(void *) { EXCEPTION_UNSUPPORTED_DEVICE; }
void noCopy(void *, const void *, size_t, llaisysMemcpyKind_t) { EXCEPTION_UNSUPPORTED_DEVICE; }
void noCopyAsync(void *, const void *, size_t, llaisysMemcpyKind_t, llaisysStream_t) {
    EXCEPTION_UNSUPPORTED_DEVICE;
}

const LlaisysRuntimeAPI kAbsent = {&noDevices, &noSetDevice, &noSync,   &noCreateStream,
                                   &noStream,  &noStream,    &noMalloc, &noFree,
                                   &noMalloc,  &noFree,      &noCopy,   &noCopyAsync};
} // namespace

const LlaisysRuntimeAPI *getRuntimeAPI(llaisysDeviceType_t device_type) {
    switch (device_type) {
    case LLAISYS_DEVICE_CPU: return cpu::getRuntimeAPI();
    case LLAISYS_DEVICE_NVIDIA: return &kAbsent;
    case LLAISYS_DEVICE_AMD: return amd::getRuntimeAPI();
    default: EXCEPTION_UNSUPPORTED_DEVICE;
    }
}

} // namespace llaisys::device
