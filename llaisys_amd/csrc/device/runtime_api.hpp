// Device runtime tables (LlaisysRuntimeAPI) and the AMD device helpers the ops need.
#pragma once

#include "llaisys/runtime.h"

namespace llaisys::device {

// Table for a device type: CPU, AMD (HIP), or the "no devices" table for NVIDIA.
// Mirrors the registry of the reference (src/device/runtime_api.cpp:73-88).
const LlaisysRuntimeAPI *getRuntimeAPI(llaisysDeviceType_t device_type);

namespace cpu {
const LlaisysRuntimeAPI *getRuntimeAPI();
}

namespace amd {
const LlaisysRuntimeAPI *getRuntimeAPI();

// Sticky per-device error word written by kernels (0 = none).  Allocated on first use;
// the device must be current.
int *errorWord(int device_id);
// Reads and clears the error word of the current device after `stream` drained.
int takeError(llaisysStream_t stream);
// Same, but prints and throws when the word is set (used by the synchronize calls).
void raiseIfError(llaisysStream_t stream);

// Grow-only scratch for multi-block kernels (partial results and a completion counter),
// one per (thread, device) because each thread launches on its own stream.  Returns at
// least `bytes` of device memory, zeroed when first allocated.  A growth moves the thread
// to a new buffer; the old one is freed once no captured graph holds it.
void *workspace(int device_id, size_t bytes);

// HIP-graph capture of the work enqueued on `stream` (the current device's context stream).
// beginCapture reserves the workspace a captured op may need (growth during capture is an
// error); the graph keeps the workspace it captured alive until destroyGraph.
void beginCapture(int device_id, llaisysStream_t stream);
llaisysGraph_t endCapture(int device_id, llaisysStream_t stream);
void launchGraph(llaisysGraph_t g);
void destroyGraph(llaisysGraph_t g);

// Checks a HIP status code; prints "[ERROR] HIP <what>: <message>" and throws.
void check(int status, const char *what);
} // namespace amd

} // namespace llaisys::device
