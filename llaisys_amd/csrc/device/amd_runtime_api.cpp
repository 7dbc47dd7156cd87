// The AMD (HIP) device table: one MI355X GPU per device id.
//
// Plays the role of the reference's (stubbed) NVIDIA table,
// src/device/nvidia/nvidia_runtime_api.cu:9-74, on HIP.  Streams are created with the
// default priority.  Host allocations are pinned (hipHostMalloc) so that tensorLoad and
// D2H copies run at full PCIe rate.
#include "runtime_api.hpp"

#include "../utils/check.hpp"

#include <hip/hip_runtime_api.h>

#include "../kernels/launch.hpp"

#include <cstdlib>
#include <memory>
#include <mutex>
#include <vector>

namespace llaisys::device::amd {

void check(int status, const char *what) {
    if (status != hipSuccess) {
        const char *msg = hipGetErrorString(static_cast<hipError_t>(status));
        LLAISYS_FAIL(std::runtime_error, "HIP " << what << ": " << msg, msg);
    }
}

namespace {

hipMemcpyKind toHip(llaisysMemcpyKind_t k) {
    switch (k) {
    case LLAISYS_MEMCPY_H2H: return hipMemcpyHostToHost;
    case LLAISYS_MEMCPY_H2D: return hipMemcpyHostToDevice;
    case LLAISYS_MEMCPY_D2H: return hipMemcpyDeviceToHost;
    case LLAISYS_MEMCPY_D2D: return hipMemcpyDeviceToDevice;
    }
    return hipMemcpyDefault;
}

int count() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError(); // no driver / no GPU: report none, leave no sticky error
        return 0;
    }
    return n;
}

void setDevice(int id) { check(hipSetDevice(id), "hipSetDevice"); }

void sync() {
    check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    raiseIfError(nullptr);
}

llaisysStream_t createStream() {
    hipStream_t s = nullptr;
    check(hipStreamCreate(&s), "hipStreamCreate");
    return s;
}

// Teardown paths ignore errors: at process exit the HIP runtime may already be gone.
void destroyStream(llaisysStream_t s) {
    if (s) (void)hipStreamDestroy(static_cast<hipStream_t>(s));
}

void streamSync(llaisysStream_t s) {
    check(hipStreamSynchronize(static_cast<hipStream_t>(s)), "hipStreamSynchronize");
    raiseIfError(s);
}

void *mallocDevice(size_t n) {
    void *p = nullptr;
    check(hipMalloc(&p, n ? n : 1), "hipMalloc");
    return p;
}

void freeDevice(void *p) {
    if (p) (void)hipFree(p);
}

void *mallocHost(size_t n) {
    void *p = nullptr;
    check(hipHostMalloc(&p, n ? n : 1, hipHostMallocDefault), "hipHostMalloc");
    return p;
}

void freeHost(void *p) {
    if (p) (void)hipHostFree(p);
}

void copy(void *dst, const void *src, size_t n, llaisysMemcpyKind_t k) {
    if (n) check(hipMemcpy(dst, src, n, toHip(k)), "hipMemcpy");
}

void copyAsync(void *dst, const void *src, size_t n, llaisysMemcpyKind_t k, llaisysStream_t s) {
    if (n)
        check(hipMemcpyAsync(dst, src, n, toHip(k), static_cast<hipStream_t>(s)),
              "hipMemcpyAsync");
}

const LlaisysRuntimeAPI kTable = {&count,         &setDevice,  &sync,         &createStream,
                                  &destroyStream, &streamSync, &mallocDevice, &freeDevice,
                                  &mallocHost,    &freeHost,   &copy,         &copyAsync};

constexpr int kMaxDevices = 64;
std::mutex g_mu;
int *g_err[kMaxDevices] = {};
// Workspaces are per thread: every thread has its own Context and hence its own stream
// per device, and stream order is what makes reuse of a workspace safe.  A buffer is
// shared: the thread's slot holds the current one, and every graph captured on it holds
// it too, so a later growth (which moves the slot to a bigger buffer) never frees memory
// that a graph's kernels still address.  The last owner frees it.
struct WsBuffer {
    void *ptr = nullptr;
    size_t size = 0;
    WsBuffer(const WsBuffer &) = delete;
    WsBuffer &operator=(const WsBuffer &) = delete;
    WsBuffer(void *p, size_t n) : ptr(p), size(n) {}
    ~WsBuffer() {
        // kernels queued on any stream may still use it; teardown ignores errors
        (void)hipDeviceSynchronize();
        (void)hipFree(ptr);
    }
};
struct WsSlots {
    std::shared_ptr<WsBuffer> buf[kMaxDevices];
    bool capturing[kMaxDevices] = {};
};
// Never destroyed: at thread (and process) exit the HIP runtime may already be gone, so
// the thread's buffers are left to the driver, as any device memory at exit.
WsSlots &wsSlots() {
    thread_local WsSlots *slots = new WsSlots();
    return *slots;
}

// Workspace reserved when a capture starts (bytes beyond the library's reserved head):
// enough for every attention launch (its partials are capped at 64 MiB).  The environment
// variable LLAISYS_GRAPH_WORKSPACE_BYTES overrides it.
size_t captureReserve() {
    if (const char *e = std::getenv("LLAISYS_GRAPH_WORKSPACE_BYTES")) {
        char *end = nullptr;
        const unsigned long long v = std::strtoull(e, &end, 10);
        if (end != e && *end == '\0') return size_t(v);
    }
    return size_t(64) << 20;
}

int currentDevice() {
    int d = 0;
    check(hipGetDevice(&d), "hipGetDevice");
    CHECK_ARGUMENT(d >= 0 && d < kMaxDevices, "device id out of range");
    return d;
}

} // namespace

const LlaisysRuntimeAPI *getRuntimeAPI() { return &kTable; }

int *errorWord(int dev) {
    CHECK_ARGUMENT(dev >= 0 && dev < kMaxDevices, "device id out of range");
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_err[dev]) {
        void *p = nullptr;
        check(hipMalloc(&p, sizeof(int)), "hipMalloc(error word)");
        check(hipMemset(p, 0, sizeof(int)), "hipMemset(error word)");
        g_err[dev] = static_cast<int *>(p);
    }
    return g_err[dev];
}

int takeError(llaisysStream_t s) {
    const int dev = currentDevice();
    int *w = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        w = g_err[dev];
    }
    if (!w) return 0; // no kernel that reports errors ran on this device yet
    check(hipStreamSynchronize(static_cast<hipStream_t>(s)), "hipStreamSynchronize");
    int code = 0;
    check(hipMemcpy(&code, w, sizeof(int), hipMemcpyDeviceToHost), "hipMemcpy(error word)");
    if (code) check(hipMemset(w, 0, sizeof(int)), "hipMemset(error word)");
    return code;
}

void raiseIfError(llaisysStream_t s) {
    const int code = takeError(s);
    if (code == 1) ASSERT(false, "Embedding index out of bound");
    if (code != 0) LLAISYS_FAIL(std::runtime_error, "device error code " << code, "device error");
}

void *workspace(int dev, size_t bytes) {
    CHECK_ARGUMENT(dev >= 0 && dev < kMaxDevices, "device id out of range");
    WsSlots &ws = wsSlots();
    std::shared_ptr<WsBuffer> &cur = ws.buf[dev];
    if (!cur || cur->size < bytes) {
        // Growing inside a capture would record a synchronisation and a memset into the
        // graph and hand the graph a buffer chosen mid-recording: refuse it.
        if (ws.capturing[dev])
            LLAISYS_FAIL(std::runtime_error,
                         "library workspace must grow to " << bytes
                             << " bytes during HIP graph capture; set LLAISYS_GRAPH_WORKSPACE_BYTES "
                                "above that before llaisysGraphBeginCapture",
                         "workspace growth during capture");
        size_t n = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
        void *p = nullptr;
        check(hipMalloc(&p, n), "hipMalloc(workspace)");
        // Kernels that keep a completion counter in the workspace expect it zeroed once.
        const int st = hipMemset(p, 0, n);
        if (st != hipSuccess) {
            (void)hipFree(p);
            check(st, "hipMemset(workspace)");
        }
        // The old buffer is freed (after a device synchronisation) once no graph holds it.
        cur = std::make_shared<WsBuffer>(p, n);
    }
    return cur->ptr;
}

} // namespace llaisys::device::amd

struct LlaisysGraph {
    hipGraph_t graph;
    hipGraphExec_t exec;
    hipStream_t stream;
    // the workspace the captured kernels address: kept alive until the graph is destroyed
    std::shared_ptr<llaisys::device::amd::WsBuffer> workspace;
};

namespace llaisys::device::amd {

void beginCapture(int dev, llaisysStream_t s) {
    // Everything an op may allocate lazily must exist before capture starts.
    (void)errorWord(dev);
    (void)workspace(dev, kernels::kScratchReserved + captureReserve());
    check(hipStreamBeginCapture(static_cast<hipStream_t>(s), hipStreamCaptureModeRelaxed),
          "hipStreamBeginCapture");
    wsSlots().capturing[dev] = true;
}

llaisysGraph_t endCapture(int dev, llaisysStream_t s) {
    CHECK_ARGUMENT(dev >= 0 && dev < kMaxDevices, "device id out of range");
    WsSlots &ws = wsSlots();
    ws.capturing[dev] = false;
    auto *g = new LlaisysGraph{nullptr, nullptr, static_cast<hipStream_t>(s), ws.buf[dev]};
    const int st = hipStreamEndCapture(g->stream, &g->graph);
    if (st != hipSuccess) {
        delete g;
        check(st, "hipStreamEndCapture");
    }
    const int st2 = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (st2 != hipSuccess) {
        (void)hipGraphDestroy(g->graph);
        delete g;
        check(st2, "hipGraphInstantiate");
    }
    return g;
}

void launchGraph(llaisysGraph_t g) {
    CHECK_ARGUMENT(g != nullptr, "null graph");
    check(hipGraphLaunch(g->exec, g->stream), "hipGraphLaunch");
}

void destroyGraph(llaisysGraph_t g) {
    if (!g) return;
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
}

} // namespace llaisys::device::amd
