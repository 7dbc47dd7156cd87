/*
 * LLAISYS C ABI -- device runtime table.
 *
 * The function-pointer table and the two entry points are the reference's
 * include/llaisys/runtime.h:9-52 (same order of the 12 members, same signatures; the
 * Python mirror is python/llaisys/libllaisys/runtime.py:24-38).  For LLAISYS_DEVICE_AMD
 * the table is filled with HIP calls (hipGetDeviceCount, hipSetDevice, hipStreamCreate,
 * hipMalloc, hipHostMalloc, hipMemcpy/Async ...).
 */
#ifndef LLAISYS_RUNTIME_H
#define LLAISYS_RUNTIME_H

#include "../llaisys.h"

__C {
    typedef int (*get_device_count_api)();
    typedef void (*set_device_api)(int);
    typedef void (*device_synchronize_api)();
    typedef llaisysStream_t (*create_stream_api)();
    typedef void (*destroy_stream_api)(llaisysStream_t);
    typedef void (*stream_synchronize_api)(llaisysStream_t);
    typedef void *(*malloc_device_api)(size_t);
    typedef void (*free_device_api)(void *);
    typedef void *(*malloc_host_api)(size_t);
    typedef void (*free_host_api)(void *);
    typedef void (*memcpy_sync_api)(void *, const void *, size_t, llaisysMemcpyKind_t);
    typedef void (*memcpy_async_api)(void *, const void *, size_t, llaisysMemcpyKind_t,
                                     llaisysStream_t);

    struct LlaisysRuntimeAPI {
        get_device_count_api get_device_count;
        set_device_api set_device;
        device_synchronize_api device_synchronize;
        create_stream_api create_stream;
        destroy_stream_api destroy_stream;
        stream_synchronize_api stream_synchronize;
        malloc_device_api malloc_device;
        free_device_api free_device;
        malloc_host_api malloc_host;
        free_host_api free_host;
        memcpy_sync_api memcpy_sync;
        memcpy_async_api memcpy_async;
    };

    /* reference runtime.h:49 */
    __export const LlaisysRuntimeAPI *llaisysGetRuntimeAPI(llaisysDeviceType_t);

    /* reference runtime.h:52 -- makes (device_type, device_id) current for this thread */
    __export void llaisysSetContextRuntime(llaisysDeviceType_t, int);

    /* Additive (no counterpart in the reference, whose stream is private to its Runtime,
     * src/core/runtime/runtime.cpp:17,101-103): makes (device_type, device_id) current for
     * this thread and returns the stream every op on that device is launched on.  Callers
     * use it to order their own work (events, copies) with the ops. */
    __export llaisysStream_t llaisysGetContextStream(llaisysDeviceType_t, int);

    /* Additive: errors found on the device cannot throw at launch time.  This waits for
     * the context stream of (device_type, device_id), returns the sticky device error
     * code and clears it: 0 = none, 1 = an embedding id outside [0, vocab) (the reference
     * throws "Embedding index out of bound", src/ops/embedding/cpu/embedding_cpu.cpp:18).
     * device_synchronize / stream_synchronize of the AMD table raise the same error
     * (print + throw, like every other LLAISYS error) when it is set. */
    __export int llaisysTakeDeviceError(llaisysDeviceType_t, int);

    /* Additive: HIP-graph capture of op sequences, for launch-bound callers (a decoder
     * layer chain issues ~7 small kernels per layer; replaying a captured graph removes the
     * per-op host launch cost).  Between Begin and End every op called on this thread for
     * (device_type, device_id) is recorded instead of run; End returns an executable graph
     * that Launch replays on the same stream, with the tensors captured at record time.
     * Only the AMD device supports capture.  Begin reserves the library scratch a captured
     * op may use (64 MiB beyond its fixed head, every attention launch fits; the environment
     * variable LLAISYS_GRAPH_WORKSPACE_BYTES sets another size); an op that would need more
     * during capture fails with a message.  A graph keeps the scratch it captured alive
     * until Destroy, so later eager ops that grow the scratch do not invalidate it. */
    typedef struct LlaisysGraph *llaisysGraph_t;
    __export void llaisysGraphBeginCapture(llaisysDeviceType_t, int);
    __export llaisysGraph_t llaisysGraphEndCapture(llaisysDeviceType_t, int);
    __export void llaisysGraphLaunch(llaisysGraph_t graph);
    __export void llaisysGraphDestroy(llaisysGraph_t graph);
}

#endif /* LLAISYS_RUNTIME_H */
