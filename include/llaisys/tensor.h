/*
 * LLAISYS C ABI -- tensor handles.
 *
 * Same entry points and signatures as the reference's include/llaisys/tensor.h:7-65
 * (implementation there: src/llaisys/tensor.cc:7-118).  A tensor is a view (shape,
 * strides in elements, byte offset) over a shared storage block on one device.
 * Ops never allocate their outputs: callers create every tensor they pass.
 */
#ifndef LLAISYS_TENSOR_H
#define LLAISYS_TENSOR_H

#include "../llaisys.h"

__C {
    typedef struct LlaisysTensor *llaisysTensor_t;

    /* reference tensor.h:9-14 -- contiguous tensor; CPU tensors are pinned host memory
     * while a GPU runtime is current. */
    __export llaisysTensor_t tensorCreate(size_t *shape, size_t ndim, llaisysDataType_t dtype,
                                          llaisysDeviceType_t device_type, int device_id);
    /* reference tensor.h:16-17 */
    __export void tensorDestroy(llaisysTensor_t tensor);
    /* reference tensor.h:19-20 -- device pointer for GPU tensors */
    __export void *tensorGetData(llaisysTensor_t tensor);
    /* reference tensor.h:22-23 */
    __export size_t tensorGetNdim(llaisysTensor_t tensor);
    /* reference tensor.h:25-27 */
    __export void tensorGetShape(llaisysTensor_t tensor, size_t *shape);
    /* reference tensor.h:29-31 */
    __export void tensorGetStrides(llaisysTensor_t tensor, ptrdiff_t *strides);
    /* reference tensor.h:33-34 */
    __export llaisysDataType_t tensorGetDataType(llaisysTensor_t tensor);
    /* reference tensor.h:36-37 */
    __export llaisysDeviceType_t tensorGetDeviceType(llaisysTensor_t tensor);
    /* reference tensor.h:39-40 */
    __export int tensorGetDeviceId(llaisysTensor_t tensor);
    /* reference tensor.h:42-43 */
    __export void tensorDebug(llaisysTensor_t tensor);
    /* reference tensor.h:45-46 */
    __export uint8_t tensorIsContiguous(llaisysTensor_t tensor);
    /* reference tensor.h:48-50 -- synchronous copy of numel*elemsize bytes from host */
    __export void tensorLoad(llaisysTensor_t tensor, const void *data);
    /* reference tensor.h:52-55 */
    __export llaisysTensor_t tensorView(llaisysTensor_t tensor, size_t *shape, size_t ndim);
    /* reference tensor.h:57-59 */
    __export llaisysTensor_t tensorPermute(llaisysTensor_t tensor, size_t *order);
    /* reference tensor.h:61-64 -- [start, end) along dim */
    __export llaisysTensor_t tensorSlice(llaisysTensor_t tensor, size_t dim, size_t start,
                                         size_t end);
    /* reference Tensor::contiguous (src/tensor/tensor.hpp:55, a stub at tensor.cpp:344-347;
     * no C entry point there) -- the tensor itself when contiguous (shared storage), else a
     * contiguous copy on the same device (llaisysRearrange on AMD devices) */
    __export llaisysTensor_t tensorContiguous(llaisysTensor_t tensor);
    /* reference Tensor::reshape (tensor.hpp:56, a stub at tensor.cpp:349-352) -- a view
     * when contiguous, else a view of tensorContiguous */
    __export llaisysTensor_t tensorReshape(llaisysTensor_t tensor, size_t *shape, size_t ndim);
    /* reference Tensor::to (tensor.hpp:57, a stub at tensor.cpp:354-357) -- the tensor itself
     * when already there, else a contiguous copy on (device_type, device); device < 0 keeps
     * the id for the same device type, else 0.  Synchronous. */
    __export llaisysTensor_t tensorTo(llaisysTensor_t tensor, llaisysDeviceType_t device_type,
                                      int device);
}

#endif /* LLAISYS_TENSOR_H */
