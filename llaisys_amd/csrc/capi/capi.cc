// extern "C" entry points of libllaisys.so.
//
// Same shape as the reference shims (src/llaisys/ops.cc:17-46, tensor.cc:6-119,
// runtime.cc:11-19): unwrap the handle, call C++, no try/catch -- an error prints and
// throws, which through ctypes ends the process, as with the reference library.
#include "llaisys/models/qwen2.h"
#include "llaisys/ops.h"
#include "llaisys/runtime.h"
#include "llaisys/tensor.h"

#include "../core/core.hpp"
#include "../device/runtime_api.hpp"
#include "../ops/ops.hpp"
#include "../tensor/tensor.hpp"
#include "../utils/check.hpp"

#include <algorithm>
#include <vector>

struct LlaisysTensor {
    llaisys::tensor_t tensor;
};

namespace {
llaisysTensor_t wrap(llaisys::tensor_t t) { return new LlaisysTensor{std::move(t)}; }
} // namespace

__C {
    // ---- runtime (reference src/llaisys/runtime.cc:11-19) ------------------------------
    void llaisysSetContextRuntime(llaisysDeviceType_t type, int id) {
        llaisys::core::context().setDevice(type, id);
    }

    const LlaisysRuntimeAPI *llaisysGetRuntimeAPI(llaisysDeviceType_t type) {
        return llaisys::device::getRuntimeAPI(type);
    }

    llaisysStream_t llaisysGetContextStream(llaisysDeviceType_t type, int id) {
        auto &ctx = llaisys::core::context();
        ctx.setDevice(type, id);
        return ctx.runtime().stream();
    }

    int llaisysTakeDeviceError(llaisysDeviceType_t type, int id) {
        if (type != LLAISYS_DEVICE_AMD) return 0;
        auto &ctx = llaisys::core::context();
        ctx.setDevice(type, id);
        return llaisys::device::amd::takeError(ctx.runtime().stream());
    }

    void llaisysGraphBeginCapture(llaisysDeviceType_t type, int id) {
        if (type != LLAISYS_DEVICE_AMD) EXCEPTION_UNSUPPORTED_DEVICE;
        auto &ctx = llaisys::core::context();
        ctx.setDevice(type, id);
        llaisys::device::amd::beginCapture(id, ctx.runtime().stream());
    }

    llaisysGraph_t llaisysGraphEndCapture(llaisysDeviceType_t type, int id) {
        if (type != LLAISYS_DEVICE_AMD) EXCEPTION_UNSUPPORTED_DEVICE;
        auto &ctx = llaisys::core::context();
        ctx.setDevice(type, id);
        return llaisys::device::amd::endCapture(id, ctx.runtime().stream());
    }

    void llaisysGraphLaunch(llaisysGraph_t g) { llaisys::device::amd::launchGraph(g); }

    void llaisysGraphDestroy(llaisysGraph_t g) { llaisys::device::amd::destroyGraph(g); }

    // ---- tensors (reference src/llaisys/tensor.cc:7-118) -------------------------------
    llaisysTensor_t tensorCreate(size_t * shape, size_t ndim, llaisysDataType_t dtype,
                                 llaisysDeviceType_t device_type, int device_id) {
        std::vector<size_t> dims(shape, shape + ndim);
        return wrap(llaisys::Tensor::create(dims, dtype, device_type, device_id));
    }

    void tensorDestroy(llaisysTensor_t t) { delete t; }

    void *tensorGetData(llaisysTensor_t t) { return t->tensor->data(); }

    size_t tensorGetNdim(llaisysTensor_t t) { return t->tensor->ndim(); }

    void tensorGetShape(llaisysTensor_t t, size_t * shape) {
        std::copy(t->tensor->shape().begin(), t->tensor->shape().end(), shape);
    }

    void tensorGetStrides(llaisysTensor_t t, ptrdiff_t * strides) {
        std::copy(t->tensor->strides().begin(), t->tensor->strides().end(), strides);
    }

    llaisysDataType_t tensorGetDataType(llaisysTensor_t t) { return t->tensor->dtype(); }

    llaisysDeviceType_t tensorGetDeviceType(llaisysTensor_t t) { return t->tensor->deviceType(); }

    int tensorGetDeviceId(llaisysTensor_t t) { return t->tensor->deviceId(); }

    void tensorDebug(llaisysTensor_t t) { t->tensor->debug(); }

    uint8_t tensorIsContiguous(llaisysTensor_t t) { return uint8_t(t->tensor->isContiguous()); }

    void tensorLoad(llaisysTensor_t t, const void *data) { t->tensor->load(data); }

    llaisysTensor_t tensorView(llaisysTensor_t t, size_t * shape, size_t ndim) {
        return wrap(t->tensor->view(std::vector<size_t>(shape, shape + ndim)));
    }

    llaisysTensor_t tensorPermute(llaisysTensor_t t, size_t * order) {
        return wrap(t->tensor->permute(std::vector<size_t>(order, order + t->tensor->ndim())));
    }

    llaisysTensor_t tensorSlice(llaisysTensor_t t, size_t dim, size_t start, size_t end) {
        return wrap(t->tensor->slice(dim, start, end));
    }

    // reference src/tensor/tensor.hpp:55-57 (C++ only there)
    llaisysTensor_t tensorContiguous(llaisysTensor_t t) { return wrap(t->tensor->contiguous()); }

    llaisysTensor_t tensorReshape(llaisysTensor_t t, size_t * shape, size_t ndim) {
        return wrap(t->tensor->reshape(std::vector<size_t>(shape, shape + ndim)));
    }

    llaisysTensor_t tensorTo(llaisysTensor_t t, llaisysDeviceType_t device_type, int device) {
        return wrap(t->tensor->to(device_type, device));
    }

    // ---- ops (reference src/llaisys/ops.cc:19-45) --------------------------------------
    void llaisysAdd(llaisysTensor_t c, llaisysTensor_t a, llaisysTensor_t b) {
        llaisys::ops::add(c->tensor, a->tensor, b->tensor);
    }
    void llaisysArgmax(llaisysTensor_t max_idx, llaisysTensor_t max_val, llaisysTensor_t vals) {
        llaisys::ops::argmax(max_idx->tensor, max_val->tensor, vals->tensor);
    }
    void llaisysEmbedding(llaisysTensor_t out, llaisysTensor_t index, llaisysTensor_t weight) {
        llaisys::ops::embedding(out->tensor, index->tensor, weight->tensor);
    }
    void llaisysLinear(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t weight,
                       llaisysTensor_t bias) {
        llaisys::ops::linear(out->tensor, in->tensor, weight->tensor, bias ? bias->tensor : nullptr);
    }
    void llaisysRearrange(llaisysTensor_t out, llaisysTensor_t in) {
        llaisys::ops::rearrange(out->tensor, in->tensor);
    }
    void llaisysRmsNorm(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t weight, float eps) {
        llaisys::ops::rmsNorm(out->tensor, in->tensor, weight->tensor, eps);
    }
    void llaisysROPE(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t pos_ids, float theta) {
        llaisys::ops::rope(out->tensor, in->tensor, pos_ids->tensor, theta);
    }
    void llaisysSelfAttention(llaisysTensor_t attn_val, llaisysTensor_t q, llaisysTensor_t k,
                              llaisysTensor_t v, float scale) {
        llaisys::ops::selfAttention(attn_val->tensor, q->tensor, k->tensor, v->tensor, scale);
    }
    void llaisysSwiGLU(llaisysTensor_t out, llaisysTensor_t gate, llaisysTensor_t up) {
        llaisys::ops::swiglu(out->tensor, gate->tensor, up->tensor);
    }
    void llaisysAddRmsNorm(llaisysTensor_t out, llaisysTensor_t residual_out, llaisysTensor_t in,
                           llaisysTensor_t residual, llaisysTensor_t weight, float eps) {
        llaisys::ops::addRmsNorm(out->tensor, residual_out->tensor, in->tensor, residual->tensor,
                                 weight->tensor, eps);
    }
    void llaisysROPEQK(llaisysTensor_t q_out, llaisysTensor_t q_in, llaisysTensor_t k_out,
                       llaisysTensor_t k_in, llaisysTensor_t pos_ids, float theta) {
        llaisys::ops::ropeQK(q_out->tensor, q_in->tensor, k_out->tensor, k_in->tensor,
                             pos_ids->tensor, theta);
    }
    void llaisysROPEKVAppendInt8(llaisysTensor_t q_out, llaisysTensor_t q_in, llaisysTensor_t k_in,
                                 llaisysTensor_t v_in, llaisysTensor_t pos_ids, float theta,
                                 llaisysTensor_t k_cache, llaisysTensor_t k_scale,
                                 llaisysTensor_t v_cache, llaisysTensor_t v_scale, size_t pos) {
        llaisys::ops::ropeKvAppendInt8(q_out->tensor, q_in->tensor, k_in->tensor, v_in->tensor,
                                       pos_ids->tensor, theta, k_cache->tensor, k_scale->tensor,
                                       v_cache->tensor, v_scale->tensor, pos);
    }
    void llaisysArgmaxRows(llaisysTensor_t max_idx, llaisysTensor_t max_val, llaisysTensor_t vals) {
        llaisys::ops::argmaxRows(max_idx->tensor, max_val->tensor, vals->tensor);
    }
    void llaisysQuantizeInt8(llaisysTensor_t q, llaisysTensor_t scale, llaisysTensor_t in) {
        llaisys::ops::quantizeInt8(q->tensor, scale->tensor, in->tensor);
    }
    void llaisysDequantizeInt8(llaisysTensor_t out, llaisysTensor_t q, llaisysTensor_t scale) {
        llaisys::ops::dequantizeInt8(out->tensor, q->tensor, scale->tensor);
    }
    void llaisysKVAppendInt8(llaisysTensor_t cache_q, llaisysTensor_t cache_scale,
                             llaisysTensor_t kv, size_t pos) {
        llaisys::ops::kvAppendInt8(cache_q->tensor, cache_scale->tensor, kv->tensor, pos);
    }
    void llaisysKVAppendInt8Pair(llaisysTensor_t k_cache, llaisysTensor_t k_scale,
                                 llaisysTensor_t v_cache, llaisysTensor_t v_scale,
                                 llaisysTensor_t k, llaisysTensor_t v, size_t pos) {
        llaisys::ops::kvAppendInt8Pair(k_cache->tensor, k_scale->tensor, v_cache->tensor,
                                       v_scale->tensor, k->tensor, v->tensor, pos);
    }
    void llaisysSelfAttentionInt8KV(llaisysTensor_t attn_val, llaisysTensor_t q,
                                    llaisysTensor_t k_codes, llaisysTensor_t k_scale,
                                    llaisysTensor_t v_codes, llaisysTensor_t v_scale, float scale) {
        llaisys::ops::selfAttentionInt8KV(attn_val->tensor, q->tensor, k_codes->tensor,
                                          k_scale->tensor, v_codes->tensor, v_scale->tensor, scale);
    }
    void llaisysSelfAttentionInt8KVNoAlloc(llaisysTensor_t attn_val, llaisysTensor_t q,
                                           llaisysTensor_t k_codes, llaisysTensor_t k_scale,
                                           llaisysTensor_t v_codes, llaisysTensor_t v_scale,
                                           float scale) {
        llaisys::ops::selfAttentionInt8KVNoAlloc(attn_val->tensor, q->tensor, k_codes->tensor,
                                                 k_scale->tensor, v_codes->tensor, v_scale->tensor,
                                                 scale);
    }
    void llaisysCast(llaisysTensor_t out, llaisysTensor_t in) {
        llaisys::ops::cast(out->tensor, in->tensor);
    }
    void llaisysDequantizeInt8Pair(llaisysTensor_t out0, llaisysTensor_t q0, llaisysTensor_t scale0,
                                   llaisysTensor_t out1, llaisysTensor_t q1, llaisysTensor_t scale1) {
        llaisys::ops::dequantizeInt8Pair(out0->tensor, q0->tensor, scale0->tensor, out1->tensor,
                                         q1->tensor, scale1->tensor);
    }

    void llaisysLinearW8A16(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t w_codes,
                            llaisysTensor_t w_scale, llaisysTensor_t bias) {
        llaisys::ops::linearW8A16(out->tensor, in->tensor, w_codes->tensor, w_scale->tensor,
                                  bias ? bias->tensor : nullptr);
    }

    void llaisysRmsNormLinear(llaisysTensor_t out, llaisysTensor_t residual_out, llaisysTensor_t in,
                              llaisysTensor_t residual, llaisysTensor_t norm_weight, float eps,
                              llaisysTensor_t weight, llaisysTensor_t weight_scale,
                              llaisysTensor_t bias, uint8_t swiglu) {
        const auto opt = [](llaisysTensor_t t) { return t ? t->tensor : nullptr; };
        llaisys::ops::rmsNormLinear(out->tensor, opt(residual_out), in->tensor, opt(residual),
                                    norm_weight->tensor, eps, weight->tensor, opt(weight_scale),
                                    opt(bias), swiglu != 0);
    }

    void llaisysRandomSample(llaisysTensor_t out_idx, llaisysTensor_t logits, float temperature,
                             int64_t top_k, float top_p, uint64_t seed) {
        llaisys::ops::randomSample(out_idx->tensor, logits->tensor, temperature, top_k, top_p, seed);
    }

    // ---- model API: out of scope, exported so the reference ctypes loader binds --------
    struct LlaisysQwen2Model *llaisysQwen2ModelCreate(const struct LlaisysQwen2Meta *,
                                                      llaisysDeviceType_t, int *, int) {
        TO_BE_IMPLEMENTED();
    }
    void llaisysQwen2ModelDestroy(struct LlaisysQwen2Model *) { TO_BE_IMPLEMENTED(); }
    struct LlaisysQwen2Weights *llaisysQwen2ModelWeights(struct LlaisysQwen2Model *) {
        TO_BE_IMPLEMENTED();
    }
    int64_t llaisysQwen2ModelInfer(struct LlaisysQwen2Model *, int64_t *, size_t) {
        TO_BE_IMPLEMENTED();
    }
}
