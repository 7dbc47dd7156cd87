/*
 * LLAISYS C ABI -- Qwen2 model entry points (OUT OF SCOPE for this library).
 *
 * Declared with the reference's signatures (include/llaisys/models/qwen2.h:7-40) only so
 * that the reference's ctypes loader (python/llaisys/libllaisys/qwen2.py:66-91), which
 * binds these four symbols at import, also loads libllaisys.so from llaisys_amd.  Each
 * one prints "[ERROR] Unimplemented function" and throws: the model driver is not part
 * of this op library.
 */
#ifndef LLAISYS_MODELS_QWEN2_H
#define LLAISYS_MODELS_QWEN2_H

#include "../tensor.h"

__C {
    struct LlaisysQwen2Meta {
        llaisysDataType_t dtype;
        size_t nlayer, hs, nh, nkvh, dh, di, maxseq, voc;
        float epsilon, theta;
        int64_t end_token;
    };

    struct LlaisysQwen2Weights {
        llaisysTensor_t in_embed;
        llaisysTensor_t out_embed;
        llaisysTensor_t out_norm_w;
        llaisysTensor_t *attn_norm_w;
        llaisysTensor_t *attn_q_w;
        llaisysTensor_t *attn_q_b;
        llaisysTensor_t *attn_k_w;
        llaisysTensor_t *attn_k_b;
        llaisysTensor_t *attn_v_w;
        llaisysTensor_t *attn_v_b;
        llaisysTensor_t *attn_o_w;
        llaisysTensor_t *mlp_norm_w;
        llaisysTensor_t *mlp_gate_w;
        llaisysTensor_t *mlp_up_w;
        llaisysTensor_t *mlp_down_w;
    };

    struct LlaisysQwen2Model;

    __export struct LlaisysQwen2Model *llaisysQwen2ModelCreate(const struct LlaisysQwen2Meta *meta,
                                                               llaisysDeviceType_t device,
                                                               int *device_ids, int ndevice);
    __export void llaisysQwen2ModelDestroy(struct LlaisysQwen2Model *model);
    __export struct LlaisysQwen2Weights *llaisysQwen2ModelWeights(struct LlaisysQwen2Model *model);
    __export int64_t llaisysQwen2ModelInfer(struct LlaisysQwen2Model *model, int64_t *token_ids,
                                            size_t ntoken);
}

#endif /* LLAISYS_MODELS_QWEN2_H */
