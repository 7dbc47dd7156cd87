// Operator dispatchers: argument checks, device selection, kernel launch.
#pragma once

#include "../tensor/tensor.hpp"

namespace llaisys::ops {

void add(tensor_t c, tensor_t a, tensor_t b);
void argmax(tensor_t max_idx, tensor_t max_val, tensor_t vals);
void argmaxRows(tensor_t max_idx, tensor_t max_val, tensor_t vals);
void embedding(tensor_t out, tensor_t index, tensor_t weight);
void rmsNorm(tensor_t out, tensor_t in, tensor_t weight, float eps);
void addRmsNorm(tensor_t out, tensor_t residual_out, tensor_t in, tensor_t residual,
                tensor_t weight, float eps);
void rope(tensor_t out, tensor_t in, tensor_t pos_ids, float theta);
void ropeQK(tensor_t q_out, tensor_t q_in, tensor_t k_out, tensor_t k_in, tensor_t pos_ids,
            float theta);
void cast(tensor_t out, tensor_t in);
void swiglu(tensor_t out, tensor_t gate, tensor_t up);
void quantizeInt8(tensor_t q, tensor_t scale, tensor_t in);
void dequantizeInt8(tensor_t out, tensor_t q, tensor_t scale);
void kvAppendInt8(tensor_t cache_q, tensor_t cache_scale, tensor_t kv, size_t pos);
void kvAppendInt8Pair(tensor_t k_cache, tensor_t k_scale, tensor_t v_cache, tensor_t v_scale,
                      tensor_t k, tensor_t v, size_t pos);
void selfAttention(tensor_t attn_val, tensor_t q, tensor_t k, tensor_t v, float scale);
void selfAttentionInt8KV(tensor_t attn_val, tensor_t q, tensor_t k_codes, tensor_t k_scale,
                         tensor_t v_codes, tensor_t v_scale, float scale);
void selfAttentionInt8KVNoAlloc(tensor_t attn_val, tensor_t q, tensor_t k_codes, tensor_t k_scale,
                                tensor_t v_codes, tensor_t v_scale, float scale);
void dequantizeInt8Pair(tensor_t out0, tensor_t q0, tensor_t scale0, tensor_t out1, tensor_t q1,
                        tensor_t scale1);
void linear(tensor_t out, tensor_t in, tensor_t weight, tensor_t bias);
void rearrange(tensor_t out, tensor_t in);
void randomSample(tensor_t out_idx, tensor_t logits, float temperature, int64_t top_k,
                  float top_p, uint64_t seed);
void linearW8A16(tensor_t out, tensor_t in, tensor_t w_codes, tensor_t w_scale, tensor_t bias);
void rmsNormLinear(tensor_t out, tensor_t residual_out, tensor_t in, tensor_t residual,
                   tensor_t norm_weight, float eps, tensor_t weight, tensor_t weight_scale,
                   tensor_t bias, bool swiglu);
void ropeKvAppendInt8(tensor_t q_out, tensor_t q_in, tensor_t k_in, tensor_t v_in,
                      tensor_t pos_ids, float theta, tensor_t k_cache, tensor_t k_scale,
                      tensor_t v_cache, tensor_t v_scale, size_t pos);

} // namespace llaisys::ops
