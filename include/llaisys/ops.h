/*
 * LLAISYS C ABI -- operators.
 *
 * The nine reference entry points keep their exact signatures (include/llaisys/ops.h:7-15;
 * shims src/llaisys/ops.cc:19-45).  All take pre-allocated tensors, return void and report
 * argument errors by printing to stderr and throwing, as the reference does
 * (src/utils/check.hpp:7-88).  On LLAISYS_DEVICE_AMD every op is one or two asynchronous
 * HIP kernel launches on the context stream (llaisysGetContextStream).
 *
 * Scope of this library: the bandwidth-bound per-layer ops and the attention that reads
 * their INT8 KV cache, the linear layers (dense, and over INT8 weights) and the strided
 * copy (rearrange) behind the tensor plumbing.  Ops on CPU tensors raise "Unsupported
 * device": this library has no CPU compute path.
 */
#ifndef LLAISYS_OPS_H
#define LLAISYS_OPS_H

#include "tensor.h"

__C {
    /* reference ops.h:7 -- c = a + b (half types add in f32 and round, add_cpu.cpp:7-17) */
    __export void llaisysAdd(llaisysTensor_t c, llaisysTensor_t a, llaisysTensor_t b);
    /* reference ops.h:8 -- flat argmax over all elements of vals; first maximum wins
     * (argmax_cpu.cpp:9-28); max_idx I32/I64, max_val dtype == vals dtype */
    __export void llaisysArgmax(llaisysTensor_t max_idx, llaisysTensor_t max_val,
                                llaisysTensor_t vals);
    /* reference ops.h:9 -- out[i,:] = weight[index[i],:]; index I32/I64 */
    __export void llaisysEmbedding(llaisysTensor_t out, llaisysTensor_t index,
                                   llaisysTensor_t weight);
    /* reference ops.h:10 -- out = in . weight^T + bias (src/ops/linear/op.cpp:10-42,
     * cpu/linear_cpu.cpp:11-41): in [.., K], weight [N, K], out [.., N], bias [N], one
     * dtype, f32 accumulation; a NULL or zero-element bias means no bias. */
    __export void llaisysLinear(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t weight,
                                llaisysTensor_t bias);
    /* reference ops.h:11 (a stub there, src/ops/rearrange/op.cpp:4-6) -- out[i] = in[i] for
     * every multi-index i: same shape, dtype and device, any strides, at most 8 dims;
     * bit-exact copy. */
    __export void llaisysRearrange(llaisysTensor_t out, llaisysTensor_t in);
    /* reference ops.h:12 -- per last-dim row: y = x * w / sqrt(mean(x^2) + eps) */
    __export void llaisysRmsNorm(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t weight,
                                 float eps);
    /* reference ops.h:13 -- rotate-half RoPE on [seq, n_heads, head_dim], pos_ids I64 */
    __export void llaisysROPE(llaisysTensor_t out, llaisysTensor_t in, llaisysTensor_t pos_ids,
                              float theta);
    /* reference ops.h:14 -- causal GQA attention (src/ops/self_attention/op.cpp:19-45,
     * cpu/self_attention_cpu.cpp:13-115): q [seq, nh, d], k [total, nkvh, d],
     * v [total, nkvh, dv], attn_val [seq, nh, dv], one dtype; query i sees keys
     * t <= total - seq + i; f32 softmax of (q . k) * scale. */
    __export void llaisysSelfAttention(llaisysTensor_t attn_val, llaisysTensor_t q,
                                       llaisysTensor_t k, llaisysTensor_t v, float scale);
    /* reference ops.h:15 -- out = up * gate / (1 + exp(-gate)) */
    __export void llaisysSwiGLU(llaisysTensor_t out, llaisysTensor_t gate, llaisysTensor_t up);

    /* ---- additive entry points (no reference kernel; same conventions) ---------------- */

    /* Fused residual add + rms_norm, replacing the reference decoder's llaisysAdd followed
     * by llaisysRmsNorm (src/models/qwen2/layer.hpp:60-71):
     *   residual_out = T(in + residual);  out = rms_norm(residual_out, weight, eps).
     * residual_out may be the same tensor as residual (in-place residual stream). */
    __export void llaisysAddRmsNorm(llaisysTensor_t out, llaisysTensor_t residual_out,
                                    llaisysTensor_t in, llaisysTensor_t residual,
                                    llaisysTensor_t weight, float eps);
    /* RoPE of q [seq, nh_q, head_dim] and k [seq, nh_k, head_dim] with the same pos_ids in
     * one launch: the reference decoder's two llaisysROPE calls on q and k
     * (src/models/qwen2/attention.hpp:54-55), each with the semantics of llaisysROPE; the
     * (cos, sin) table of a token is computed once for both. */
    __export void llaisysROPEQK(llaisysTensor_t q_out, llaisysTensor_t q_in, llaisysTensor_t k_out,
                                llaisysTensor_t k_in, llaisysTensor_t pos_ids, float theta);
    /* Fused RoPE + INT8 KV-cache append (quantize-on-append), one launch for the reference
     * decoder's rope(q), rope(k) and cache update (src/models/qwen2/attention.hpp:54-59,
     * :108-123) with an INT8 cache:
     *   q_out = llaisysROPE(q_in, pos_ids, theta)
     *   k_cache / k_scale rows pos .. pos+seq-1 = llaisysKVAppendInt8 of llaisysROPE(k_in)
     *   v_cache / v_scale rows pos .. pos+seq-1 = llaisysKVAppendInt8 of v_in
     * bit-identical to that composition; the rope'd k is never stored in its element type.
     * q [seq, nh_q, d]; k, v [seq, n_kvh, d]; caches [max_seq, n_kvh, d] I8 and
     * [max_seq, n_kvh] F32; pos + seq <= max_seq. */
    __export void llaisysROPEKVAppendInt8(llaisysTensor_t q_out, llaisysTensor_t q_in,
                                          llaisysTensor_t k_in, llaisysTensor_t v_in,
                                          llaisysTensor_t pos_ids, float theta,
                                          llaisysTensor_t k_cache, llaisysTensor_t k_scale,
                                          llaisysTensor_t v_cache, llaisysTensor_t v_scale,
                                          size_t pos);
    /* Row-wise argmax: the reference argmax (argmax_cpu.cpp:9-28) applied to each row of
     * vals [rows, cols]; max_idx [rows] I32/I64, max_val [rows] with the dtype of vals. */
    __export void llaisysArgmaxRows(llaisysTensor_t max_idx, llaisysTensor_t max_val,
                                    llaisysTensor_t vals);
    /* Symmetric INT8 absmax quantization per last-dim row of in [..., cols]
     * (F32/BF16/F16): scale[r] = max|x| / 127 (F32, shape in.shape[:-1]),
     * q = clamp(round_half_even(x / scale), -127, 127) (I8, shape of in); an all-zero row
     * gives scale 0 and codes 0; a NaN quotient gives code 0. */
    __export void llaisysQuantizeInt8(llaisysTensor_t q, llaisysTensor_t scale,
                                      llaisysTensor_t in);
    /* out = T(float(q) * scale[row]) for q [..., cols] I8 and scale [...] F32. */
    __export void llaisysDequantizeInt8(llaisysTensor_t out, llaisysTensor_t q,
                                        llaisysTensor_t scale);
    /* INT8 KV-cache append, replacing the f32 row copy of the reference decoder's cache
     * update (src/models/qwen2/attention.hpp:108-123): quantizes kv [n_tok, n_kvh, head_dim]
     * per (token, head) row with the rule of llaisysQuantizeInt8 and writes the codes to
     * cache_q [max_seq, n_kvh, head_dim] (I8) rows pos .. pos+n_tok-1 and the scales to
     * cache_scale [max_seq, n_kvh] (F32).  Requires pos + n_tok <= max_seq. */
    __export void llaisysKVAppendInt8(llaisysTensor_t cache_q, llaisysTensor_t cache_scale,
                                      llaisysTensor_t kv, size_t pos);
    /* The k and v cache appends of one decoder step (the reference updates both caches,
     * src/models/qwen2/attention.hpp:108-123) in one launch: equal to
     * llaisysKVAppendInt8(k_cache, k_scale, k, pos) followed by
     * llaisysKVAppendInt8(v_cache, v_scale, v, pos); k and v share dtype and head_dim. */
    __export void llaisysKVAppendInt8Pair(llaisysTensor_t k_cache, llaisysTensor_t k_scale,
                                          llaisysTensor_t v_cache, llaisysTensor_t v_scale,
                                          llaisysTensor_t k, llaisysTensor_t v, size_t pos);
    /* Two dequantizations in one launch (the k and v slices of an INT8 cache read for
     * attention, src/models/qwen2/attention.hpp:70-73): equal to
     * llaisysDequantizeInt8(out0, q0, scale0) followed by llaisysDequantizeInt8(out1, q1,
     * scale1); the outputs share dtype and last dimension. */
    __export void llaisysDequantizeInt8Pair(llaisysTensor_t out0, llaisysTensor_t q0,
                                            llaisysTensor_t scale0, llaisysTensor_t out1,
                                            llaisysTensor_t q1, llaisysTensor_t scale1);
    /* llaisysSelfAttention over an INT8 KV cache (the reference decoder's attention over
     * its cache slice, src/models/qwen2/attention.hpp:70-73, with the cache of
     * llaisysKVAppendInt8): k_codes [total, nkvh, d] and v_codes [total, nkvh, dv] I8,
     * k_scale / v_scale [total, nkvh] F32.  Equal to llaisysDequantizeInt8 of both caches
     * into q's dtype followed by llaisysSelfAttention; the caches are read as codes. */
    __export void llaisysSelfAttentionInt8KV(llaisysTensor_t attn_val, llaisysTensor_t q,
                                             llaisysTensor_t k_codes, llaisysTensor_t k_scale,
                                             llaisysTensor_t v_codes, llaisysTensor_t v_scale,
                                             float scale);
    /* No counterpart in the reference: llaisysSelfAttentionInt8KV for callers that cannot
     * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
     * that forbid hipMalloc).  Same arguments, checks and result bits as
     * llaisysSelfAttentionInt8KV, but its workspace is a file-scope device scratch of 24 MiB
     * per GPU (held until the process ends) instead of the library workspace, and it calls
     * no allocator.  Decode-shaped calls put their split partials there; one whose partials
     * exceed the scratch -- queries x q heads x (head_dim + 2) x 4 KiB, e.g. more than 47
     * query-heads at head_dim 128 -- fails with a message.  A bf16 prefill (16 or more
     * queries, head_dim 128) dequantizes the caches into the scratch when they fit and
     * otherwise converts the codes inside its kernel.  Calls on one GPU share the scratch:
     * calls that overlap (other threads or streams) race. */
    __export void llaisysSelfAttentionInt8KVNoAlloc(llaisysTensor_t attn_val, llaisysTensor_t q,
                                                    llaisysTensor_t k_codes, llaisysTensor_t k_scale,
                                                    llaisysTensor_t v_codes, llaisysTensor_t v_scale,
                                                    float scale);
    /* Device-side dtype conversion: out[i] = cast<out dtype>(in[i]) with the reference's
     * cast<To>(From) (src/utils/types.hpp:116-139: through f32; f32 -> bf16 rounds half to
     * even by "+0x7FFF + lsb" with no NaN case, f32 -> f16 truncates, widening is exact,
     * equal types copy the bits).  out and in: same shape, contiguous, F32 / BF16 / F16,
     * same device.  It replaces the reference loader's host upcast of bf16 / f16 weights to
     * f32 (python/llaisys/models/qwen2.py:118-120): weights stay bf16 in HBM, uploaded as
     * bf16 bits, or as f32 and cast here. */
    __export void llaisysCast(llaisysTensor_t out, llaisysTensor_t in);
    /* llaisysLinear with INT8 weights (no reference counterpart; the decoder's projections,
     * src/models/qwen2/components.hpp:114, with weights quantized by llaisysQuantizeInt8 per output row):
     * w_codes [N, K] I8, w_scale [N] F32, in / out / bias of one float dtype;
     * out[m][n] = T(w_scale[n] * sum_k in[m][k] * code[n][k] + bias[n]), f32 accumulation.
     * Bias NULL or zero-element means no bias. */
    __export void llaisysLinearW8A16(llaisysTensor_t out, llaisysTensor_t in,
                                     llaisysTensor_t w_codes, llaisysTensor_t w_scale,
                                     llaisysTensor_t bias);
    /* rms_norm fused ahead of a linear, optionally with swiglu after it (no reference
     * counterpart; the decoder's input_layernorm -> q/k/v projections and add ->
     * post_attention_layernorm -> gate / up -> swiglu, src/models/qwen2/layer.hpp:51-53,
     * :66-71, src/models/qwen2/mlp.hpp:22-33).  h = residual ? in + residual : in (rounded as
     * llaisysAdd; stored to residual_out, which must not overlap in or residual; both NULL for
     * no add); xn = llaisysRmsNorm(h, norm_weight, eps); y = llaisysLinear(xn, weight, bias), or
     * llaisysLinearW8A16 when weight_scale is non-NULL; out = y, or with swiglu != 0 out[m][n] =
     * swiglu(gate = y[m][n], up = y[m][n + Nw/2]) for a weight of Nw rows (out [rows, Nw/2]).
     * bias NULL or zero-element means no bias.  One launch for one row; other row counts run
     * the ops one after another. */
    __export void llaisysRmsNormLinear(llaisysTensor_t out, llaisysTensor_t residual_out,
                                       llaisysTensor_t in, llaisysTensor_t residual,
                                       llaisysTensor_t norm_weight, float eps,
                                       llaisysTensor_t weight, llaisysTensor_t weight_scale,
                                       llaisysTensor_t bias, uint8_t swiglu);
    /* Random sampling after argmax (no reference kernel: README.md:397-399 asks for a random
     * sample operator with temperature, top-k and top-p; python/llaisys/models/qwen2.py:216-218
     * takes the three and ignores them).  logits [V] or [rows, V] (F32 / BF16 / F16), out_idx
     * I64 / I32 with one index per row.  temperature <= 0 or top_k == 1: the row's argmax
     * (first maximum).  Otherwise top_k in [2, 1024] (clamped to V): z = x * (1/T); the
     * top_k largest z (ties by lower index); weights w = floor(2^31 * 2^((z - zmax) log2 e))
     * from a fixed exp2 polynomial; top_p < 1 keeps the shortest (z desc, index asc) prefix
     * whose weight sum reaches floor(top_p * W) (at least one token); the token is drawn by
     * inverse CDF over that prefix with the uniform (splitmix64(seed + row) >> 40) / 2^24.
     * Deterministic: equal inputs and seed give equal indices. */
    __export void llaisysRandomSample(llaisysTensor_t out_idx, llaisysTensor_t logits,
                                      float temperature, int64_t top_k, float top_p,
                                      uint64_t seed);
}

#endif /* LLAISYS_OPS_H */
