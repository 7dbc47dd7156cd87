// Operator dispatchers.
//
// Each op runs the checks of the reference dispatcher it replaces (cited per op), then
// makes the tensors' device current and launches the gfx950 kernel on that device's
// context stream.  Where the reference leaves an output size unchecked (rms_norm, swiglu
// dtypes, embedding output, argmax outputs) a check is added here: on a GPU an undersized
// output would be an out-of-bounds write, not a CPU heap overrun.  Only the AMD device
// computes; CPU tensors raise "Unsupported device" (the reference CPU kernels are the
// test oracle, not a fallback of this library).
#include "ops.hpp"

#include "../device/runtime_api.hpp"
#include "../kernels/launch.hpp"
#include "../utils/check.hpp"
#include "../utils/types.hpp"

namespace llaisys::ops {

namespace {

bool isFloat(llaisysDataType_t dt) {
    return dt == LLAISYS_DTYPE_F32 || dt == LLAISYS_DTYPE_BF16 || dt == LLAISYS_DTYPE_F16;
}

void requireFloat(llaisysDataType_t dt) {
    if (!isFloat(dt)) EXCEPTION_UNSUPPORTED_DATATYPE(dt);
}

// Makes the device of `t` current and returns its stream; only the AMD device computes.
hipStream_t streamFor(const tensor_t &t) {
    if (t->deviceType() != LLAISYS_DEVICE_AMD) EXCEPTION_UNSUPPORTED_DEVICE;
    auto &ctx = core::context();
    ctx.setDevice(t->deviceType(), t->deviceId());
    return static_cast<hipStream_t>(ctx.runtime().stream());
}

// Reports a failed launch (bad configuration, no code object for this GPU) at the call.
void launched(const char *op) { device::amd::check(hipGetLastError(), op); }

size_t lastDim(const tensor_t &t) {
    ASSERT(t->ndim() >= 1, "tensor must have at least one dimension");
    return t->shape().back();
}

} // namespace

// reference src/ops/add/op.cpp:11-38
void add(tensor_t c, tensor_t a, tensor_t b) {
    CHECK_SAME_DEVICE(c, a, b);
    CHECK_SAME_SHAPE(c->shape(), a->shape(), b->shape());
    CHECK_SAME_DTYPE(c->dtype(), a->dtype(), b->dtype());
    ASSERT(c->isContiguous() && a->isContiguous() && b->isContiguous(),
           "Add: all tensors must be contiguous.");
    requireFloat(c->dtype());
    auto s = streamFor(c);
    kernels::add(c->data(), a->data(), b->data(), c->numel(), c->dtype(), s);
    launched("add");
}

// reference src/ops/argmax/op.cpp:13-40 (flat over every element of vals)
void argmax(tensor_t max_idx, tensor_t max_val, tensor_t vals) {
    CHECK_SAME_DEVICE(max_idx, max_val, vals);
    CHECK_SAME_DTYPE(max_val->dtype(), vals->dtype());
    ASSERT(max_idx->isContiguous() && max_val->isContiguous() && vals->isContiguous(),
           "Argmax: input tensor must be contiguous.");
    ASSERT(max_idx->dtype() == LLAISYS_DTYPE_I32 || max_idx->dtype() == LLAISYS_DTYPE_I64,
           "Argmax: max_idx must be INT32 or INT64");
    requireFloat(vals->dtype());
    ASSERT(max_idx->numel() >= 1 && max_val->numel() >= 1, "Argmax: outputs must hold one element");
    auto s = streamFor(vals);
    const size_t n = vals->numel();
    if (n == 0) return;
    void *ws = device::amd::workspace(vals->deviceId(), kernels::argmaxWorkspaceBytes(n, vals->dtype()));
    kernels::argmax(max_idx->data(), max_idx->dtype() == LLAISYS_DTYPE_I64, max_val->data(),
                    vals->data(), n, vals->dtype(), ws, s);
    launched("argmax");
}

// Row-wise variant: the reference argmax applied to each row of vals [rows, cols].
void argmaxRows(tensor_t max_idx, tensor_t max_val, tensor_t vals) {
    CHECK_SAME_DEVICE(max_idx, max_val, vals);
    CHECK_SAME_DTYPE(max_val->dtype(), vals->dtype());
    ASSERT(max_idx->isContiguous() && max_val->isContiguous() && vals->isContiguous(),
           "ArgmaxRows: tensors must be contiguous.");
    ASSERT(max_idx->dtype() == LLAISYS_DTYPE_I32 || max_idx->dtype() == LLAISYS_DTYPE_I64,
           "ArgmaxRows: max_idx must be INT32 or INT64");
    requireFloat(vals->dtype());
    ASSERT(vals->ndim() == 2, "ArgmaxRows: vals must be 2-D [rows, cols]");
    const size_t rows = vals->shape()[0], cols = vals->shape()[1];
    ASSERT(max_idx->numel() == rows && max_val->numel() == rows,
           "ArgmaxRows: outputs must hold one element per row");
    auto s = streamFor(vals);
    kernels::argmaxRows(max_idx->data(), max_idx->dtype() == LLAISYS_DTYPE_I64, max_val->data(),
                        vals->data(), rows, cols, vals->dtype(), s);
    launched("argmaxRows");
}

// reference src/ops/embedding/op.cpp:15-46
void embedding(tensor_t out, tensor_t index, tensor_t weight) {
    CHECK_SAME_DEVICE(out, index, weight);
    ASSERT(out->isContiguous() && index->isContiguous() && weight->isContiguous(),
           "Embedding inputs must be contiguous");
    CHECK_SAME_DTYPE(out->dtype(), weight->dtype());
    ASSERT(index->dtype() == LLAISYS_DTYPE_I32 || index->dtype() == LLAISYS_DTYPE_I64,
           "Embedding parameter index data type must be INT32 or INT64");
    ASSERT(weight->ndim() == 2, "Embedding weight must be 2-D [vocab, dim]");
    const size_t n = index->numel();
    const size_t vocab = weight->shape()[0], dim = weight->shape()[1];
    ASSERT(out->numel() == n * dim, "Embedding output must hold index.numel() rows of dim");
    auto s = streamFor(weight);
    int *err = device::amd::errorWord(weight->deviceId());
    kernels::embedding(out->data(), index->data(), index->dtype() == LLAISYS_DTYPE_I64, n,
                       weight->data(), vocab, dim * weight->elementSize(), err, s);
    launched("embedding");
}

// reference src/ops/rms_norm/op.cpp:9-42
void rmsNorm(tensor_t out, tensor_t in, tensor_t weight, float eps) {
    CHECK_SAME_DEVICE(out, in, weight);
    const size_t cols = lastDim(in);
    ASSERT(weight->ndim() == 1, "RMSNorm weight must be 1D");
    ASSERT(weight->shape()[0] == cols, "RMSNorm weight shape mismatch");
    CHECK_SAME_DTYPE(out->dtype(), in->dtype(), weight->dtype());
    ASSERT(out->isContiguous() && in->isContiguous() && weight->isContiguous(),
           "RMSNorm input must be contiguous");
    CHECK_SAME_SHAPE(out->shape(), in->shape());
    requireFloat(in->dtype());
    auto s = streamFor(in);
    kernels::rmsNorm(out->data(), nullptr, in->data(), nullptr, weight->data(),
                     cols ? in->numel() / cols : 0, cols, eps, in->dtype(), s);
    launched("rmsNorm");
}

// Fused residual add + rms_norm (reference call pattern src/models/qwen2/layer.hpp:60-71:
// ops::add then RMSNorm; checks of both dispatchers).
void addRmsNorm(tensor_t out, tensor_t residual_out, tensor_t in, tensor_t residual,
                tensor_t weight, float eps) {
    CHECK_SAME_DEVICE(out, residual_out, in, residual, weight);
    const size_t cols = lastDim(in);
    ASSERT(weight->ndim() == 1, "RMSNorm weight must be 1D");
    ASSERT(weight->shape()[0] == cols, "RMSNorm weight shape mismatch");
    CHECK_SAME_DTYPE(out->dtype(), residual_out->dtype(), in->dtype(), residual->dtype(),
                     weight->dtype());
    CHECK_SAME_SHAPE(out->shape(), residual_out->shape(), in->shape(), residual->shape());
    ASSERT(out->isContiguous() && residual_out->isContiguous() && in->isContiguous() &&
               residual->isContiguous() && weight->isContiguous(),
           "AddRmsNorm: all tensors must be contiguous");
    requireFloat(in->dtype());
    auto s = streamFor(in);
    kernels::rmsNorm(out->data(), residual_out->data(), in->data(), residual->data(),
                     weight->data(), cols ? in->numel() / cols : 0, cols, eps, in->dtype(), s);
    launched("rmsNorm");
}

// reference src/ops/rope/op.cpp:8-51
void rope(tensor_t out, tensor_t in, tensor_t pos_ids, float theta) {
    CHECK_SAME_DEVICE(out, in, pos_ids);
    ASSERT(in->isContiguous() && out->isContiguous() && pos_ids->isContiguous(),
           "RoPE paremeter must be contiguous");
    ASSERT(in->ndim() == 3, "input shape must be 3");
    CHECK_SAME_SHAPE(in->shape(), out->shape());
    const size_t seq = in->shape()[0], nh = in->shape()[1], d = in->shape()[2];
    ASSERT(pos_ids->numel() == seq, "pos_ids length must match Seq_Len");
    ASSERT(d % 2 == 0, "Head dimension must be even for RoPE");
    CHECK_SAME_DTYPE(in->dtype(), out->dtype());
    ASSERT(pos_ids->dtype() == LLAISYS_DTYPE_I64, "token id data type must be INT64");
    requireFloat(in->dtype());
    auto s = streamFor(in);
    kernels::rope(out->data(), in->data(), reinterpret_cast<const int64_t *>(pos_ids->data()),
                  seq, nh, d, theta, in->dtype(), s);
    launched("rope");
}

// RoPE of q and k of the same tokens in one launch (the reference decoder calls rope on q
// and then on k, src/models/qwen2/attention.hpp:54-55; each gets the checks of
// src/ops/rope/op.cpp:8-51).
void ropeQK(tensor_t q_out, tensor_t q_in, tensor_t k_out, tensor_t k_in, tensor_t pos_ids,
            float theta) {
    CHECK_SAME_DEVICE(q_out, q_in, k_out, k_in, pos_ids);
    ASSERT(q_in->isContiguous() && q_out->isContiguous() && k_in->isContiguous() &&
               k_out->isContiguous() && pos_ids->isContiguous(),
           "RoPE paremeter must be contiguous");
    ASSERT(q_in->ndim() == 3 && k_in->ndim() == 3, "input shape must be 3");
    CHECK_SAME_SHAPE(q_in->shape(), q_out->shape());
    CHECK_SAME_SHAPE(k_in->shape(), k_out->shape());
    const size_t seq = q_in->shape()[0], d = q_in->shape()[2];
    ASSERT(k_in->shape()[0] == seq && k_in->shape()[2] == d,
           "RoPEQK: q and k must share seq_len and head_dim");
    ASSERT(pos_ids->numel() == seq, "pos_ids length must match Seq_Len");
    ASSERT(d % 2 == 0, "Head dimension must be even for RoPE");
    CHECK_SAME_DTYPE(q_in->dtype(), q_out->dtype(), k_in->dtype(), k_out->dtype());
    ASSERT(pos_ids->dtype() == LLAISYS_DTYPE_I64, "token id data type must be INT64");
    requireFloat(q_in->dtype());
    auto s = streamFor(q_in);
    kernels::ropeQK(q_out->data(), q_in->data(), q_in->shape()[1], k_out->data(), k_in->data(),
                    k_in->shape()[1], reinterpret_cast<const int64_t *>(pos_ids->data()), seq, d,
                    theta, q_in->dtype(), s);
    launched("ropeQK");
}

// Device-side dtype conversion (no reference op; it replaces the reference loader's host
// upcast of every bf16 / f16 weight to f32, python/llaisys/models/qwen2.py:118-120, and
// follows its cast<To>(From), src/utils/types.hpp:116-139): out[i] = cast(in[i]), same
// shape, contiguous, F32 / BF16 / F16.
void cast(tensor_t out, tensor_t in) {
    CHECK_SAME_DEVICE(out, in);
    CHECK_SAME_SHAPE(out->shape(), in->shape());
    ASSERT(out->isContiguous() && in->isContiguous(), "Cast: tensors must be contiguous");
    requireFloat(out->dtype());
    requireFloat(in->dtype());
    auto s = streamFor(out);
    const size_t n = out->numel();
    if (out->dtype() == in->dtype()) { // cast<T>(T) is the value itself
        if (n && out->data() != in->data())
            device::amd::check(hipMemcpyAsync(out->data(), in->data(), n * out->elementSize(),
                                              hipMemcpyDeviceToDevice, s),
                               "hipMemcpyAsync(cast)");
        return;
    }
    kernels::cast(out->data(), out->dtype(), in->data(), in->dtype(), n, s);
    launched("cast");
}

// reference src/ops/swiglu/op.cpp:7-38
void swiglu(tensor_t out, tensor_t gate, tensor_t up) {
    CHECK_SAME_DEVICE(out, gate, up);
    ASSERT(out->isContiguous() && gate->isContiguous() && up->isContiguous(), "must be contiguous");
    CHECK_SAME_SHAPE(out->shape(), gate->shape(), up->shape());
    ASSERT(out->ndim() == 2, "ensure 2D");
    CHECK_SAME_DTYPE(out->dtype(), gate->dtype(), up->dtype());
    requireFloat(out->dtype());
    auto s = streamFor(gate);
    kernels::swiglu(out->data(), gate->data(), up->data(), gate->numel(), out->dtype(), s);
    launched("swiglu");
}

namespace {
void checkQuantPair(const tensor_t &codes, const tensor_t &scale, const tensor_t &values,
                    const char *op) {
    CHECK_SAME_DEVICE(codes, scale, values);
    ASSERT(codes->isContiguous() && scale->isContiguous() && values->isContiguous(),
           op << ": tensors must be contiguous");
    ASSERT(codes->dtype() == LLAISYS_DTYPE_I8, op << ": codes must be INT8");
    ASSERT(scale->dtype() == LLAISYS_DTYPE_F32, op << ": scales must be F32");
    requireFloat(values->dtype());
    CHECK_SAME_SHAPE(codes->shape(), values->shape());
    const size_t cols = lastDim(values);
    ASSERT(scale->numel() * cols == values->numel(), op << ": one scale per last-dim row");
}
} // namespace

void quantizeInt8(tensor_t q, tensor_t scale, tensor_t in) {
    checkQuantPair(q, scale, in, "QuantizeInt8");
    auto s = streamFor(in);
    const size_t cols = lastDim(in);
    kernels::quantizeInt8(reinterpret_cast<int8_t *>(q->data()),
                          reinterpret_cast<float *>(scale->data()), in->data(),
                          cols ? in->numel() / cols : 0, cols, in->dtype(), s);
    launched("quantizeInt8");
}

void dequantizeInt8(tensor_t out, tensor_t q, tensor_t scale) {
    checkQuantPair(q, scale, out, "DequantizeInt8");
    auto s = streamFor(out);
    const size_t cols = lastDim(out);
    kernels::dequantizeInt8(out->data(), reinterpret_cast<const int8_t *>(q->data()),
                            reinterpret_cast<const float *>(scale->data()),
                            cols ? out->numel() / cols : 0, cols, out->dtype(), s);
    launched("dequantizeInt8");
}

namespace {
// Checks of one INT8 KV append; returns the first cache row, pos * n_kvh.
size_t checkKvAppend(const tensor_t &cache_q, const tensor_t &cache_scale, const tensor_t &kv,
                     size_t pos, const char *op) {
    CHECK_SAME_DEVICE(cache_q, cache_scale, kv);
    ASSERT(cache_q->isContiguous() && cache_scale->isContiguous() && kv->isContiguous(),
           op << ": tensors must be contiguous");
    ASSERT(cache_q->dtype() == LLAISYS_DTYPE_I8, op << ": cache codes must be INT8");
    ASSERT(cache_scale->dtype() == LLAISYS_DTYPE_F32, op << ": cache scales must be F32");
    requireFloat(kv->dtype());
    ASSERT(cache_q->ndim() == 3 && kv->ndim() == 3 && cache_scale->ndim() == 2,
           op << ": cache [max_seq, n_kvh, d], scales [max_seq, n_kvh], kv [n_tok, n_kvh, d]");
    const size_t max_seq = cache_q->shape()[0], nkvh = cache_q->shape()[1], d = cache_q->shape()[2];
    const size_t ntok = kv->shape()[0];
    ASSERT(kv->shape()[1] == nkvh && kv->shape()[2] == d, op << ": kv head shape mismatch");
    ASSERT(cache_scale->shape()[0] == max_seq && cache_scale->shape()[1] == nkvh,
           op << ": scale cache shape mismatch");
    ASSERT(pos <= max_seq && ntok <= max_seq - pos, op << ": append past the cache end");
    return pos * nkvh;
}
} // namespace

// Replaces the f32 cache-row copy of src/models/qwen2/attention.hpp:108-123.
void kvAppendInt8(tensor_t cache_q, tensor_t cache_scale, tensor_t kv, size_t pos) {
    const size_t r0 = checkKvAppend(cache_q, cache_scale, kv, pos, "KVAppendInt8");
    auto s = streamFor(kv);
    const size_t d = kv->shape()[2];
    kernels::quantizeInt8(reinterpret_cast<int8_t *>(cache_q->data()) + r0 * d,
                          reinterpret_cast<float *>(cache_scale->data()) + r0, kv->data(),
                          kv->numel() / (d ? d : 1), d, kv->dtype(), s);
    launched("quantizeInt8");
}

// The k and v appends of one decoder step (attention.hpp:108-123 updates both caches) in
// one launch; equal to kvAppendInt8(k_cache, k_scale, k, pos) then
// kvAppendInt8(v_cache, v_scale, v, pos).
void kvAppendInt8Pair(tensor_t k_cache, tensor_t k_scale, tensor_t v_cache, tensor_t v_scale,
                      tensor_t k, tensor_t v, size_t pos) {
    const size_t rk = checkKvAppend(k_cache, k_scale, k, pos, "KVAppendInt8Pair");
    const size_t rv = checkKvAppend(v_cache, v_scale, v, pos, "KVAppendInt8Pair");
    CHECK_SAME_DEVICE(k, v);
    CHECK_SAME_DTYPE(k->dtype(), v->dtype());
    ASSERT(k->shape()[2] == v->shape()[2], "KVAppendInt8Pair: k and v must share head_dim");
    auto s = streamFor(k);
    const size_t d = k->shape()[2], div = d ? d : 1;
    kernels::quantizeInt8Pair(reinterpret_cast<int8_t *>(k_cache->data()) + rk * d,
                              reinterpret_cast<float *>(k_scale->data()) + rk, k->data(),
                              k->numel() / div, reinterpret_cast<int8_t *>(v_cache->data()) + rv * d,
                              reinterpret_cast<float *>(v_scale->data()) + rv, v->data(),
                              v->numel() / div, d, k->dtype(), s);
    launched("quantizeInt8Pair");
}

// Two dequantizations in one launch (e.g. the k and v slices of an INT8 cache); equal to
// dequantizeInt8(out0, q0, scale0) then dequantizeInt8(out1, q1, scale1).
void dequantizeInt8Pair(tensor_t out0, tensor_t q0, tensor_t scale0, tensor_t out1, tensor_t q1,
                        tensor_t scale1) {
    checkQuantPair(q0, scale0, out0, "DequantizeInt8Pair");
    checkQuantPair(q1, scale1, out1, "DequantizeInt8Pair");
    CHECK_SAME_DEVICE(out0, out1);
    CHECK_SAME_DTYPE(out0->dtype(), out1->dtype());
    const size_t cols = lastDim(out0);
    ASSERT(lastDim(out1) == cols, "DequantizeInt8Pair: outputs must share the last dimension");
    auto s = streamFor(out0);
    kernels::dequantizeInt8Pair(out0->data(), reinterpret_cast<const int8_t *>(q0->data()),
                                reinterpret_cast<const float *>(scale0->data()),
                                cols ? out0->numel() / cols : 0, out1->data(),
                                reinterpret_cast<const int8_t *>(q1->data()),
                                reinterpret_cast<const float *>(scale1->data()),
                                cols ? out1->numel() / cols : 0, cols, out0->dtype(), s);
    launched("dequantizeInt8Pair");
}

namespace {
// Shape checks of reference src/ops/self_attention/op.cpp:19-45 (messages kept), plus the
// ones a GPU kernel needs (a non-zero kv head count, the output's head_dim).
void checkAttention(const tensor_t &attn_val, const tensor_t &q, const tensor_t &k,
                    const tensor_t &v) {
    ASSERT(attn_val->isContiguous() && q->isContiguous() && k->isContiguous() && v->isContiguous(),
           "Tensor shoule be contiguous");
    ASSERT(q->shape().size() == 3, "Q shape must be 3D");
    ASSERT(k->shape().size() == 3, "K shape must be 3D");
    ASSERT(v->shape().size() == 3, "V shape must be 3D");
    ASSERT(attn_val->shape().size() == 3, "Attn_Val shape must be 3D");
    const size_t seq = q->shape()[0], nh = q->shape()[1], d = q->shape()[2];
    const size_t total = k->shape()[0], nkvh = k->shape()[1];
    ASSERT(seq == attn_val->shape()[0], "attn_val seq_len mismatch");
    ASSERT(nh == attn_val->shape()[1], "attn_val nhead mismatch");
    ASSERT(total == v->shape()[0], "K/V total_len mismatch");
    ASSERT(d == k->shape()[2], "K head_dim mismatch");
    ASSERT(nkvh == v->shape()[1], "K/V head mismatch");
    ASSERT(nkvh > 0 && nh % nkvh == 0, "nhead must be divisible by kv_head (GQA)");
    ASSERT(attn_val->shape()[2] == v->shape()[2], "attn_val v_head_dim mismatch");
}

void launchAttention(const tensor_t &attn_val, const tensor_t &q, const tensor_t &k,
                     const tensor_t &v, const float *ks, const float *vs, float scale) {
    auto s = streamFor(q);
    const size_t d = q->shape()[2];
    const size_t reserved = kernels::kScratchReserved;
    const size_t need = kernels::selfAttentionWorkspaceBytes(q->shape()[0], q->shape()[1], d);
    char *ws = static_cast<char *>(device::amd::workspace(q->deviceId(), reserved + need));
    kernels::selfAttention(attn_val->data(), q->data(), k->data(), v->data(), ks, vs, q->shape()[0],
                           k->shape()[0], q->shape()[1], k->shape()[1], d, v->shape()[2], scale,
                           q->dtype(), ws + reserved, need, s);
    launched("selfAttention");
}
} // namespace

// reference src/ops/self_attention/op.cpp:19-45
void selfAttention(tensor_t attn_val, tensor_t q, tensor_t k, tensor_t v, float scale) {
    CHECK_SAME_DEVICE(attn_val, q, k, v);
    checkAttention(attn_val, q, k, v);
    CHECK_SAME_DTYPE(attn_val->dtype(), q->dtype(), k->dtype(), v->dtype());
    requireFloat(q->dtype());
    launchAttention(attn_val, q, k, v, nullptr, nullptr, scale);
}

// Attention over an INT8 cache: the composition dequantizeInt8 (into q's dtype) then
// selfAttention, reading the caches as codes.
namespace {
void checkAttentionInt8KV(const tensor_t &attn_val, const tensor_t &q, const tensor_t &k_codes,
                          const tensor_t &k_scale, const tensor_t &v_codes, const tensor_t &v_scale) {
    CHECK_SAME_DEVICE(attn_val, q, k_codes, v_codes);
    CHECK_SAME_DEVICE(q, k_scale, v_scale);
    checkAttention(attn_val, q, k_codes, v_codes);
    CHECK_SAME_DTYPE(attn_val->dtype(), q->dtype());
    requireFloat(q->dtype());
    ASSERT(k_codes->dtype() == LLAISYS_DTYPE_I8 && v_codes->dtype() == LLAISYS_DTYPE_I8,
           "SelfAttentionInt8KV: cache codes must be INT8");
    ASSERT(k_scale->dtype() == LLAISYS_DTYPE_F32 && v_scale->dtype() == LLAISYS_DTYPE_F32,
           "SelfAttentionInt8KV: cache scales must be F32");
    ASSERT(k_scale->isContiguous() && v_scale->isContiguous(), "Tensor shoule be contiguous");
    const size_t total = k_codes->shape()[0], nkvh = k_codes->shape()[1];
    ASSERT(k_scale->ndim() == 2 && k_scale->shape()[0] == total && k_scale->shape()[1] == nkvh &&
               v_scale->ndim() == 2 && v_scale->shape()[0] == total && v_scale->shape()[1] == nkvh,
           "SelfAttentionInt8KV: scales must be [total_len, kv_head]");
}
} // namespace

void selfAttentionInt8KV(tensor_t attn_val, tensor_t q, tensor_t k_codes, tensor_t k_scale,
                         tensor_t v_codes, tensor_t v_scale, float scale) {
    checkAttentionInt8KV(attn_val, q, k_codes, k_scale, v_codes, v_scale);
    launchAttention(attn_val, q, k_codes, v_codes, reinterpret_cast<const float *>(k_scale->data()),
                    reinterpret_cast<const float *>(v_scale->data()), scale);
}

// The same op with its workspace in the library's file-scope device scratch
// (kernels::kNoAllocScratchBytes per GPU): nothing is allocated.  Decode and the vector
// kernels put their split partials there with the chunking selfAttentionInt8KV uses (the
// same bits), and calls whose partials would not fit are rejected.  A bf16 prefill on the
// MFMA kernel dequantizes the caches into the scratch when they fit, else the kernel
// converts the codes itself; either way the same operands in the same MFMA order, so the
// same bits.  Calls on one GPU share the scratch: overlapping calls (several threads or
// streams) race.
void selfAttentionInt8KVNoAlloc(tensor_t attn_val, tensor_t q, tensor_t k_codes, tensor_t k_scale,
                                tensor_t v_codes, tensor_t v_scale, float scale) {
    checkAttentionInt8KV(attn_val, q, k_codes, k_scale, v_codes, v_scale);
    const size_t seq = q->shape()[0], nh = q->shape()[1], d = q->shape()[2];
    const size_t need = kernels::selfAttentionInt8KVScratchBytes(
        attn_val->data(), q->data(), k_codes->data(), v_codes->data(), seq, k_codes->shape()[0], nh,
        k_codes->shape()[1], d, v_codes->shape()[2], scale, q->dtype(), kernels::kNoAllocScratchBytes);
    if (need > kernels::kNoAllocScratchBytes)
        LLAISYS_FAIL(std::invalid_argument,
                     "SelfAttentionInt8KVNoAlloc: the call needs " << need << " bytes of scratch, more than the "
                         << kernels::kNoAllocScratchBytes << " it holds (queries x heads x (head_dim + 2) x 4 KiB); "
                            "use llaisysSelfAttentionInt8KV",
                     "scratch too small");
    auto s = streamFor(q); // makes q's device current
    char err[256] = {};
    void *ws = kernels::noAllocScratch(q->deviceId(), err, sizeof err);
    if (!ws) LLAISYS_FAIL(std::runtime_error, "SelfAttentionInt8KVNoAlloc: " << err, "no scratch");
    kernels::selfAttention(attn_val->data(), q->data(), k_codes->data(), v_codes->data(),
                           reinterpret_cast<const float *>(k_scale->data()),
                           reinterpret_cast<const float *>(v_scale->data()), seq, k_codes->shape()[0],
                           nh, k_codes->shape()[1], d, v_codes->shape()[2], scale, q->dtype(), ws,
                           need, s);
    launched("selfAttentionInt8KVNoAlloc");
}

// reference src/ops/rearrange/op.cpp:4-6 (a stub there): out[i] = in[i] for every
// multi-index, between any two layouts of one shape (Tensor::copyInto on the GPU).
void rearrange(tensor_t out, tensor_t in) {
    CHECK_SAME_DEVICE(out, in);
    CHECK_SAME_SHAPE(out->shape(), in->shape());
    CHECK_SAME_DTYPE(out->dtype(), in->dtype());
    ASSERT(in->ndim() <= 8, "Rearrange: at most 8 dimensions");
    streamFor(out); // AMD tensors only: this library has no CPU compute path
    in->copyInto(out);
}

// Random sampling after argmax (no reference kernel; README.md:397-399 asks for it,
// python/llaisys/models/qwen2.py:216-218 takes its parameters): one index per row of
// logits [V] or [rows, V].
void randomSample(tensor_t out_idx, tensor_t logits, float temperature, int64_t top_k,
                  float top_p, uint64_t seed) {
    CHECK_SAME_DEVICE(out_idx, logits);
    ASSERT(out_idx->isContiguous() && logits->isContiguous(), "RandomSample: tensors must be contiguous");
    ASSERT(out_idx->dtype() == LLAISYS_DTYPE_I32 || out_idx->dtype() == LLAISYS_DTYPE_I64,
           "RandomSample: out_idx must be INT32 or INT64");
    requireFloat(logits->dtype());
    ASSERT(logits->ndim() == 1 || logits->ndim() == 2, "RandomSample: logits must be [V] or [rows, V]");
    const size_t rows = logits->ndim() == 2 ? logits->shape()[0] : 1;
    const size_t V = logits->shape().back();
    ASSERT(out_idx->numel() == rows, "RandomSample: out_idx must hold one index per row");
    ASSERT(V > 0 && V < (size_t(1) << 31), "RandomSample: vocabulary size must be in [1, 2^31)");
    const bool greedy = !(temperature > 0.0f) || top_k == 1;
    ASSERT(greedy || (top_k >= 2 && top_k <= 1024),
           "RandomSample: top_k must be 1 or in [2, 1024] when sampling");
    auto s = streamFor(logits);
    void *ws = device::amd::workspace(logits->deviceId(),
                                      kernels::kScratchReserved +
                                          kernels::randomSampleWorkspaceBytes(rows, V, logits->dtype()));
    kernels::randomSample(out_idx->data(), out_idx->dtype() == LLAISYS_DTYPE_I64, logits->data(), rows,
                          V, logits->dtype(), temperature, top_k, top_p, seed, ws, s);
    launched("randomSample");
}

namespace {
// Shape checks of reference src/ops/linear/op.cpp:10-42 (messages kept); a bias that is
// null or has no elements means no bias.  Returns the row count.
size_t checkLinear(const tensor_t &out, const tensor_t &in, const tensor_t &weight,
                   const tensor_t &bias, bool has_bias) {
    ASSERT(weight->ndim() == 2, "Linear: weight must be 2D");
    const size_t in_features = weight->shape()[1], out_features = weight->shape()[0];
    ASSERT(lastDim(in) == in_features, "Linear: input feature dim mismatch");
    ASSERT(lastDim(out) == out_features, "Linear: output feature dim mismatch");
    ASSERT(in_features > 0 && out_features > 0, "Linear: empty weight");
    const size_t rows = in->numel() / in_features;
    ASSERT(out->numel() / out_features == rows, "Linear: input/output rows mismatch");
    if (has_bias) ASSERT(bias->numel() == out_features, "Linear: bias shape mismatch");
    ASSERT(out->isContiguous() && in->isContiguous() && weight->isContiguous(),
           "Linear inputs must be contiguous");
    if (has_bias) ASSERT(bias->isContiguous(), "Linear bias must be contiguous");
    ASSERT(rows < (size_t(1) << 31) && in_features < (size_t(1) << 31) &&
               out_features < (size_t(1) << 31),
           "Linear: dimensions must be below 2^31");
    return rows;
}
} // namespace

// reference src/ops/linear/op.cpp:10-42
void linear(tensor_t out, tensor_t in, tensor_t weight, tensor_t bias) {
    const bool has_bias = bias != nullptr && bias->numel() > 0;
    if (has_bias) {
        CHECK_SAME_DEVICE(out, in, weight, bias);
        CHECK_SAME_DTYPE(out->dtype(), in->dtype(), weight->dtype(), bias->dtype());
    } else {
        CHECK_SAME_DEVICE(out, in, weight);
        CHECK_SAME_DTYPE(out->dtype(), in->dtype(), weight->dtype());
    }
    const size_t rows = checkLinear(out, in, weight, bias, has_bias);
    requireFloat(in->dtype());
    auto s = streamFor(in);
    kernels::linear(out->data(), in->data(), weight->data(), nullptr,
                    has_bias ? bias->data() : nullptr, rows, weight->shape()[1],
                    weight->shape()[0], in->dtype(), s);
    launched("linear");
}

// linear with INT8 weight codes [N, K] and one F32 scale per output channel:
// out = T(w_scale[n] * sum_k in[m][k] * code[n][k] + bias[n]).
void linearW8A16(tensor_t out, tensor_t in, tensor_t w_codes, tensor_t w_scale, tensor_t bias) {
    const bool has_bias = bias != nullptr && bias->numel() > 0;
    CHECK_SAME_DEVICE(out, in, w_codes, w_scale);
    CHECK_SAME_DTYPE(out->dtype(), in->dtype());
    if (has_bias) {
        CHECK_SAME_DEVICE(out, bias);
        CHECK_SAME_DTYPE(out->dtype(), bias->dtype());
    }
    ASSERT(w_codes->dtype() == LLAISYS_DTYPE_I8, "LinearW8A16: weight codes must be INT8");
    ASSERT(w_scale->dtype() == LLAISYS_DTYPE_F32, "LinearW8A16: weight scales must be F32");
    const size_t rows = checkLinear(out, in, w_codes, bias, has_bias);
    ASSERT(w_scale->isContiguous() && w_scale->numel() == w_codes->shape()[0],
           "LinearW8A16: one contiguous scale per output feature");
    requireFloat(in->dtype());
    auto s = streamFor(in);
    kernels::linear(out->data(), in->data(), w_codes->data(),
                    reinterpret_cast<const float *>(w_scale->data()),
                    has_bias ? bias->data() : nullptr, rows, w_codes->shape()[1],
                    w_codes->shape()[0], in->dtype(), s);
    launched("linearW8A16");
}

namespace {
// Byte ranges of two contiguous tensors intersect.
bool overlaps(const tensor_t &a, const tensor_t &b) {
    const std::byte *a0 = a->data(), *b0 = b->data();
    return a0 < b0 + b->numel() * b->elementSize() && b0 < a0 + a->numel() * a->elementSize();
}
} // namespace

// rms_norm (after an optional residual add) fused ahead of a linear, and optionally swiglu
// after it: the decoder's input_layernorm -> q/k/v projections and add ->
// post_attention_layernorm -> gate / up projections -> swiglu (reference
// src/models/qwen2/layer.hpp:51-53, :66-71, src/models/qwen2/mlp.hpp:22-33) as one launch
// for one row.  weight is [Nw, K] (INT8 codes with weight_scale, else the activation type);
// with swiglu its rows [0, Nw/2) are the gate and [Nw/2, Nw) the up projection and out is
// [rows, Nw/2].  Other row counts and shapes run the same ops one after another.
void rmsNormLinear(tensor_t out, tensor_t residual_out, tensor_t in, tensor_t residual,
                   tensor_t norm_weight, float eps, tensor_t weight, tensor_t weight_scale,
                   tensor_t bias, bool swiglu) {
    const bool has_res = residual != nullptr, has_bias = bias != nullptr && bias->numel() > 0;
    const bool int8 = weight_scale != nullptr;
    CHECK_SAME_DEVICE(out, in, norm_weight, weight);
    ASSERT(has_res == (residual_out != nullptr),
           "RmsNormLinear: residual and residual_out come together");
    if (has_res) CHECK_SAME_DEVICE(out, residual, residual_out);
    if (int8) CHECK_SAME_DEVICE(out, weight_scale);
    if (has_bias) CHECK_SAME_DEVICE(out, bias);
    CHECK_SAME_DTYPE(out->dtype(), in->dtype(), norm_weight->dtype());
    if (has_res) CHECK_SAME_DTYPE(out->dtype(), residual->dtype(), residual_out->dtype());
    if (has_bias) CHECK_SAME_DTYPE(out->dtype(), bias->dtype());
    requireFloat(in->dtype());
    for (const auto &t : {out, in, norm_weight, weight})
        ASSERT(t->isContiguous(), "RmsNormLinear: tensors must be contiguous");
    const size_t K = lastDim(in);
    ASSERT(K > 0, "RmsNormLinear: empty rows");
    const size_t rows = in->numel() / K;
    ASSERT(norm_weight->ndim() == 1, "RMSNorm weight must be 1D");
    ASSERT(norm_weight->shape()[0] == K, "RMSNorm weight shape mismatch");
    if (has_res) {
        ASSERT(residual->isContiguous() && residual_out->isContiguous(),
               "RmsNormLinear: tensors must be contiguous");
        CHECK_SAME_SHAPE(in->shape(), residual->shape(), residual_out->shape());
        ASSERT(!overlaps(residual_out, in) && !overlaps(residual_out, residual),
               "RmsNormLinear: residual_out must not overlap in or residual");
    }
    ASSERT(weight->ndim() == 2, "Linear: weight must be 2D");
    ASSERT(weight->shape()[1] == K, "Linear: input feature dim mismatch");
    const size_t Nw = weight->shape()[0];
    ASSERT(Nw > 0, "Linear: empty weight");
    if (int8) {
        ASSERT(weight->dtype() == LLAISYS_DTYPE_I8, "LinearW8A16: weight codes must be INT8");
        ASSERT(weight_scale->dtype() == LLAISYS_DTYPE_F32, "LinearW8A16: weight scales must be F32");
        ASSERT(weight_scale->isContiguous() && weight_scale->numel() == Nw,
               "LinearW8A16: one contiguous scale per output feature");
    } else {
        CHECK_SAME_DTYPE(out->dtype(), weight->dtype());
    }
    if (swiglu) ASSERT(Nw % 2 == 0, "RmsNormLinear: swiglu needs an even number of weight rows");
    const size_t N = swiglu ? Nw / 2 : Nw;
    ASSERT(lastDim(out) == N, "Linear: output feature dim mismatch");
    ASSERT(out->numel() / N == rows, "Linear: input/output rows mismatch");
    if (has_bias) {
        ASSERT(bias->numel() == Nw, "Linear: bias shape mismatch");
        ASSERT(bias->isContiguous(), "Linear bias must be contiguous");
    }
    ASSERT(!overlaps(out, in) && !(has_res && (overlaps(out, residual) || overlaps(out, residual_out))),
           "RmsNormLinear: out must not overlap in, residual or residual_out");
    ASSERT(rows < (size_t(1) << 31) && K < (size_t(1) << 31) && Nw < (size_t(1) << 31),
           "Linear: dimensions must be below 2^31");
    if (rows == 0) return;
    auto s = streamFor(in);
    const auto *sc = int8 ? reinterpret_cast<const float *>(weight_scale->data()) : nullptr;
    const void *bp = has_bias ? bias->data() : nullptr;
    void *ro = has_res ? residual_out->data() : nullptr;
    const void *ri = has_res ? residual->data() : nullptr;
    if (kernels::rmsNormLinearFused(out->data(), ro, in->data(), ri, norm_weight->data(), eps,
                                    weight->data(), sc, bp, rows, K, N, swiglu, in->dtype(), s)) {
        launched("rmsNormLinear");
        return;
    }
    // The same ops one after another through library scratch: xn [rows, K], then (swiglu)
    // gate and up [rows, N] from the two halves of the weight.
    const size_t es = in->elementSize(), xb = (rows * K * es + 255) / 256 * 256;
    const size_t gb = swiglu ? (rows * N * es + 255) / 256 * 256 : 0;
    char *ws = static_cast<char *>(device::amd::workspace(
                   in->deviceId(), kernels::kScratchReserved + xb + 2 * gb)) +
               kernels::kScratchReserved;
    kernels::rmsNorm(ws, ro, in->data(), ri, norm_weight->data(), rows, K, eps, in->dtype(), s);
    if (!swiglu) {
        kernels::linear(out->data(), ws, weight->data(), sc, bp, rows, K, N, in->dtype(), s);
    } else {
        const size_t wb = N * K * weight->elementSize();
        char *g = ws + xb, *u = ws + xb + gb;
        kernels::linear(g, ws, weight->data(), sc, bp, rows, K, N, in->dtype(), s);
        kernels::linear(u, ws, weight->data() + wb, sc ? sc + N : nullptr,
                        bp ? static_cast<const char *>(bp) + N * es : nullptr, rows, K, N,
                        in->dtype(), s);
        kernels::swiglu(out->data(), g, u, rows * N, in->dtype(), s);
    }
    launched("rmsNormLinear (composed)");
}

} // namespace llaisys::ops

namespace llaisys::ops {

// Fused RoPE + INT8 KV append: the reference decoder's rope(q), rope(k) and cache update
// (src/models/qwen2/attention.hpp:54-59, :108-123) with the cache in INT8.
void ropeKvAppendInt8(tensor_t q_out, tensor_t q_in, tensor_t k_in, tensor_t v_in,
                      tensor_t pos_ids, float theta, tensor_t k_cache, tensor_t k_scale,
                      tensor_t v_cache, tensor_t v_scale, size_t pos) {
    CHECK_SAME_DEVICE(q_out, q_in, k_in, v_in, pos_ids, k_cache, k_scale, v_cache, v_scale);
    for (const auto &t : {q_out, q_in, k_in, v_in, pos_ids, k_cache, k_scale, v_cache, v_scale})
        ASSERT(t->isContiguous(), "RoPEKVAppend: tensors must be contiguous");
    ASSERT(q_in->ndim() == 3 && k_in->ndim() == 3 && v_in->ndim() == 3, "input shape must be 3");
    CHECK_SAME_SHAPE(q_in->shape(), q_out->shape());
    CHECK_SAME_SHAPE(k_in->shape(), v_in->shape());
    const size_t seq = q_in->shape()[0], nq = q_in->shape()[1], d = q_in->shape()[2];
    const size_t nk = k_in->shape()[1];
    ASSERT(k_in->shape()[0] == seq && k_in->shape()[2] == d,
           "RoPEKVAppend: q and k must share seq_len and head_dim");
    ASSERT(pos_ids->numel() == seq, "pos_ids length must match Seq_Len");
    ASSERT(d % 2 == 0, "Head dimension must be even for RoPE");
    CHECK_SAME_DTYPE(q_in->dtype(), q_out->dtype(), k_in->dtype(), v_in->dtype());
    ASSERT(pos_ids->dtype() == LLAISYS_DTYPE_I64, "token id data type must be INT64");
    requireFloat(q_in->dtype());
    ASSERT(k_cache->dtype() == LLAISYS_DTYPE_I8 && v_cache->dtype() == LLAISYS_DTYPE_I8,
           "RoPEKVAppend: cache codes must be INT8");
    ASSERT(k_scale->dtype() == LLAISYS_DTYPE_F32 && v_scale->dtype() == LLAISYS_DTYPE_F32,
           "RoPEKVAppend: cache scales must be F32");
    ASSERT(k_cache->ndim() == 3 && k_scale->ndim() == 2, "RoPEKVAppend: cache [max_seq, n_kvh, d], scales [max_seq, n_kvh]");
    CHECK_SAME_SHAPE(k_cache->shape(), v_cache->shape());
    CHECK_SAME_SHAPE(k_scale->shape(), v_scale->shape());
    const size_t max_seq = k_cache->shape()[0];
    ASSERT(k_cache->shape()[1] == nk && k_cache->shape()[2] == d, "RoPEKVAppend: kv head shape mismatch");
    ASSERT(k_scale->shape()[0] == max_seq && k_scale->shape()[1] == nk, "RoPEKVAppend: scale cache shape mismatch");
    ASSERT(pos <= max_seq && seq <= max_seq - pos, "RoPEKVAppend: append past the cache end");
    auto s = streamFor(q_in);
    const size_t r0 = pos * nk;
    auto *kc = reinterpret_cast<int8_t *>(k_cache->data()) + r0 * d;
    auto *vc = reinterpret_cast<int8_t *>(v_cache->data()) + r0 * d;
    auto *ks = reinterpret_cast<float *>(k_scale->data()) + r0;
    auto *vs = reinterpret_cast<float *>(v_scale->data()) + r0;
    const auto *p = reinterpret_cast<const int64_t *>(pos_ids->data());
    if (kernels::ropeKvAppendFused(q_out->data(), q_in->data(), nq, k_in->data(), v_in->data(), nk,
                                   kc, ks, vc, vs, p, seq, d, theta, q_in->dtype(), s)) {
        launched("ropeKvAppend");
        return;
    }
    // Shapes outside the fused kernel: the same composition through library scratch.
    void *tmp = static_cast<char *>(device::amd::workspace(
                    q_in->deviceId(), kernels::kScratchReserved +
                                          kernels::ropeKvAppendWorkspaceBytes(seq, nk, d, q_in->dtype()))) +
                kernels::kScratchReserved;
    kernels::ropeQK(q_out->data(), q_in->data(), nq, tmp, k_in->data(), nk, p, seq, d, theta,
                    q_in->dtype(), s);
    kernels::quantizeInt8(kc, ks, tmp, seq * nk, d, q_in->dtype(), s);
    kernels::quantizeInt8(vc, vs, v_in->data(), seq * nk, d, q_in->dtype(), s);
    launched("ropeKvAppend (composed)");
}

} // namespace llaisys::ops
