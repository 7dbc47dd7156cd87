// Host-side launchers of the gfx950 kernels: plain pointers, sizes and a stream.
//
// Callers (the op dispatchers) have already validated shapes, dtypes and devices; the
// launchers choose the kernel variant (vectorised 16-byte path when sizes and addresses
// allow, scalar path otherwise) and enqueue it asynchronously on `stream`.
#pragma once

#include "llaisys.h"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace llaisys::kernels {

// y = rms_norm(x) per row of `cols`; when `residual` is non-null the input is first
// h = round(x + residual), h is stored to `residual_out` and normalised instead.
void rmsNorm(void *out, void *residual_out, const void *in, const void *residual,
             const void *weight, size_t rows, size_t cols, float eps, llaisysDataType_t dt,
             hipStream_t stream);

// Rotate-half RoPE on [seq, n_heads, head_dim] with int64 positions.
void rope(void *out, const void *in, const int64_t *pos, size_t seq, size_t n_heads,
          size_t head_dim, float theta, llaisysDataType_t dt, hipStream_t stream);

// RoPE of q [seq, nh_q, head_dim] and k [seq, nh_k, head_dim] (same positions) in one launch.
void ropeQK(void *q_out, const void *q_in, size_t nh_q, void *k_out, const void *k_in,
            size_t nh_k, const int64_t *pos, size_t seq, size_t head_dim, float theta,
            llaisysDataType_t dt, hipStream_t stream);

// Fused RoPE + INT8 KV append: q_out = rope(q); codes / scales of quantize(rope(k)) and
// quantize(v) written to the cache rows the pointers start at.  Returns false (nothing
// launched) for shapes the fused kernel does not cover; the caller then composes the ops.
bool ropeKvAppendFused(void *q_out, const void *q_in, size_t nh_q, const void *k_in,
                       const void *v_in, size_t nh_kv, int8_t *k_codes, float *k_scale,
                       int8_t *v_codes, float *v_scale, const int64_t *pos, size_t seq,
                       size_t head_dim, float theta, llaisysDataType_t dt, hipStream_t stream);
size_t ropeKvAppendWorkspaceBytes(size_t seq, size_t nh_kv, size_t head_dim, llaisysDataType_t dt);

// out[i] = cast<out type>(in[i]) over n elements of F32 / BF16 / F16, through f32 with the
// reference's rounding rules (types.hpp:116-139); the caller copies equal types itself.
void cast(void *out, llaisysDataType_t out_dt, const void *in, llaisysDataType_t in_dt, size_t n,
          hipStream_t stream);

// out = up * gate / (1 + exp(-gate)) over n elements.
void swiglu(void *out, const void *gate, const void *up, size_t n, llaisysDataType_t dt,
            hipStream_t stream);

// c = a + b over n elements (half types: f32 add, then round).
void add(void *c, const void *a, const void *b, size_t n, llaisysDataType_t dt,
         hipStream_t stream);

// out[i, :] = weight[index[i], :] for rows of `row_bytes`; an id outside [0, vocab)
// leaves its row untouched and ORs 1 into *err.
void embedding(void *out, const void *index, bool index_i64, size_t n_index, const void *weight,
               size_t vocab, size_t row_bytes, int *err, hipStream_t stream);

// Per-row argmax of vals [rows, cols]; idx is I32 or I64, val has the dtype of vals.
void argmaxRows(void *idx, bool idx_i64, void *val, const void *vals, size_t rows, size_t cols,
                llaisysDataType_t dt, hipStream_t stream);

// Library scratch layout (zeroed once when allocated): bytes [0, 256) hold the flat argmax's
// completion counter and [kSampleStateOffset, kScratchReserved) the sampler's per-row
// histograms and counters; both stay zero between launches.  Other users of the scratch
// start at kScratchReserved.
constexpr size_t kSampleRows = 16;            // rows per sampler launch
constexpr size_t kSampleRowStateBytes = 16400;
constexpr size_t kSampleStateOffset = 256;
constexpr size_t kScratchReserved =
    (kSampleStateOffset + kSampleRows * kSampleRowStateBytes + 255) / 256 * 256;

// Flat argmax over n elements; `workspace` (>= argmaxWorkspaceBytes(n)) holds the
// completion counter (first kScratchReserved bytes, zero before the first call; the kernel
// leaves it zero again) and the per-block partials after it.
size_t argmaxWorkspaceBytes(size_t n, llaisysDataType_t dt);
void argmax(void *idx, bool idx_i64, void *val, const void *vals, size_t n,
            llaisysDataType_t dt, void *workspace, hipStream_t stream);

// INT8 symmetric absmax quantization per row of `cols` elements.
void quantizeInt8(int8_t *q, float *scale, const void *in, size_t rows, size_t cols,
                  llaisysDataType_t dt, hipStream_t stream);

// Two quantizations of rows of the same length and type in one launch (rows1 may be 0).
void quantizeInt8Pair(int8_t *q0, float *scale0, const void *in0, size_t rows0, int8_t *q1,
                      float *scale1, const void *in1, size_t rows1, size_t cols,
                      llaisysDataType_t dt, hipStream_t stream);

// out = T(float(q) * scale[row]).
void dequantizeInt8(void *out, const int8_t *q, const float *scale, size_t rows, size_t cols,
                    llaisysDataType_t dt, hipStream_t stream);

// Two dequantizations of rows of the same length and type in one launch (rows1 may be 0).
void dequantizeInt8Pair(void *out0, const int8_t *q0, const float *scale0, size_t rows0,
                        void *out1, const int8_t *q1, const float *scale1, size_t rows1,
                        size_t cols, llaisysDataType_t dt, hipStream_t stream);

// Causal GQA self-attention: q [seq, nh, d], k [total, nkvh, d], v [total, nkvh, dv],
// out [seq, nh, dv].  With k_scale / v_scale non-null, k and v are INT8 codes with one F32
// scale per (token, kv head) row.  `ws` (ws_bytes) holds the partials of a split launch;
// selfAttentionWorkspaceBytes(seq, nh, d) lets it split decode launches fully.
size_t selfAttentionWorkspaceBytes(size_t seq, size_t nh, size_t head_dim);

// Scratch of the allocation-free attention entry point: a file-scope device array of
// kNoAllocScratchBytes per GPU.  noAllocScratch returns its device address on `device`
// (which must be current), resolved once per device by hipGetSymbolAddress; on failure it
// returns null and writes the reason to err.
constexpr size_t kNoAllocScratchBytes = size_t(24) << 20;
void *noAllocScratch(int device, char *err, size_t err_len);
// Workspace bytes selfAttention over an INT8 cache uses for these arguments: the bf16
// prefill (MFMA) path only needs room for the dequantized caches, 2 * total * nkvh * d bf16
// (0 if that exceeds `cap`: the kernel then converts the codes itself, with the same bits);
// every other path the split partials, selfAttentionWorkspaceBytes(seq, nh, d).
size_t selfAttentionInt8KVScratchBytes(const void *out, const void *q, const void *k, const void *v,
                                       size_t seq, size_t total, size_t nh, size_t nkvh, size_t d,
                                       size_t dv, float scale, llaisysDataType_t dt, size_t cap);
void selfAttention(void *out, const void *q, const void *k, const void *v, const float *k_scale,
                   const float *v_scale, size_t seq, size_t total, size_t nh, size_t nkvh,
                   size_t d, size_t dv, float scale, llaisysDataType_t dt, void *ws,
                   size_t ws_bytes, hipStream_t stream);

// out [rows, N] = x [rows, K] w^T (+ bias [N]); with w_scale non-null w is INT8 codes
// [N, K] and the sum of each output channel n is multiplied by w_scale[n] (W8A16).  rows,
// K and N below 2^31.
void linear(void *out, const void *x, const void *w, const float *w_scale, const void *bias,
            size_t rows, size_t in_features, size_t out_features, llaisysDataType_t dt,
            hipStream_t stream);

// One row: h = residual ? T(in + residual) : in (h stored to residual_out when residual is
// non-null), xn = rms_norm(h) as rmsNorm computes it, y = linear(xn) (W8A16 when w_scale is
// non-null) as linear computes one row with its GEMV, and out = y, or with `swiglu`
// out[n] = swiglu(gate = y[n], up = y[n + out_features]) over a weight of 2 * out_features
// rows.  residual_out must not overlap in or residual.  Returns false (nothing launched)
// for shapes the fused kernel does not cover; the caller then composes the ops.
bool rmsNormLinearFused(void *out, void *residual_out, const void *in, const void *residual,
                        const void *norm_weight, float eps, const void *w, const float *w_scale,
                        const void *bias, size_t rows, size_t in_features, size_t out_features,
                        bool swiglu, llaisysDataType_t dt, hipStream_t stream);

// out[i] = in[i] for every multi-index i of `shape` (ndim <= 8), element strides per layout,
// elements of esize (1, 2, 4 or 8) bytes.
void rearrange(void *out, const void *in, size_t ndim, const size_t *shape, const ptrdiff_t *in_strides,
               const ptrdiff_t *out_strides, size_t esize, hipStream_t stream);

// Random sampling of one index per row of logits [rows, V] (rule: temperature <= 0 or
// top_k == 1 -> argmax; else top_k in [2, 1024] (clamped to V), top_p, splitmix64(seed +
// row) uniform).  `ws` is the library scratch of at least kScratchReserved +
// randomSampleWorkspaceBytes(rows, V, dt) bytes.
size_t randomSampleWorkspaceBytes(size_t rows, size_t V, llaisysDataType_t dt);
void randomSample(void *out_idx, bool i64, const void *logits, size_t rows, size_t V,
                  llaisysDataType_t dt, float temperature, int64_t top_k, float top_p,
                  uint64_t seed, void *ws, hipStream_t stream);

} // namespace llaisys::kernels
