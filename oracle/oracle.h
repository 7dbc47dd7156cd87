/*
 * CPU oracle for the LLAISYS per-layer ops -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU arithmetic (cited per function in
 * oracle.c).  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it, and only as the checker / timed CPU baseline.  The product library
 * (llaisys_amd, libllaisys.so) never links, loads or calls it.
 *
 * Data-type codes are the llaisysDataType_t values: F16 = 12, F32 = 13, BF16 = 19,
 * I32 = 5, I64 = 6.  All buffers are contiguous host memory.
 */
#ifndef LLAISYS_ORACLE_H
#define LLAISYS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#define ORC_F16 12
#define ORC_F32 13
#define ORC_BF16 19
#define ORC_I32 5
#define ORC_I64 6

uint16_t orc_f32_to_bf16(float v);
float orc_bf16_to_f32(uint16_t v);
uint16_t orc_f32_to_f16(float v);
float orc_f16_to_f32(uint16_t v);
/* out[i] = cast<out type>(in[i]) as the reference's types.hpp:116-139 (through f32) */
void orc_cast(void *out, int out_dtype, const void *in, int in_dtype, size_t n);

void orc_add(void *c, const void *a, const void *b, size_t n, int dtype);
void orc_rms_norm(void *out, const void *in, const void *w, size_t rows, size_t cols,
                  float eps, int dtype);
void orc_add_rms_norm(void *out, void *residual_out, const void *in, const void *residual,
                      const void *w, size_t rows, size_t cols, float eps, int dtype);
void orc_rope(void *out, const void *in, const int64_t *pos_ids, size_t seq_len,
              size_t n_heads, size_t head_dim, float theta, int dtype);
void orc_swiglu(void *out, const void *gate, const void *up, size_t n, int dtype);
/* Returns 0, or -1 (after copying the rows before it) at the first id outside [0, vocab). */
int orc_embedding(void *out, const void *index, int index_dtype, size_t n_index,
                  const void *weight, size_t vocab, size_t dim, int dtype);
void orc_argmax(void *max_idx, int idx_dtype, void *max_val, const void *vals, size_t n,
                int dtype);
void orc_argmax_rows(void *max_idx, int idx_dtype, void *max_val, const void *vals,
                     size_t rows, size_t cols, int dtype);
void orc_quantize_int8(int8_t *q, float *scale, const void *in, size_t rows, size_t cols,
                       int dtype);
void orc_dequantize_int8(void *out, const int8_t *q, const float *scale, size_t rows,
                         size_t cols, int dtype);
/* Returns -1 if pos + n_tok > max_seq (nothing written), else 0. */
int orc_kv_append_int8(int8_t *cache_q, float *cache_scale, size_t max_seq, const void *kv,
                       size_t n_tok, size_t n_kvh, size_t head_dim, size_t pos, int dtype);

/* self_attention_cpu.cpp:13-115; -1 on an invalid head split */
int orc_self_attention(void *out, const void *q, const void *k, const void *v, size_t seq,
                       size_t total, size_t nh, size_t nkvh, size_t d, size_t dv, float scale,
                       int dtype);

/* linear_cpu.cpp:11-41 (bias may be NULL) */
void orc_linear(void *out, const void *x, const void *w, const void *bias, size_t rows,
                size_t in_features, size_t out_features, int dtype);
/* W8A16 rule: T(scale[n] * sum_k x * code + bias[n]) */
void orc_linear_w8a16(void *out, const void *x, const int8_t *code, const float *scale,
                      const void *bias, size_t rows, size_t in_features, size_t out_features,
                      int dtype);

/* Random sampling after argmax (no reference kernel: README.md:397-399 asks for
 * temperature, top-k and top-p; python/llaisys/models/qwen2.py:216-218 takes them and
 * ignores them).  The rule, per row of `logits` [rows, V]:
 *   temperature <= 0 or top_k == 1: the row's argmax (first maximum);
 *   else z = x * (1 / temperature) (1/T rounded to f32 once), order the V elements by
 *   (key(z) desc, index asc) with key the order-preserving u32 of the f32 bits (a NaN z
 *   takes the key of -inf), keep the first min(top_k, V) (top_k must be in [2, 1024]),
 *   weights w = floor(p * 2^31) with p = orc_sample_exp2((z - zmax) * log2(e)), where
 *   z - zmax counts as 0 for an element whose key equals the first one's (so infinite
 *   ties weigh 2^0 and W > 0), W = sum of w; top_p < 1 keeps the shortest
 *   prefix whose w-sum >= max(1, floor(top_p * W)) (top_p <= 0: the first element);
 *   then with u24 = splitmix64(seed + row) >> 40 and r = floor(u24 * W_kept / 2^24), the
 *   sample is the first element of the kept prefix whose running w-sum exceeds r.
 * Returns 0, or -1 for a top_k outside the supported range. */
int orc_random_sample(int64_t *out_idx, const void *logits, size_t rows, size_t V, int dtype,
                      float temperature, int64_t top_k, float top_p, uint64_t seed);
/* 2^t for t <= 0 as the sampler computes it: degree-7 Taylor polynomial of e^(g ln 2) on
 * g = frac(t) - 1/2, times sqrt(2), scaled by 2^floor(t); 0 below 2^-126. */
float orc_sample_exp2(float t);
uint64_t orc_splitmix64(uint64_t x);

#endif
