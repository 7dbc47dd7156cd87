/*
 * CPU oracle for the LLAISYS per-layer ops -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates, in plain C, the arithmetic of the reference CPU kernels so that the HIP
 * kernels of llaisys_amd can be checked against it on identical inputs.  Every function
 * names the reference file:line it follows (paths relative to the reference checkout).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this file.
 *
 * Build: gcc -std=c11 -O3 -ffp-contract=off (oracle/Makefile).  ISO mode plus
 * -ffp-contract=off keeps every multiply and add separately rounded, as in the
 * reference's g++ -std=c++17 build on x86-64.
 *
 * Pinning (tests/test_oracle.py): rms_norm, rope, swiglu, add, embedding, argmax,
 * self_attention and the bf16/f16 conversions are compared bit-for-bit with golden vectors
 * written by the compiled reference library (tests/golden/) and with that library on
 * random shapes; self_attention also against a textbook f64 evaluation and closed forms
 * (one key, equal keys, causality, the GQA head mapping); the INT8 functions and the fused
 * add+rms_norm have no reference counterpart and are pinned by closed-form checks
 * (codes of exact scale multiples, +-127 at the row's absmax, round-half-even ties,
 * zero rows, and add+rms_norm == add then rms_norm of the reference goldens).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- scalar conversions: src/utils/types.cpp:6-84 ---------------------------------- */

/* bf16 -> f32 widens by 16 bits (types.cpp:66-72). */
float orc_bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* f32 -> bf16 rounds half to even by adding 0x7FFF plus the kept LSB, with no NaN
 * special case (types.cpp:74-84). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t lsb = (u >> 16) & 1u;
    return (uint16_t)((u + 0x7FFFu + lsb) >> 16);
}

/* f16 -> f32, exact including subnormals (types.cpp:6-38). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int32_t e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FFu;
    uint32_t u;
    if (e == 31) {
        u = sign | 0x7F800000u | (m << 13);
    } else if (e == 0) {
        if (m == 0) {
            u = sign;
        } else {
            /* normalise the subnormal: value = m * 2^-24 */
            int32_t ex = -14;
            while (!(m & 0x400u)) {
                m <<= 1;
                ex -= 1;
            }
            u = sign | ((uint32_t)(ex + 127) << 23) | ((m & 0x3FFu) << 13);
        }
    } else {
        u = sign | ((uint32_t)(e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* f32 -> f16 TRUNCATES the mantissa; |x| >= 2^16 becomes inf, NaN becomes 0x7E00
 * (types.cpp:40-64). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    int32_t e = (int32_t)((u >> 23) & 0xFFu) - 127;
    uint32_t m = u & 0x7FFFFFu;
    if (e >= 16) {
        if (e == 128 && m != 0) return (uint16_t)(sign | 0x7E00u);
        return (uint16_t)(sign | 0x7C00u);
    }
    if (e >= -14) return (uint16_t)(sign | ((uint32_t)(e + 15) << 10) | (m >> 13));
    if (e >= -24) {
        m |= 0x800000u;
        m >>= (uint32_t)(-14 - e);
        return (uint16_t)(sign | (m >> 13));
    }
    return sign;
}

/* element load / store in the reference's cast<> semantics (types.hpp:116-139) */
static inline float ld(const void *p, size_t i, int dt) {
    switch (dt) {
    case ORC_F32: return ((const float *)p)[i];
    case ORC_BF16: return orc_bf16_to_f32(((const uint16_t *)p)[i]);
    default: return orc_f16_to_f32(((const uint16_t *)p)[i]);
    }
}

static inline void st(void *p, size_t i, int dt, float v) {
    switch (dt) {
    case ORC_F32: ((float *)p)[i] = v; break;
    case ORC_BF16: ((uint16_t *)p)[i] = orc_f32_to_bf16(v); break;
    default: ((uint16_t *)p)[i] = orc_f32_to_f16(v); break;
    }
}

static inline size_t esize(int dt) { return dt == ORC_F32 ? 4 : 2; }

/* ---- add: src/ops/add/cpu/add_cpu.cpp:7-17 ------------------------------------------ */
/* f32 adds natively; half types widen, add in f32 and round back. */
void orc_add(void *c, const void *a, const void *b, size_t n, int dt) {
    for (size_t i = 0; i < n; i++) st(c, i, dt, ld(a, i, dt) + ld(b, i, dt));
}

/* ---- rms_norm: src/ops/rms_norm/cpu/rms_norm_cpu.cpp:6-35 --------------------------- */
/* Per row: sequential f32 sum of squares; rms = sqrtf(sum / cols + eps); inv = 1 / rms;
 * y = (x * w) * inv rounded to the element type. */
static void rms_row(void *out, size_t ro, const void *in, size_t ri, const void *w,
                    size_t cols, float eps, int dt) {
    float s = 0.0f;
    for (size_t j = 0; j < cols; j++) {
        float x = ld(in, ri + j, dt);
        s += x * x;
    }
    float rms = sqrtf(s / (float)cols + eps);
    float inv = 1.0f / rms;
    for (size_t j = 0; j < cols; j++) {
        float x = ld(in, ri + j, dt);
        float wv = ld(w, j, dt);
        st(out, ro + j, dt, x * wv * inv);
    }
}

void orc_rms_norm(void *out, const void *in, const void *w, size_t rows, size_t cols,
                  float eps, int dt) {
    for (size_t r = 0; r < rows; r++) rms_row(out, r * cols, in, r * cols, w, cols, eps, dt);
}

/* ---- fused residual add + rms_norm (no reference kernel) ----------------------------- */
/* Composition of the reference decoder-layer call sequence (src/models/qwen2/layer.hpp:
 * 60-71): h = add(x, r) rounded to the element type (add_cpu.cpp:12), residual_out = h,
 * out = rms_norm(h). */
void orc_add_rms_norm(void *out, void *res_out, const void *in, const void *res,
                      const void *w, size_t rows, size_t cols, float eps, int dt) {
    orc_add(res_out, in, res, rows * cols, dt);
    orc_rms_norm(out, res_out, w, rows, cols, eps, dt);
}

/* ---- rope: src/ops/rope/cpu/rope_cpu.cpp:6-49 ---------------------------------------- */
/* exponent = 2.0f * j / head_dim in f32; freq = 1 / pow((double)theta, exponent) in
 * double; angle = (double)p * freq; cos/sin and the rotation of the pair (j, j + d/2)
 * in double; the result is rounded double -> float -> element type. */
void orc_rope(void *out, const void *in, const int64_t *pos, size_t seq, size_t nh,
              size_t d, float theta, int dt) {
    size_t half = d / 2;
    for (size_t i = 0; i < seq; i++) {
        int64_t p = pos[i];
        for (size_t h = 0; h < nh; h++) {
            size_t base = (i * nh + h) * d;
            for (size_t j = 0; j < half; j++) {
                float ex = 2.0f * (float)j / (float)d;
                double freq = 1.0 / pow((double)theta, (double)ex);
                double ang = (double)p * freq;
                double c = cos(ang), s = sin(ang);
                double a = (double)ld(in, base + j, dt);
                double b = (double)ld(in, base + j + half, dt);
                double ya = a * c - b * s;
                double yb = b * c + a * s;
                st(out, base + j, dt, (float)ya);
                st(out, base + j + half, dt, (float)yb);
            }
        }
    }
}

/* ---- swiglu: src/ops/swiglu/cpu/swiglu_cpu.cpp:6-22 ---------------------------------- */
/* out = u * (g / (1 + expf(-g))) in f32. */
void orc_swiglu(void *out, const void *gate, const void *up, size_t n, int dt) {
    for (size_t i = 0; i < n; i++) {
        float g = ld(gate, i, dt);
        float u = ld(up, i, dt);
        float silu = g / (1.0f + expf(-g));
        st(out, i, dt, u * silu);
    }
}

/* ---- embedding: src/ops/embedding/cpu/embedding_cpu.cpp:6-23 ------------------------- */
/* Row copy out[i] = weight[index[i]]; an id outside [0, vocab) stops with an error
 * after the rows before it were copied (embedding_cpu.cpp:18). */
int orc_embedding(void *out, const void *index, int idt, size_t n, const void *weight,
                  size_t vocab, size_t dim, int dt) {
    size_t row = dim * esize(dt);
    for (size_t i = 0; i < n; i++) {
        int64_t id = idt == ORC_I32 ? (int64_t)((const int32_t *)index)[i]
                                    : ((const int64_t *)index)[i];
        if (id < 0 || (uint64_t)id >= vocab) return -1;
        memcpy((char *)out + i * row, (const char *)weight + (size_t)id * row, row);
    }
    return 0;
}

/* ---- argmax: src/ops/argmax/cpu/argmax_cpu.cpp:9-28 ---------------------------------- */
/* Seed with element 0, replace only on a strictly greater f32 value: the first maximum
 * wins and a NaN never wins unless it is element 0.  max_val = T(f32 max). */
static void argmax_one(void *idx, int idt, size_t io, void *val, const void *v, size_t vo,
                       size_t n, int dt) {
    if (n == 0) return;
    size_t best = 0;
    float m = ld(v, vo, dt);
    for (size_t i = 1; i < n; i++) {
        float x = ld(v, vo + i, dt);
        if (x > m) {
            m = x;
            best = i;
        }
    }
    st(val, io, dt, m);
    if (idt == ORC_I32)
        ((int32_t *)idx)[io] = (int32_t)best;
    else if (idt == ORC_I64)
        ((int64_t *)idx)[io] = (int64_t)best;
}

void orc_argmax(void *idx, int idt, void *val, const void *vals, size_t n, int dt) {
    argmax_one(idx, idt, 0, val, vals, 0, n, dt);
}

/* Row-wise argmax: the reference argmax applied to each row slice of [rows, cols]. */
void orc_argmax_rows(void *idx, int idt, void *val, const void *vals, size_t rows,
                     size_t cols, int dt) {
    for (size_t r = 0; r < rows; r++) argmax_one(idx, idt, r, val, vals, r * cols, cols, dt);
}

/* ---- INT8 symmetric absmax quantization (no reference kernel) ------------------------ */
/* Rule, per row of `cols` elements:
 *   amax  = max |x| over the row in f32 (NaN elements never raise it)
 *   scale = amax / 127.0f                      (f32, correctly rounded division)
 *   q     = 0 if amax == 0 or x / scale is NaN,
 *           else clamp(rintf(x / scale), -127, 127)   (round half to even)
 * dequant: y = T(float(q) * scale) with the reference f32 -> T rounding. */
static void quant_row(int8_t *q, float *scale, const void *in, size_t off, size_t cols,
                      int dt) {
    float amax = 0.0f;
    for (size_t j = 0; j < cols; j++) {
        float a = fabsf(ld(in, off + j, dt));
        if (a > amax) amax = a;
    }
    float s = amax / 127.0f;
    *scale = s;
    for (size_t j = 0; j < cols; j++) {
        int8_t code = 0;
        if (amax != 0.0f) {
            float t = ld(in, off + j, dt) / s;
            if (t == t) {
                t = rintf(t);
                if (t > 127.0f) t = 127.0f;
                if (t < -127.0f) t = -127.0f;
                code = (int8_t)t;
            }
        }
        q[j] = code;
    }
}

void orc_quantize_int8(int8_t *q, float *scale, const void *in, size_t rows, size_t cols,
                       int dt) {
    for (size_t r = 0; r < rows; r++) quant_row(q + r * cols, scale + r, in, r * cols, cols, dt);
}

void orc_dequantize_int8(void *out, const int8_t *q, const float *scale, size_t rows,
                         size_t cols, int dt) {
    for (size_t r = 0; r < rows; r++)
        for (size_t j = 0; j < cols; j++)
            st(out, r * cols + j, dt, (float)q[r * cols + j] * scale[r]);
}

/* INT8 KV-cache append: quantizes kv [n_tok, n_kvh, head_dim] per (token, head) row and
 * writes codes to rows pos .. pos + n_tok of cache_q [max_seq, n_kvh, head_dim] and scales
 * to cache_scale [max_seq, n_kvh].  Replaces the f32 row copy of the reference decoder's
 * cache update (src/models/qwen2/attention.hpp:108-123). */
int orc_kv_append_int8(int8_t *cache_q, float *cache_scale, size_t max_seq, const void *kv,
                       size_t n_tok, size_t n_kvh, size_t d, size_t pos, int dt) {
    if (pos > max_seq || n_tok > max_seq - pos) return -1;
    size_t r0 = pos * n_kvh;
    orc_quantize_int8(cache_q + r0 * d, cache_scale + r0, kv, n_tok * n_kvh, d, dt);
    return 0;
}

/* ---- self_attention: src/ops/self_attention/cpu/self_attention_cpu.cpp:13-115 ---------
 * q [seq, nh, d], k [total, nkvh, d], v [total, nkvh, dv], out [seq, nh, dv], nh a
 * multiple of nkvh; q head h reads kv head h / (nh / nkvh).  Per (head, query):
 * scores[t] = (sequential f32 sum of q*k) * scale (:76-92); the query sits at
 * current_pos = total - seq + i in size_t arithmetic (:95, so seq > total wraps and masks
 * nothing); keys t > current_pos get -inf, max over all scores (:101-108); -inf scores
 * become 0, the rest expf(s - max), summed left to right (:110-118); each divided by the
 * sum (:120-122); out[dv] = sequential f32 sum of p * v, rounded to the element type
 * (:127-140).  Returns -1 (nothing written) on a zero nkvh or nh % nkvh != 0. */
int orc_self_attention(void *out, const void *q, const void *k, const void *v, size_t seq,
                       size_t total, size_t nh, size_t nkvh, size_t d, size_t dv, float scale,
                       int dt) {
    if (nkvh == 0 || nh % nkvh != 0) return -1;
    const size_t group = nh / nkvh;
    float *scores = (float *)malloc((total ? total : 1) * sizeof(float));
    if (!scores) return -1;
    for (size_t h = 0; h < nh; h++) {
        const size_t kvh = h / group;
        for (size_t i = 0; i < seq; i++) {
            const size_t qo = i * nh * d + h * d;
            for (size_t t = 0; t < total; t++) {
                const size_t ko = t * nkvh * d + kvh * d;
                float dot = 0.0f;
                for (size_t e = 0; e < d; e++) dot += ld(q, qo + e, dt) * ld(k, ko + e, dt);
                scores[t] = dot * scale;
            }
            const size_t cur = total - seq + i;
            float mx = -INFINITY;
            for (size_t t = 0; t < total; t++) {
                if (t > cur) scores[t] = -INFINITY;
                if (scores[t] > mx) mx = scores[t];
            }
            float sum = 0.0f;
            for (size_t t = 0; t < total; t++) {
                if (scores[t] == -INFINITY)
                    scores[t] = 0.0f;
                else
                    scores[t] = expf(scores[t] - mx);
                sum += scores[t];
            }
            for (size_t t = 0; t < total; t++) scores[t] /= sum;
            const size_t oo = i * nh * dv + h * dv;
            for (size_t e = 0; e < dv; e++) {
                float val = 0.0f;
                for (size_t t = 0; t < total; t++) val += scores[t] * ld(v, t * nkvh * dv + kvh * dv + e, dt);
                st(out, oo + e, dt, val);
            }
        }
    }
    free(scores);
    return 0;
}

/* ---- linear: src/ops/linear/cpu/linear_cpu.cpp:11-41 -------------------------------
 * out[m][n] = T(sum_k x[m][k] * w[n][k] (left to right, f32) + bias[n]) for x [rows, in],
 * w [out, in], bias [out] or NULL. */
void orc_linear(void *out, const void *x, const void *w, const void *bias, size_t rows,
                size_t in_f, size_t out_f, int dt) {
    for (size_t m = 0; m < rows; m++)
        for (size_t n = 0; n < out_f; n++) {
            float sum = 0.0f;
            for (size_t k = 0; k < in_f; k++) sum += ld(x, m * in_f + k, dt) * ld(w, n * in_f + k, dt);
            if (bias) sum += ld(bias, n, dt);
            st(out, m * out_f + n, dt, sum);
        }
}

/* W8A16 linear over INT8 weights (no reference kernel; the rule of llaisysLinearW8A16):
 * out[m][n] = T(scale[n] * (sum_k x[m][k] * code[n][k], left to right in f32) + bias[n]).
 * Each product of a bf16 / f16 activation and an INT8 code is exact in f32. */
void orc_linear_w8a16(void *out, const void *x, const int8_t *code, const float *scale,
                      const void *bias, size_t rows, size_t in_f, size_t out_f, int dt) {
    for (size_t m = 0; m < rows; m++)
        for (size_t n = 0; n < out_f; n++) {
            float sum = 0.0f;
            for (size_t k = 0; k < in_f; k++) sum += ld(x, m * in_f + k, dt) * (float)code[n * in_f + k];
            sum = scale[n] * sum;
            if (bias) sum += ld(bias, n, dt);
            st(out, m * out_f + n, dt, sum);
        }
}

/* ---- dtype conversion (the reference's cast<To>(From), types.hpp:116-139) -------------
 * Same type: the value itself (bit copy).  Otherwise through f32 with the rules above:
 * bf16 -> f32 and f16 -> f32 exact, f32 -> bf16 round-half-even by "+0x7FFF + lsb" with no
 * NaN case (types.cpp:74-84), f32 -> f16 truncating (types.cpp:55). */
void orc_cast(void *out, int out_dt, const void *in, int in_dt, size_t n) {
    const size_t es = in_dt == ORC_F32 ? 4 : 2;
    if (out_dt == in_dt) {
        memcpy(out, in, n * es);
        return;
    }
    for (size_t i = 0; i < n; i++) st(out, i, out_dt, ld(in, i, in_dt));
}

/* ---- random sampling (no reference kernel; rule in oracle.h) ------------------------- */

uint64_t orc_splitmix64(uint64_t x) {
    /* splitmix64 finaliser (Steele, Lea and Flood, "Fast splittable pseudorandom number
     * generators", OOPSLA 2014) applied to x + golden gamma */
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

float orc_sample_exp2(float t) {
    if (!(t > -126.0f)) return 0.0f;
    const float n = floorf(t);
    const float g = (t - n) - 0.5f;
    /* (ln 2)^k / k!, k = 7 .. 1 */
    float y = 1.525273380405984e-05f;
    y = y * g + 0.00015403530393381608f;
    y = y * g + 0.0013333558146428443f;
    y = y * g + 0.009618129107628477f;
    y = y * g + 0.05550410866482158f;
    y = y * g + 0.2402265069591007f;
    y = y * g + 0.6931471805599453f;
    y = y * g + 1.0f;
    return ldexpf(y * 1.4142135623730951f, (int)n);
}

/* a NaN z (either sign) takes the key of -inf: never preferred to a number */
static uint32_t smp_key(float z) {
    uint32_t b;
    if (z != z) z = -INFINITY;
    memcpy(&b, &z, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static float smp_unkey(uint32_t k) {
    const uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    float z;
    memcpy(&z, &b, 4);
    return z;
}

typedef struct {
    uint32_t key;
    uint32_t idx;
} smp_item;

static int smp_cmp(const void *a, const void *b) {
    const smp_item *x = a, *y = b;
    if (x->key != y->key) return x->key > y->key ? -1 : 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

int orc_random_sample(int64_t *out_idx, const void *logits, size_t rows, size_t V, int dt,
                      float temperature, int64_t top_k, float top_p, uint64_t seed) {
    if (!(temperature > 0.0f) || top_k == 1) {
        for (size_t r = 0; r < rows; r++) {
            float m = ld(logits, r * V, dt);
            size_t mi = 0;
            for (size_t i = 1; i < V; i++) {
                const float v = ld(logits, r * V + i, dt);
                if (v > m) { m = v; mi = i; }
            }
            out_idx[r] = (int64_t)mi;
        }
        return 0;
    }
    if (top_k < 2 || top_k > 1024) return -1;
    const float inv = 1.0f / temperature;
    const size_t k = (size_t)top_k < V ? (size_t)top_k : V;
    smp_item *it = malloc(V * sizeof(smp_item));
    uint64_t *cum = malloc(k * sizeof(uint64_t));
    uint32_t *w = malloc(k * sizeof(uint32_t));
    for (size_t r = 0; r < rows; r++) {
        for (size_t i = 0; i < V; i++) {
            it[i].key = smp_key(ld(logits, r * V + i, dt) * inv);
            it[i].idx = (uint32_t)i;
        }
        qsort(it, V, sizeof(smp_item), smp_cmp);
        const float zmax = smp_unkey(it[0].key);
        uint64_t W = 0;
        for (size_t j = 0; j < k; j++) {
            /* (z - zmax) is 0 for candidates tied with the top key, infinite ties included */
            const float p = it[j].key == it[0].key
                                ? orc_sample_exp2(0.0f)
                                : orc_sample_exp2((smp_unkey(it[j].key) - zmax) * 1.4426950408889634f);
            w[j] = (uint32_t)(p * 2147483648.0f);
            W += w[j];
            cum[j] = W;
        }
        size_t kept = k;
        if (top_p < 1.0f) {
            uint64_t target = 1;
            if (top_p > 0.0f) {
                target = (uint64_t)((double)top_p * (double)W);
                if (target == 0) target = 1;
            }
            kept = 0;
            while (cum[kept] < target) kept++;
            kept++;
        }
        const uint64_t Wk = cum[kept - 1];
        const uint64_t u24 = orc_splitmix64(seed + r) >> 40;
        const unsigned __int128 prod = (unsigned __int128)u24 * Wk;
        const uint64_t rr = (uint64_t)(prod >> 24);
        size_t j = 0;
        while (cum[j] <= rr) j++;
        out_idx[r] = (int64_t)it[j].idx;
    }
    free(it);
    free(cum);
    free(w);
    return 0;
}
