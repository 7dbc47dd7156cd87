// INT8 code arithmetic shared by the quantize, KV-append and fused RoPE + KV-append
// kernels.  Rule (no reference kernel exists; oracle/oracle.c states the same rule): per
// row, amax = max|x| in f32 (a NaN never raises it), scale = amax / 127.0f,
// q = clamp(rint(x / scale), -127, 127) with the IEEE quotient and round-half-even, and
// q = 0 for an all-zero row or a NaN quotient.
#pragma once

#include "common.hpp"

namespace llaisys::kernels {

__device__ __forceinline__ uint32_t codeOf(float x, float amax, float scale) {
    if (amax == 0.0f) return 0;
    float t = x / scale;
    if (t != t) return 0;
    t = rintf(t);
    t = t > 127.0f ? 127.0f : (t < -127.0f ? -127.0f : t);
    return uint32_t(int32_t(t)) & 0xFFu;
}

// Codes of one 16-byte vector of a row.  q = clamp(rint(x / s), -127, 127) needs the
// correctly rounded quotient only to decide which side of a half-integer it falls on, so
// the common path multiplies by r = 1/s (both IEEE, once per row) and rounds:
//  * |x| <= 127 s, so |x*r - x/s| <= 127 (2^-24 + 2^-24 + 2^-48) < 1.52e-5 and the
//    correctly rounded x/s is within another 127 * 2^-25 < 3.8e-6 of x/s: together
//    < 1.9e-5 < 2^-15, so when x*r is farther than 2^-15 from every half-integer both
//    quotients round to the same integer (and the clamp is a no-op: |x*r| <= 127.00001);
//  * when s is a power of two, x*r == x/s exactly, so x*r is always right;
//  * x = +-amax/2 lands within 63.5 * 2^-24 of the tie 63.5 in every row: its code is
//    computed once per row with the IEEE quotient;
//  * anything else near a half-integer (random near-ties, ~6e-5 of the elements) or NaN
//    redoes the vector with IEEE quotients.
// 16-bit data makes exact ties common (a row whose amax has mantissa 127 has a power-of-two
// scale, and x = amax/2 recurs in most rows): handling them without the IEEE path took the
// quantizer from a divergent slow path on ~60 % of wavefront-vectors to ~3 %.
struct RowQuantizer {
    float amax, scale, recip, half;
    uint32_t half_code;
    bool pow2, exact_only;
    __device__ explicit RowQuantizer(float a) : amax(a), scale(a / 127.0f) {
        recip = 1.0f / scale;
        exact_only = !(scale >= 0x1p-120f);
        pow2 = (__float_as_uint(scale) & 0x7FFFFFu) == 0;
        half = a * 0.5f;
        half_code = codeOf(half, amax, scale);
    }
    template <int N>
    __device__ __forceinline__ void codes(const float *x, uint32_t *c) const {
        bool slow = exact_only;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float t = x[e] * recip;
            const float q = rintf(t);
            const bool is_half = fabsf(x[e]) == half;
            const bool near = !(fabsf(t - q) < 0.5f - 0x1p-15f); // also true for NaN
            slow |= near && !is_half && !(pow2 && t == t);
            const uint32_t hc = x[e] < 0.0f ? (0u - half_code) : half_code;
            c[e] = (is_half ? hc : uint32_t(int32_t(q))) & 0xFFu;
        }
        if (__builtin_expect(slow, 0)) {
#pragma unroll
            for (int e = 0; e < N; ++e) c[e] = codeOf(x[e], amax, scale);
        }
    }
};

template <int N>
__device__ __forceinline__ void storeCodes(int8_t *q, size_t i, const uint32_t *c) {
    if constexpr (N == 8) {
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        const v2u r{c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24),
                    c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24)};
        __builtin_nontemporal_store(r, reinterpret_cast<v2u *>(q + i));
    } else {
        __builtin_nontemporal_store(c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24),
                                    reinterpret_cast<uint32_t *>(q + i));
    }
}

} // namespace llaisys::kernels
