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

// ---- row absmax on the packed elements -----------------------------------------------
// For non-NaN values |x| orders like the integer value of its magnitude bits, so the row
// maximum is an integer max over (bits & ~sign) -- one packed-u16 max per two bf16 / f16
// elements, no unpacking.  A NaN's magnitude bits exceed the infinity pattern; a row
// whose integer maximum does so holds a NaN; its kernel recomputes amax with the float
// rule ("a NaN never raises it").

typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));

template <typename T>
struct AbsBits;

template <>
struct AbsBits<F32> {
    static constexpr uint32_t kInf = 0x7F800000u;
    __device__ static uint32_t fold(uint32_t m, const v4u &r) {
        const uint32_t a = max(r.x & 0x7FFFFFFFu, r.y & 0x7FFFFFFFu);
        const uint32_t b = max(r.z & 0x7FFFFFFFu, r.w & 0x7FFFFFFFu);
        return max(m, max(a, b));
    }
    __device__ static uint32_t finish(uint32_t m) { return m; }
    __device__ static float value(uint32_t m) { return __uint_as_float(m); }
};

template <uint32_t kInfBits, typename Cvt>
struct AbsBits16 {
    static constexpr uint32_t kInf = kInfBits;
    // m: two running 16-bit maxima (even / odd elements)
    __device__ static uint32_t fold(uint32_t m, const v4u &r) {
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
        v2u16 acc = __builtin_bit_cast(v2u16, m);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            acc = __builtin_elementwise_max(acc, __builtin_bit_cast(v2u16, w[k] & 0x7FFF7FFFu));
        return __builtin_bit_cast(uint32_t, acc);
    }
    __device__ static uint32_t finish(uint32_t m) { return max(m & 0xFFFFu, m >> 16); }
    __device__ static float value(uint32_t m) { return Cvt::widen(m); }
};

template <>
struct AbsBits<BF16> : AbsBits16<0x7F80u, Bf16Cvt> {};
template <>
struct AbsBits<F16> : AbsBits16<0x7C00u, F16Cvt> {};

struct MaxU32Op {
    __device__ static uint32_t apply(uint32_t a, uint32_t b) { return max(a, b); }
};

// ---- codes -----------------------------------------------------------------------------
// q needs the correctly rounded quotient x / s.  With r = RN(1 / s), q0 = RN(x r),
// e = fma(-q0, s, x) and q1 = fma(e, r, q0), q1 == RN(x / s): the final step of
// Markstein's division (IA-64), valid while nothing under- or overflows -- here for every
// row with s >= 2^-96.  Checked exhaustively for bf16 and f16 data (every amax, every
// |x| <= amax: 2.05e9 pairs) and on 5.1e8 random and near-tie f32 pairs against IEEE
// division: no code differs.  Rows with a smaller scale (including the all-zero row) use
// the IEEE quotient.  rint and the clamp then come from one add: q1 + 1.5 * 2^23 rounds
// to an integer half-to-even and leaves q1's integer in the low bits of the sum's
// mantissa (|q1| <= 127 (1 + 2^-23) < 127.5, so the clamp never acts); the code is the
// sum's low byte.  A NaN quotient from bf16 / f16 data (a NaN x, or x = inf with
// amax = inf) carries zero low bits, so its low byte is already code 0; f32 data checks.
struct RowQuantizer {
    float amax, scale, recip;
    bool exact_only;
    __device__ explicit RowQuantizer(float a) : amax(a), scale(a / 127.0f) {
        recip = 1.0f / scale;
        exact_only = !(scale >= 0x1p-96f);
    }
    // c[e]: the code in the low byte (upper bits arbitrary); rows with exact_only set must
    // use codes() or codeOf instead
    template <int N, bool kCheckNaN>
    __device__ __forceinline__ void fastCodes(const float *x, uint32_t *c) const {
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float q0 = x[e] * recip;
            const float err = __builtin_fmaf(-q0, scale, x[e]);
            const float q1 = __builtin_fmaf(err, recip, q0);
            const uint32_t m = __float_as_uint(q1 + 12582912.0f);
            c[e] = kCheckNaN && q1 != q1 ? 0u : m;
        }
    }
    template <int N, bool kCheckNaN>
    __device__ __forceinline__ void codes(const float *x, uint32_t *c) const {
        if (__builtin_expect(exact_only, 0)) {
#pragma unroll
            for (int e = 0; e < N; ++e) c[e] = codeOf(x[e], amax, scale);
            return;
        }
        fastCodes<N, kCheckNaN>(x, c);
    }
};

// Low bytes of c[0..3] as one word.
__device__ __forceinline__ uint32_t packCodes4(const uint32_t *c) {
    const uint32_t lo = __builtin_amdgcn_perm(c[1], c[0], 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(c[3], c[2], 0x0c0c0400u);
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

template <int N>
__device__ __forceinline__ void storeCodes(int8_t *q, size_t i, const uint32_t *c) {
    if constexpr (N == 8) {
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        const v2u r{packCodes4(c), packCodes4(c + 4)};
        __builtin_nontemporal_store(r, reinterpret_cast<v2u *>(q + i));
    } else {
        __builtin_nontemporal_store(packCodes4(c), reinterpret_cast<uint32_t *>(q + i));
    }
}

} // namespace llaisys::kernels
