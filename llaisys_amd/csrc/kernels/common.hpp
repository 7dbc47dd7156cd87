// Device helpers shared by the gfx950 kernels.
//
// Element formats are handled as 16-byte vectors (one global_load_dwordx4 per lane):
// 4 x f32, 8 x bf16 or 8 x f16.  Arithmetic is always f32 (f64 for RoPE).  The 16-bit
// conversions reproduce the reference's rules bit for bit (src/utils/types.cpp:6-84):
// bf16 rounds half to even through "+0x7FFF + lsb" with no NaN special case, f16
// truncates.  The hardware converters are not used because they differ on NaN inputs
// (bf16, f16) and round instead of truncating (f16).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace llaisys::kernels {

constexpr int kWave = 64;

// 16 bytes as a native vector (non-temporal builtins need a clang vector type).
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// ---- scalar conversions ---------------------------------------------------------------

__device__ __forceinline__ float bf16ToF32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint32_t f32ToBf16(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float f16ToF32(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    if (e == 0x1Fu) return __uint_as_float(sign | 0x7F800000u | (m << 13));
    if (e != 0) return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
    // zero or subnormal: value is m * 2^-24, exact in f32
    return __uint_as_float(sign | __float_as_uint(float(m) * 5.9604644775390625e-8f));
}

__device__ __forceinline__ uint32_t f32ToF16(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int e = int((u >> 23) & 0xFFu) - 127;
    uint32_t m = u & 0x7FFFFFu;
    if (e >= 16) return sign | ((e == 128 && m) ? 0x7E00u : 0x7C00u);
    if (e >= -14) return sign | (uint32_t(e + 15) << 10) | (m >> 13);
    if (e >= -24) return sign | (((m | 0x800000u) >> (-14 - e)) >> 13);
    return sign;
}

// ---- element formats --------------------------------------------------------------------

struct F32 {};
struct BF16 {};
struct F16 {};

template <typename T>
struct Fmt;

template <>
struct Fmt<F32> {
    static constexpr int kBytes = 4;
    static constexpr int kVec = 4; // elements per 16-byte vector
    __device__ static float get(const void *p, size_t i) { return static_cast<const float *>(p)[i]; }
    __device__ static void put(void *p, size_t i, float v) { static_cast<float *>(p)[i] = v; }
    __device__ static float round(float v) { return v; }
    __device__ static void unpack(const v4u &r, float *f) {
        f[0] = __uint_as_float(r.x);
        f[1] = __uint_as_float(r.y);
        f[2] = __uint_as_float(r.z);
        f[3] = __uint_as_float(r.w);
    }
    __device__ static v4u pack(const float *f) {
        return v4u{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                   __float_as_uint(f[3])};
    }
};

template <typename Cvt>
struct Half16 {
    static constexpr int kBytes = 2;
    static constexpr int kVec = 8;
    __device__ static float get(const void *p, size_t i) {
        return Cvt::widen(static_cast<const uint16_t *>(p)[i]);
    }
    __device__ static void put(void *p, size_t i, float v) {
        static_cast<uint16_t *>(p)[i] = uint16_t(Cvt::narrow(v));
    }
    __device__ static float round(float v) { return Cvt::widen(Cvt::narrow(v)); }
    __device__ static void unpack(const v4u &r, float *f) {
        const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            f[2 * k] = Cvt::widen(w[k] & 0xFFFFu);
            f[2 * k + 1] = Cvt::widen(w[k] >> 16);
        }
    }
    __device__ static v4u pack(const float *f) {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = Cvt::narrow(f[2 * k]) | (Cvt::narrow(f[2 * k + 1]) << 16);
        return v4u{w[0], w[1], w[2], w[3]};
    }
};

struct Bf16Cvt {
    __device__ static float widen(uint32_t b) { return bf16ToF32(b); }
    __device__ static uint32_t narrow(float f) { return f32ToBf16(f); }
};
struct F16Cvt {
    __device__ static float widen(uint32_t h) { return f16ToF32(h); }
    __device__ static uint32_t narrow(float f) { return f32ToF16(f); }
};

template <>
struct Fmt<BF16> : Half16<Bf16Cvt> {};
template <>
struct Fmt<F16> : Half16<F16Cvt> {};

// ---- 16-byte global access (element offsets) ----------------------------------------
// load16 / store16 are ordinary accesses, for data that is reused (norm weights, tables
// that stay hot).  The *Stream variants are non-temporal: data read once or written once
// streams past the caches instead of evicting reused lines, which measured 5-10 % faster
// on MI355X for every pure streaming pattern.

template <typename T>
__device__ __forceinline__ v4u load16(const void *base, size_t elem) {
    return *reinterpret_cast<const v4u *>(static_cast<const char *>(base) + elem * Fmt<T>::kBytes);
}

template <typename T>
__device__ __forceinline__ void store16(void *base, size_t elem, const v4u &v) {
    *reinterpret_cast<v4u *>(static_cast<char *>(base) + elem * Fmt<T>::kBytes) = v;
}

template <typename T>
__device__ __forceinline__ v4u load16Stream(const void *base, size_t elem) {
    return __builtin_nontemporal_load(
        reinterpret_cast<const v4u *>(static_cast<const char *>(base) + elem * Fmt<T>::kBytes));
}

template <typename T>
__device__ __forceinline__ void store16Stream(void *base, size_t elem, const v4u &v) {
    __builtin_nontemporal_store(v, reinterpret_cast<v4u *>(static_cast<char *>(base) + elem * Fmt<T>::kBytes));
}

// ---- reductions over a group of G consecutive lanes ------------------------------------
// G <= 64: butterfly inside the wavefront.  G > 64: butterfly per wave, then the G/64
// wave partials of the group are combined in a fixed order through LDS (`red` holds one
// slot per wave of the block).  Every thread of the block must call these (barriers).

struct SumOp {
    __device__ static float apply(float a, float b) { return a + b; }
};
// Max that never lets a NaN win (a NaN operand is dropped), matching "if (a > m) m = a".
struct MaxOp {
    __device__ static float apply(float a, float b) { return b > a ? b : a; }
};

template <int G, typename Op>
__device__ __forceinline__ float groupReduce(float v, float *red) {
    constexpr int kSteps = G < kWave ? G : kWave;
#pragma unroll
    for (int m = kSteps / 2; m > 0; m >>= 1) v = Op::apply(v, __shfl_xor(v, m, kWave));
    if constexpr (G > kWave) {
        const int wave = threadIdx.x / kWave;
        if (threadIdx.x % kWave == 0) red[wave] = v;
        __syncthreads();
        const int first = (threadIdx.x / G) * (G / kWave);
        v = red[first];
#pragma unroll
        for (int k = 1; k < G / kWave; ++k) v = Op::apply(v, red[first + k]);
        __syncthreads();
    }
    return v;
}

} // namespace llaisys::kernels
