// Device helpers shared by the gfx950 kernels.
//
// Element formats are handled as 16-byte vectors (one global_load_dwordx4 per lane):
// 4 x f32, 8 x bf16 or 8 x f16.  Arithmetic is always f32 (f64 for RoPE).  The 16-bit
// conversions reproduce the reference's rules bit for bit (src/utils/types.cpp:6-84):
// bf16 rounds half to even through "+0x7FFF + lsb" with no NaN special case, f16
// truncates.  `pack` applies these rules to any f32.  `packQ` may use gfx950's
// v_cvt_pk_bf16_f32 (one instruction per two elements instead of five): compared over all
// 2^32 f32 inputs on MI355X it equals the reference rule for every non-NaN value and for
// every quiet NaN whose low 16 bits are zero, and differs only for signalling NaNs and NaN
// payloads in the low 16 bits (it quiets and truncates them).  Every f32 that a kernel
// computes by arithmetic from bf16 / f16 inputs is in the first class (a NaN result is
// quiet and carries an input's payload or the default NaN), so kernels use packQ unless
// an f32 operand supplied by the caller (eps, theta, a dequantization scale) is a NaN.
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
    __device__ static v4u packQ(const float *f) { return pack(f); }
    static constexpr uint32_t kSignBits = 0x80000000u; // sign bits of the elements in a word
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
    __device__ static v4u packQ(const float *f) {
        return v4u{Cvt::narrow2Q(f[0], f[1]), Cvt::narrow2Q(f[2], f[3]), Cvt::narrow2Q(f[4], f[5]),
                   Cvt::narrow2Q(f[6], f[7])};
    }
    static constexpr uint32_t kSignBits = 0x80008000u;
};

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

struct Bf16Cvt {
    __device__ static float widen(uint32_t b) { return bf16ToF32(b); }
    __device__ static uint32_t narrow(float f) { return f32ToBf16(f); }
    // two elements, (lo, hi), by v_cvt_pk_bf16_f32 (see packQ above)
    __device__ static uint32_t narrow2Q(float lo, float hi) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v2f{lo, hi}, v2bf));
    }
};
struct F16Cvt {
    __device__ static float widen(uint32_t h) { return f16ToF32(h); }
    __device__ static uint32_t narrow(float f) { return f32ToF16(f); }
    __device__ static uint32_t narrow2Q(float lo, float hi) { return narrow(lo) | (narrow(hi) << 16); }
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
// G <= 64: butterfly inside the wavefront without LDS: DPP quad permutes for distances 1
// and 2, row half-mirror and row mirror for 4 and 8 (equivalent to xor 4 / xor 8 once the
// smaller groups are uniform), v_permlane16_swap / v_permlane32_swap for 16 and 32.  Both
// lanes of a pair combine the same two values in the same order, so every lane of the
// group ends with the same bits.  G > 64: butterfly per wave, then the G/64 wave partials
// of the group are combined in a fixed order through LDS (`red` holds one slot per wave of
// the block).  Every thread of the block must call these (barriers).

struct SumOp {
    __device__ static float apply(float a, float b) { return a + b; }
};
// Max that never lets a NaN win (a NaN operand is dropped), matching "if (a > m) m = a".
struct MaxOp {
    __device__ static float apply(float a, float b) { return b > a ? b : a; }
};

template <int M, typename Op, typename V>
__device__ __forceinline__ V butterflyStep(V v) {
    static_assert(sizeof(V) == 4, "32-bit values");
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    if constexpr (M <= 8) {
        constexpr int kCtrl = M == 1 ? 0xB1 : (M == 2 ? 0x4E : (M == 4 ? 0x141 : 0x140));
        const uint32_t p = uint32_t(__builtin_amdgcn_mov_dpp(int(u), kCtrl, 0xF, 0xF, false));
        // lo / hi: the pair's lower lane's value first in both lanes
        const bool lower = (threadIdx.x & (2 * M - 1)) < M;
        const V a = __builtin_bit_cast(V, lower ? u : p), b = __builtin_bit_cast(V, lower ? p : u);
        return Op::apply(a, b);
    } else {
        static_assert(M == 16 || M == 32, "distance");
        const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                               : __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return Op::apply(__builtin_bit_cast(V, uint32_t(r[0])), __builtin_bit_cast(V, uint32_t(r[1])));
    }
}

// Reduction over aligned groups of G <= 64 consecutive lanes; every lane gets the result.
template <int G, typename Op, typename V>
__device__ __forceinline__ V waveGroupReduce(V v) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8 || G == 16 || G == 32 || G == 64, "group");
    if constexpr (G >= 2) v = butterflyStep<1, Op>(v);
    if constexpr (G >= 4) v = butterflyStep<2, Op>(v);
    if constexpr (G >= 8) v = butterflyStep<4, Op>(v);
    if constexpr (G >= 16) v = butterflyStep<8, Op>(v);
    if constexpr (G >= 32) v = butterflyStep<16, Op>(v);
    if constexpr (G >= 64) v = butterflyStep<32, Op>(v);
    return v;
}

// Workgroup barrier for an LDS hand-off only: waits for this wave's LDS accesses, not for
// its global loads and stores.  __syncthreads() carries a workgroup fence, for which the
// compiler waits on every outstanding global access (s_waitcnt vmcnt(0), which on gfx9
// counts stores too) -- that would drain loads issued ahead of the barrier to overlap it.
__device__ __forceinline__ void ldsBarrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Wait until at most VM of this wave's vector-memory loads are outstanding.
template <int VM>
__device__ __forceinline__ void waitVmcnt() {
    // s_waitcnt fields: vmcnt [3:0] and [15:14], expcnt [6:4] (7: no wait), lgkmcnt [11:8] (15: no wait)
    __builtin_amdgcn_s_waitcnt((VM & 0xF) | (0x7 << 4) | (0xF << 8) | ((VM >> 4) << 14));
}

template <int G, typename Op, typename V>
__device__ __forceinline__ V groupReduce(V v, V *red) {
    v = waveGroupReduce<(G < kWave ? G : kWave), Op>(v);
    if constexpr (G > kWave) {
        const int wave = threadIdx.x / kWave;
        if (threadIdx.x % kWave == 0) red[wave] = v;
        ldsBarrier();
        const int first = (threadIdx.x / G) * (G / kWave);
        v = red[first];
#pragma unroll
        for (int k = 1; k < G / kWave; ++k) v = Op::apply(v, red[first + k]);
        ldsBarrier();
    }
    return v;
}

// swiglu of one element, reference src/ops/swiglu/cpu/swiglu_cpu.cpp:15-20: u * (g / (1 +
// exp(-g))) in f32.  g / d is g * rcp(d) plus one Newton correction; where 1 / d would be
// subnormal or zero it is the IEEE quotient.
struct SwigluOp {
    __device__ static float apply(float g, float u) {
        const float d = 1.0f + __expf(-g);
        float q;
        if (__builtin_expect(d < 0x1p126f, 1)) {
            const float r = __builtin_amdgcn_rcpf(d);
            q = g * r;
            q = __builtin_fmaf(__builtin_fmaf(-d, q, g), r, q);
        } else {
            q = g / d; // 1/d would be subnormal or 0: take the IEEE quotient
        }
        return u * q;
    }
};
} // namespace llaisys::kernels
