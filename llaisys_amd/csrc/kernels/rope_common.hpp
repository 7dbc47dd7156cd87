// Pieces shared by the RoPE kernels (rope.hip, rope_kv.hip): the host-side frequency table
// and the cross-lane partner exchange.
#pragma once

#include "common.hpp"
#include "sincos.hpp"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <type_traits>

namespace llaisys::kernels::rope_detail {

constexpr int kMaxHalf = 128;   // head_dim <= 256 uses the host frequency table
constexpr int kLdsPairs = 1024; // (cos, sin) doubles staged per block: 16 KB

struct FreqTable {
    double f[kMaxHalf];
};

__device__ __forceinline__ double freqOf(const FreqTable &ft, int j, int d, float theta) {
    if (j < kMaxHalf) return ft.f[j];
    return 1.0 / pow(double(theta), double(2.0f * float(j) / float(d)));
}

// Tokens per 256-thread block for items_per_token 16-byte items, at most 1024 items and
// kLdsPairs (cos, sin) pairs: the fewest tokens that give >= 384 items (1.5+ per lane)
// with >= 85 % of the lanes' item slots busy, else the count with the most slots busy.
// Measured on MI355X (bf16, head_dim 128): q+k of Qwen2 (224 items / token) 2 tokens,
// 13.4 us vs 14.4 with 1 and 14.1 with 4; q alone (192) 4 tokens, 12.0 us vs 12.9 with
// 1; the fused q+k+v (256) 2 tokens, 5.7 us vs 5.9 with 1 and 6.5 with 4 (2048 tokens);
// Llama-8B q+k (640) stays at 1.  A block of 128 threads (2 items per lane, 1 token) ran
// 16 % slower than 2 tokens on 256 threads.
inline size_t tokensPerBlock(size_t per_tok, size_t half, int max_items) {
    const size_t cap = std::min(size_t(max_items) / per_tok, size_t(kLdsPairs) / half);
    size_t best = 1, best_busy = 0; // busy: per mille of slots
    for (size_t t = 1; t <= cap; ++t) {
        const size_t items = t * per_tok, slots = (items + 255) / 256 * 256;
        const size_t busy = items * 1000 / slots;
        if (items >= 384 && busy >= 850) return t;
        if (busy > best_busy) best = t, best_busy = busy;
    }
    return best;
}

// Device library sincos, out of line: its registers then count only on the rare path
// that calls it, not against the kernels' common path.
static __device__ __attribute__((noinline)) void librarySinCos(double ang, double *s, double *c) {
    sincos(ang, s, c);
}

// (cos, sin) of the block's ntok tokens x half frequencies into LDS (cs[t * half + j]),
// shared by every head of those tokens, in two calls:
//  * firstAngle(), before the kernel issues its 16-byte item loads, loads this thread's
//    first (position, frequency) pair.  Vector-memory loads complete in issue order, so
//    a pair loaded after the item loads could only be used once those had arrived too;
//    loaded first, the trig below runs while the item loads are still in flight.
//  * blockCosSin() computes the pairs.  The reduced-argument routine of sincos.hpp (within
//    an ulp of glibc) covers |angle| <= 2^30; an angle beyond flags the block, which then
//    recomputes those entries with the device library on a block-uniform path.  Every
//    thread of the block must call it (barriers); it ends with a barrier.
__device__ __forceinline__ double angleAt(const int64_t *pos, size_t t0, int i, int half,
                                          const FreqTable &ft) {
    return double(pos[t0 + i / half]) * ft.f[i % half];
}

struct AngleInputs {
    int64_t p;
    double f;
};

__device__ __forceinline__ AngleInputs firstAngle(const int64_t *pos, size_t t0, int ntok,
                                                  int half, const FreqTable &ft) {
    // unconditional (a clamped index for idle threads): a load under a branch would make
    // the compiler wait for every outstanding load, the item loads included, before use
    const int i = int(threadIdx.x) < ntok * half ? int(threadIdx.x) : 0;
    return AngleInputs{pos[t0 + i / half], ft.f[i % half]};
}

__device__ __forceinline__ void blockCosSin(double2 *cs, AngleInputs first, const int64_t *pos,
                                            size_t t0, int ntok, int half, const FreqTable &ft) {
    __shared__ int far_angle;
    if (threadIdx.x == 0) far_angle = 0;
    ldsBarrier(); // LDS only: the item loads the caller issued stay in flight
    bool far = false;
    for (int i = threadIdx.x; i < ntok * half; i += blockDim.x) {
        const double ang =
            i == int(threadIdx.x) ? double(first.p) * first.f : angleAt(pos, t0, i, half, ft);
        double sn = 0.0, c = 0.0;
        if (fabs(ang) <= kSincosFastLimit)
            sincosReduced(ang, &sn, &c);
        else
            far = true; // also NaN
        cs[i] = make_double2(c, sn);
    }
    if (far) far_angle = 1;
    ldsBarrier();
    if (__builtin_expect(far_angle != 0, 0)) {
        for (int i = threadIdx.x; i < ntok * half; i += blockDim.x) {
            const double ang = angleAt(pos, t0, i, half, ft);
            if (!(fabs(ang) <= kSincosFastLimit)) {
                double sn, c;
                librarySinCos(ang, &sn, &c);
                cs[i] = make_double2(c, sn);
            }
        }
        __syncthreads();
    }
}

// One angle (the scalar kernels).
__device__ __forceinline__ void angleSinCos(double ang, double *s, double *c) {
    if (fabs(ang) <= kSincosFastLimit)
        sincosReduced(ang, s, c);
    else
        librarySinCos(ang, s, c);
}

// Partner exchange: the vector VPH lanes away.  For VPH = 8 (bf16 / f16 with head_dim 128)
// the partner is in the same 16-lane DPP row, rotated by 8 (= lane ^ 8): a DPP move,
// no LDS traffic.  Other widths use a cross-lane shuffle.
template <int VPH>
__device__ __forceinline__ uint32_t partnerOf(uint32_t v) {
    if constexpr (VPH == 8)
        return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x128 /* row_ror:8 */, 0xF, 0xF, false));
    else
        return uint32_t(__shfl_xor(int(v), VPH, kWave));
}

// A chunk: 4 consecutive elements of one half of a head row, the unit of the half-pair
// layout (rope.hip's ropeHalves, rope_kv.hip): 8 bytes of bf16 / f16, 16 bytes of f32.
template <typename T, int E = 4>
struct Chunk4 {
    using F = Fmt<T>;
    static constexpr int kElems = E;
    static constexpr int kBytes = E * F::kBytes;
    static constexpr int kWords = kBytes / 4;
    typedef uint32_t V __attribute__((ext_vector_type(kWords)));
    __device__ static V load(const char *p) { return __builtin_nontemporal_load(reinterpret_cast<const V *>(p)); }
    __device__ static void store(char *p, const V &v) { __builtin_nontemporal_store(v, reinterpret_cast<V *>(p)); }
    __device__ static void unpack(const V &v, float *f) {
        if constexpr (std::is_same_v<T, F32>) {
#pragma unroll
            for (int w = 0; w < kWords; ++w) f[w] = __uint_as_float(v[w]);
        } else {
            using Cvt = std::conditional_t<std::is_same_v<T, BF16>, Bf16Cvt, F16Cvt>;
#pragma unroll
            for (int w = 0; w < kWords; ++w) f[2 * w] = Cvt::widen(v[w] & 0xFFFFu), f[2 * w + 1] = Cvt::widen(v[w] >> 16);
        }
    }
    __device__ static V packQ(const float *f) {
        V v;
        if constexpr (std::is_same_v<T, F32>) {
#pragma unroll
            for (int w = 0; w < kWords; ++w) v[w] = __float_as_uint(f[w]);
        } else {
            using Cvt = std::conditional_t<std::is_same_v<T, BF16>, Bf16Cvt, F16Cvt>;
#pragma unroll
            for (int w = 0; w < kWords; ++w) v[w] = Cvt::narrow2Q(f[2 * w], f[2 * w + 1]);
        }
        return v;
    }
};

// The reference's rotation of one pair (rope_cpu.cpp:38-41): both products rounded in f64,
// then their sum, then the rounding to float.  Compiled with -ffp-contract=off, so no
// product is fused into the sum.
__device__ __forceinline__ void rotatePair(float a, float b, double c, double s, float &out_a,
                                           float &out_b) {
    const double A = double(a), B = double(b);
    out_a = float(A * c - B * s);
    out_b = float(B * c + A * s);
}

inline FreqTable hostFreqs(size_t d, float theta) {
    FreqTable ft{};
    for (size_t j = 0; j < d / 2 && j < size_t(kMaxHalf); ++j) {
        // Same expression and libm call as rope_cpu.cpp:31.
        const float ex = 2.0f * float(j) / float(d);
        ft.f[j] = 1.0 / std::pow(double(theta), double(ex));
    }
    return ft;
}

} // namespace llaisys::kernels::rope_detail
