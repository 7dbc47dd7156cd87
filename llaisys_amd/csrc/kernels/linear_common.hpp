// Device pieces shared by the linear kernels (linear.hip) and the fused rms_norm -> linear
// kernels (norm_linear.hip).  Sharing them is what makes a fused kernel equal, bit for bit,
// to the separate launches it replaces: the same lanes sum the same products in the same
// order.
#pragma once

#include "common.hpp"

#include <type_traits>

namespace llaisys::kernels::lin {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

// 16 x 16 x 32: A[m = l % 16][k = 8 (l / 16) + j], B[k = 8 (l / 16) + j][n = l % 16],
// D[m = 4 (l / 16) + i][n = l % 16]
template <typename T>
__device__ __forceinline__ f32x4 mfma(const v4u &a, const v4u &b, f32x4 c) {
    if constexpr (std::is_same_v<T, BF16>)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 8 INT8 codes as 8 elements of T (exact: |code| <= 127 fits both 8- and 11-bit mantissas)
template <typename T>
__device__ __forceinline__ v4u codesToT(const v2u &c) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t src = e < 2 ? c.x : c.y;
        const int sh = 16 * (e % 2);
        const float lo = float(int8_t(src >> sh)), hi = float(int8_t(src >> (sh + 8)));
        if constexpr (std::is_same_v<T, BF16>)
            w[e] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u); // exact: 8-bit values
        else
            w[e] = f32ToF16(lo) | (f32ToF16(hi) << 16);
    }
    return v4u{w[0], w[1], w[2], w[3]};
}

// ---- few rows (M <= 16): the skinny MFMA loop ------------------------------------------
// A block owns 16 output channels and its nw waves split K into groups of 128 k.  A load
// instruction that hands MFMA operands straight to registers touches 16 weight rows (lane l
// holds row l % 16), which streams HBM measurably slower than touching 4 rows with 256
// contiguous bytes each; so each wave loads its group row-contiguously, transposes it
// through its own padded LDS tile (conflict-free on both sides) and reads the MFMA operand
// from there.  k order inside a group (A and B agree, so the MFMA sum covers every k once):
//   16-bit weights: step s, lane (r, g) holds k = 32 s + 8 g + [0, 8)
//   INT8 weights:   step s, lane (r, g) holds k = 64 (s / 2) + 16 g + 8 (s % 2) + [0, 8)
// (an INT8 lane reads 16 codes, two steps' worth, in one LDS read).
constexpr int kSkK = 128; // k per group
constexpr int skinnyPitch(bool int8) { return (int8 ? kSkK : 2 * kSkK) + 16; }

// k of step s of a group for the lane's 16-lane group g4 (see above)
template <bool kInt8>
__device__ __forceinline__ int skinnyK(int kg, int s, int g4) {
    return kg + (kInt8 ? 64 * (s / 2) + 16 * g4 + 8 * (s % 2) : 32 * s + 8 * g4);
}

// Shape of a group's row-contiguous weight loads: instruction j, lane l -> row j *
// kRowsPerLoad + l / kLanesPerRow, 16 bytes at column (l % kLanesPerRow).
template <bool kInt8>
struct SkinnyLoads {
    static constexpr int kRowB = kInt8 ? kSkK : 2 * kSkK; // bytes of one weight row in a group
    static constexpr int kLanesPerRow = kRowB / 16;        // lanes covering a row in one load
    static constexpr int kRowsPerLoad = kWave / kLanesPerRow;
    static constexpr int kLoads = 16 / kRowsPerLoad;       // loads per group and set: 4 (16-bit) / 2 (INT8)
    static constexpr int kElemB = kInt8 ? 1 : 2;
};

// The weight loads of group g for R sets of 16 rows (set r starts at row rows0[r]; rows
// past `nrows` read row nrows - 1; chunks past K read column 0 and are zeroed by the caller).
template <bool kInt8, int R>
__device__ __forceinline__ void skinnyLoad(v4u (&wl)[R][SkinnyLoads<kInt8>::kLoads], const char *wbase,
                                           const int (&rows0)[R], int nrows, int K, int g, int lane) {
    using S = SkinnyLoads<kInt8>;
    const int lrow = lane / S::kLanesPerRow, lcol = lane % S::kLanesPerRow;
    const int kw = g * kSkK + lcol * (16 / S::kElemB);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < S::kLoads; ++j) {
            const int row = min(rows0[r] + j * S::kRowsPerLoad + lrow, nrows - 1);
            wl[r][j] = *reinterpret_cast<const v4u *>(wbase + (size_t(row) * K + (kw < K ? kw : 0)) * S::kElemB);
        }
}

// The wave's share of the groups for R sets of 16 weight rows: acc[r] += the set's 16 x 16
// MFMA partial, D[m = 4 g4 + e][n = r16].  xop(k) gives the lane's 8 activations at k (zeros
// for activation rows past M or k past K).  `tile` is the wave's R x 16 rows of skinnyPitch
// bytes of LDS.
template <typename T, bool kInt8, int R, typename XOp>
__device__ __forceinline__ void skinnyGroups(f32x4 (&acc)[R], const char *wbase, const int (&rows0)[R],
                                             int nrows, int K, char *tile, int wave, int nw, int lane, XOp xop) {
    using S = SkinnyLoads<kInt8>;
    constexpr int kPitch = skinnyPitch(kInt8); // LDS row pitch: rows shift by 4 banks
    constexpr int kLoads = S::kLoads;
    const int r16 = lane % 16, g4 = lane / 16;
    const int ng = (K + kSkK - 1) / kSkK;
    const int lrow = lane / S::kLanesPerRow, lcol = lane % S::kLanesPerRow;
    const v4u z4 = {0u, 0u, 0u, 0u};
    for (int g = wave; g < ng; g += nw) {
        const int kg = g * kSkK;
        // weights: all loads of the group first
        v4u wl[R][kLoads];
        const int kw = kg + lcol * (16 / S::kElemB);
        const bool win = kw < K; // K % (16 / element bytes) == 0: a 16-byte chunk is all in or out
        skinnyLoad<kInt8, R>(wl, wbase, rows0, nrows, K, g, lane);
        // activations, in the MFMA's A layout
        v4u xa[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) xa[s] = xop(skinnyK<kInt8>(kg, s, g4));
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < kLoads; ++j)
                *reinterpret_cast<v4u *>(tile + ((r * 16) + j * S::kRowsPerLoad + lrow) * kPitch + 16 * lcol) = win ? wl[r][j] : z4;
        // same wave writes and reads its tile: LDS executes a wave's accesses in order
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const char *t = tile + r * 16 * kPitch;
            if constexpr (kInt8) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const v4u c = *reinterpret_cast<const v4u *>(t + r16 * kPitch + 64 * h + 16 * g4);
                    acc[r] = mfma<T>(xa[2 * h], codesToT<T>(v2u{c.x, c.y}), acc[r]);
                    acc[r] = mfma<T>(xa[2 * h + 1], codesToT<T>(v2u{c.z, c.w}), acc[r]);
                }
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    acc[r] = mfma<T>(xa[s], *reinterpret_cast<const v4u *>(t + r16 * kPitch + 64 * s + 16 * g4), acc[r]);
            }
        }
        // the next group's writes must not overtake this group's reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// Waves per skinny block: enough blocks x waves to fill the chip, at most one wave per group
// of 128 k (a function of N and K only, so that every caller splits K the same way).
inline int skinnyWaves(int N, int K) {
    const int tiles = (N + 15) / 16, ng = (K + kSkK - 1) / kSkK;
    const int a = 2048 / tiles > 2 ? 2048 / tiles : 2;
    int nw = a < ng ? a : ng;
    nw = nw < 16 ? nw : 16;
    return nw > 1 ? nw : 1;
}

// ---- the normalised row -------------------------------------------------------------------
// xs = T(rms_norm(h)) with h = residual ? T(in + residual) : in, formed exactly as
// rmsNormRows<T, G, VMAX, residual, true> forms one row: lane gl = tid % G of the group holds
// the 16-byte vectors gl + v G, sums its squares in (v, element) order, the group reduces
// (groupReduce<G>), then y = x * w * inv rounds to T.  Called by the G threads of the group
// (all 256 of the block when G == 256, which then meets a block barrier inside); h is stored
// to res_out when store_h.  `red` holds 256 / 64 floats of LDS.
template <typename T, int G, int VMAX>
__device__ __forceinline__ void normRow(char *xs, const void *in, const void *res, void *res_out,
                                        const void *norm_w, float eps, int K, float *red, bool store_h) {
    using F = Fmt<T>;
    constexpr int NV = F::kVec;
    const int gl = int(threadIdx.x) % G;
    const int nvec = K / NV;
    const bool fused = res != nullptr;
    v4u raw[VMAX], rv[VMAX], nwv[VMAX];
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = gl + v * G;
        if (vi < nvec) {
            raw[v] = load16<T>(in, size_t(vi) * NV);
            if (fused) rv[v] = load16<T>(res, size_t(vi) * NV);
            nwv[v] = load16<T>(norm_w, size_t(vi) * NV);
        }
    }
    if (fused) {
#pragma unroll
        for (int v = 0; v < VMAX; ++v) {
            const int vi = gl + v * G;
            if (vi < nvec) {
                float x[NV], r[NV];
                F::unpack(raw[v], x);
                F::unpack(rv[v], r);
#pragma unroll
                for (int e = 0; e < NV; ++e) x[e] = x[e] + r[e];
                raw[v] = F::packQ(x); // h = T(x + r), the value the reference's add stores
                if (store_h) store16<T>(res_out, size_t(vi) * NV, raw[v]);
            }
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        if (gl + v * G < nvec) {
            float x[NV];
            F::unpack(raw[v], x);
#pragma unroll
            for (int e = 0; e < NV; ++e) ss = fmaf(x[e], x[e], ss);
        }
    }
    ss = groupReduce<G, SumOp>(ss, red);
    const float rms = sqrtf(ss / float(K) + eps);
    const float inv = 1.0f / rms;
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = gl + v * G;
        if (vi < nvec) {
            float x[NV], w[NV], y[NV];
            F::unpack(raw[v], x);
            F::unpack(nwv[v], w);
#pragma unroll
            for (int e = 0; e < NV; ++e) y[e] = x[e] * w[e] * inv;
            *reinterpret_cast<v4u *>(xs + size_t(vi) * 16) = F::packQ(y);
        }
    }
}

} // namespace llaisys::kernels::lin
