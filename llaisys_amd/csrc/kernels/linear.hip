// Linear layers for gfx950: the reference's dense linear and W8A16 over INT8 weights.
//
// Semantics: reference src/ops/linear/cpu/linear_cpu.cpp:11-41 -- out[m][n] =
// T(sum_k x[m][k] * w[n][k] + bias[n]) with an f32 sum, x [rows, K], w [N, K].  W8A16 (no
// reference kernel): w is INT8 codes [N, K] with one f32 scale per output channel n, and
// out[m][n] = T(scale[n] * sum_k x[m][k] * code[n][k] + bias[n]).  The MFMA path sums the
// exact products of bf16 / f16 operands (INT8 codes are exact in both) in f32; the order of
// the sum differs from the reference's left-to-right loop, which the tests bound by the f32
// accumulation error.
//
// Design (MFMA-bound for prefill-sized M): v_mfma_f32_16x16x32_{bf16,f16} with both
// operands read straight from their rows -- A is 16 rows of x with 8 consecutive k per lane,
// B is 16 rows of w (out-channel major, k contiguous) with 8 consecutive k per lane, which
// is exactly the MFMA's B layout -- so no transpose and no LDS.  A wave owns a 64 x 64 output
// tile (16 accumulators), a block of 4 waves 128 x 128; the loads of K step s + 1 are issued
// before the 16 MFMAs of step s.  INT8 codes enter B as exact bf16 / f16 values and the
// per-channel scale multiplies the f32 sum once.  Other shapes / types: one thread per
// output, the reference's sequential sum.
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

#include <algorithm>
#include <type_traits>

namespace llaisys::kernels {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

struct LinearArgs {
    void *out;
    const void *x;
    const void *w;       // elements of T, or INT8 codes
    const float *scale;  // INT8 only
    const void *bias;    // T, or null
    int M, N, K;
};

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

constexpr int kWM = 64, kWN = 64;        // wave tile
constexpr int kBM = 128, kBN = 128;      // block tile (2 x 2 waves)
constexpr int kKS = 32;                  // K per step

template <typename T, bool kInt8>
__global__ void __launch_bounds__(256)
    linearMfma(LinearArgs a) {
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const int r16 = lane % 16, g4 = lane / 16;
    // block tiles: N-major order so that consecutive blocks share the x rows of an M tile
    const int nbn = (a.N + kBN - 1) / kBN;
    const int bm = int(blockIdx.x) / nbn, bn = int(blockIdx.x) % nbn;
    const int m0 = bm * kBM + (wave / 2) * kWM, n0 = bn * kBN + (wave % 2) * kWN;
    const char *xb = static_cast<const char *>(a.x);
    const char *wb = static_cast<const char *>(a.w);
    constexpr int wbytes = kInt8 ? 1 : 2;
    // rows this lane loads (clamped into range; results of clamped rows are not stored)
    int xr[4], wr[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        xr[t] = min(m0 + 16 * t + r16, a.M - 1);
        wr[t] = min(n0 + 16 * t + r16, a.N - 1);
    }
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const auto load = [&](int k0, v4u (&xa)[4], v4u (&wa)[4]) {
        const int kk = k0 + 8 * g4;
        const bool in = kk < a.K; // K % 8 == 0 on this path: a group is all in or all out
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            xa[t] = in ? *reinterpret_cast<const v4u *>(xb + (size_t(xr[t]) * a.K + kk) * 2) : v4u{0u, 0u, 0u, 0u};
            if constexpr (kInt8) {
                const v2u c = in ? *reinterpret_cast<const v2u *>(wb + size_t(wr[t]) * a.K + kk) : v2u{0u, 0u};
                wa[t] = v4u{c.x, c.y, 0u, 0u};
            } else {
                wa[t] = in ? *reinterpret_cast<const v4u *>(wb + (size_t(wr[t]) * a.K + kk) * wbytes) : v4u{0u, 0u, 0u, 0u};
            }
        }
    };
    v4u xa[4], wa[4], xn[4], wn[4];
    load(0, xa, wa);
    for (int k0 = 0; k0 < a.K; k0 += kKS) {
        if (k0 + kKS < a.K) load(k0 + kKS, xn, wn);
        v4u wt[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if constexpr (kInt8)
                wt[t] = codesToT<T>(v2u{wa[t].x, wa[t].y});
            else
                wt[t] = wa[t];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma<T>(xa[i], wt[j], acc[i][j]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            xa[t] = xn[t];
            wa[t] = wn[t];
        }
    }
    // D[m = 4g + e][n = r16] of tile (i, j)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + 16 * j + r16;
        if (n >= a.N) continue;
        const float sc = kInt8 ? a.scale[n] : 1.0f;
        const float bv = a.bias ? Fmt<T>::get(a.bias, n) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + 16 * i + 4 * g4 + e;
                if (m < a.M) {
                    const float s = kInt8 ? sc * acc[i][j][e] : acc[i][j][e];
                    Fmt<T>::put(a.out, size_t(m) * a.N + n, a.bias ? s + bv : s);
                }
            }
    }
}

// Few rows (M <= 16, decode): HBM-bound on the weights.  A block owns 16 output channels
// and its waves split K into groups of 128 k.  A load instruction that hands MFMA operands
// straight to registers touches 16 weight rows (lane l holds row l % 16), which streams
// HBM measurably slower than touching 4 rows with 256 contiguous bytes each; so each wave
// loads its group row-contiguously, transposes it through its own padded LDS tile
// (conflict-free on both sides) and reads the MFMA operand from there.  x rows >= M enter
// as zeros.  The waves' 16 x 16 partials are summed in LDS in wave order.
//
// k order inside a group (A and B agree, so the MFMA sum covers every k once):
//   16-bit weights: step s, lane (r, g) holds k = 32 s + 8 g + [0, 8)
//   INT8 weights:   step s, lane (r, g) holds k = 64 (s / 2) + 16 g + 8 (s % 2) + [0, 8)
// (an INT8 lane reads 16 codes, two steps' worth, in one LDS read).
constexpr int kSkK = 128; // k per group
constexpr int skinnyPitch(bool int8) { return (int8 ? kSkK : 2 * kSkK) + 16; }

template <typename T, bool kInt8>
__global__ void __launch_bounds__(1024)
    linearSkinny(LinearArgs a) {
    constexpr int kRowB = kInt8 ? kSkK : 2 * kSkK;  // bytes of one weight row in a group
    constexpr int kPitch = skinnyPitch(kInt8);       // LDS row pitch: rows shift by 4 banks
    constexpr int kLanesPerRow = kRowB / 16;         // lanes covering a row in one load
    constexpr int kRowsPerLoad = kWave / kLanesPerRow;
    constexpr int kLoads = 16 / kRowsPerLoad;        // loads per group: 4 (16-bit) / 2 (INT8)
    constexpr int kElemB = kInt8 ? 1 : 2;
    // dynamic LDS, sized by the launch: nw transpose tiles, then nw partial tiles
    extern __shared__ __align__(16) char smem[];
    const int nw = int(blockDim.x) / kWave;
    char(*stage)[16 * kPitch] = reinterpret_cast<char(*)[16 * kPitch]>(smem);
    float(*red)[256] = reinterpret_cast<float(*)[256]>(smem + nw * 16 * kPitch);
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const int r16 = lane % 16, g4 = lane / 16;
    const int n0 = int(blockIdx.x) * 16;
    const int ng = (a.K + kSkK - 1) / kSkK;
    char *tile = stage[wave];
    // row-contiguous load: instruction j, lane l -> row j * kRowsPerLoad + l / kLanesPerRow,
    // 16 bytes at column (l % kLanesPerRow)
    const int lrow = lane / kLanesPerRow, lcol = lane % kLanesPerRow;
    const char *wbase = static_cast<const char *>(a.w);
    const char *xrow = static_cast<const char *>(a.x) + size_t(min(r16, a.M - 1)) * a.K * 2;
    const bool xlane = r16 < a.M;
    const v4u z4 = {0u, 0u, 0u, 0u};
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int g = wave; g < ng; g += nw) {
        const int kg = g * kSkK;
        // weights: all loads of the group first
        v4u wl[kLoads];
        const int kw = kg + lcol * (16 / kElemB);
        const bool win = kw < a.K; // K % (16 / element bytes) == 0: a 16-byte chunk is all in or out
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int row = min(n0 + j * kRowsPerLoad + lrow, a.N - 1);
            wl[j] = *reinterpret_cast<const v4u *>(wbase + (size_t(row) * a.K + (win ? kw : 0)) * kElemB);
        }
        // activations (few rows, cache-resident), in the MFMA's A layout
        v4u xa[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int k = kg + (kInt8 ? 64 * (s / 2) + 16 * g4 + 8 * (s % 2) : 32 * s + 8 * g4);
            xa[s] = *reinterpret_cast<const v4u *>(xrow + size_t(k < a.K ? k : 0) * 2);
            if (!(xlane && k < a.K)) xa[s] = z4;
        }
#pragma unroll
        for (int j = 0; j < kLoads; ++j)
            *reinterpret_cast<v4u *>(tile + (j * kRowsPerLoad + lrow) * kPitch + 16 * lcol) = win ? wl[j] : z4;
        // same wave writes and reads its tile: LDS executes a wave's accesses in order
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if constexpr (kInt8) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const v4u c = *reinterpret_cast<const v4u *>(tile + r16 * kPitch + 64 * h + 16 * g4);
                acc = mfma<T>(xa[2 * h], codesToT<T>(v2u{c.x, c.y}), acc);
                acc = mfma<T>(xa[2 * h + 1], codesToT<T>(v2u{c.z, c.w}), acc);
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc = mfma<T>(xa[s], *reinterpret_cast<const v4u *>(tile + r16 * kPitch + 64 * s + 16 * g4), acc);
        }
        // the next group's writes must not overtake this group's reads
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // D[m = 4 g + e][n = r16]
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][(4 * g4 + e) * 16 + r16] = acc[e];
    __syncthreads();
    for (int t = int(threadIdx.x); t < 16 * a.M; t += int(blockDim.x)) {
        const int m = t / 16, n = n0 + t % 16;
        if (n < a.N) {
            float s = 0.0f;
            for (int w = 0; w < nw; ++w) s += red[w][t];
            if constexpr (kInt8) s = a.scale[n] * s;
            if (a.bias) s = s + Fmt<T>::get(a.bias, n);
            Fmt<T>::put(a.out, size_t(m) * a.N + n, s);
        }
    }
}

// Any shape and type: one thread per output, the sum in the reference's order.
template <typename T, bool kInt8>
__global__ void __launch_bounds__(256)
    linearScalar(LinearArgs a) {
    const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= size_t(a.M) * a.N) return;
    const size_t m = idx / a.N, n = idx % a.N;
    float sum = 0.0f;
    for (int k = 0; k < a.K; ++k) {
        const float wv = kInt8 ? float(static_cast<const int8_t *>(a.w)[n * a.K + k]) : Fmt<T>::get(a.w, n * a.K + k);
        sum = sum + Fmt<T>::get(a.x, m * a.K + k) * wv;
    }
    if constexpr (kInt8) sum = a.scale[n] * sum;
    if (a.bias) sum = sum + Fmt<T>::get(a.bias, n);
    Fmt<T>::put(a.out, idx, sum);
}

template <typename T, bool kInt8>
void launch(const LinearArgs &a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    const auto al = [](const void *p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; };
    constexpr bool kMfmaType = std::is_same_v<T, BF16> || std::is_same_v<T, F16>;
    if (kMfmaType && a.K % 8 == 0 && a.K > 0 && al(a.x, 16) && al(a.w, kInt8 ? 8 : 16)) {
        if (a.M <= 16 && (!kInt8 || a.K % 16 == 0) && al(a.w, 16)) {
            // waves per block: enough blocks x waves to fill the chip, at most one wave per
            // group of 128 k
            const int tiles = (a.N + 15) / 16, ng = (a.K + kSkK - 1) / kSkK;
            const int nw = std::max(1, std::min({16, ng, std::max(2, 2048 / tiles)}));
            const size_t lds = size_t(nw) * (16 * skinnyPitch(kInt8) + 256 * sizeof(float));
            if constexpr (kMfmaType) linearSkinny<T, kInt8><<<unsigned(tiles), unsigned(nw * kWave), lds, s>>>(a);
            return;
        }
        const unsigned blocks = unsigned((a.M + kBM - 1) / kBM) * unsigned((a.N + kBN - 1) / kBN);
        if constexpr (kMfmaType) linearMfma<T, kInt8><<<blocks, 256, 0, s>>>(a);
        return;
    }
    const size_t n = size_t(a.M) * a.N;
    linearScalar<T, kInt8><<<unsigned((n + 255) / 256), 256, 0, s>>>(a);
}

template <bool kInt8>
void dispatch(const LinearArgs &a, llaisysDataType_t dt, hipStream_t s) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launch<F32, kInt8>(a, s);
    case LLAISYS_DTYPE_BF16: return launch<BF16, kInt8>(a, s);
    case LLAISYS_DTYPE_F16: return launch<F16, kInt8>(a, s);
    default: return;
    }
}

} // namespace

void linear(void *out, const void *x, const void *w, const float *w_scale, const void *bias,
            size_t rows, size_t in_features, size_t out_features, llaisysDataType_t dt,
            hipStream_t s) {
    const LinearArgs a{out, x, w, w_scale, bias, int(rows), int(out_features), int(in_features)};
    if (w_scale)
        dispatch<true>(a, dt, s);
    else
        dispatch<false>(a, dt, s);
}

} // namespace llaisys::kernels
