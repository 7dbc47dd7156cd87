// rms_norm (after an optional residual add) fused ahead of a one-row projection, and
// optionally swiglu after it, for gfx950.
//
// Semantics: the composition of the library's own ops, bit for bit --
//   h  = in + residual, rounded as src/ops/add/cpu/add_cpu.cpp:12 (stored to residual_out),
//   xn = rms_norm(h) as src/ops/rms_norm/cpu/rms_norm_cpu.cpp:15-33, computed exactly as the
//        rmsNormRows kernel computes a row (same lane groups, same sums, same rounding),
//   y  = linear(xn) as src/ops/linear/cpu/linear_cpu.cpp:11-41 (W8A16 with per-channel
//        scales), each lane summing its chunks lane, lane + 64, lane + 128, ... with the
//        same FMAs as the one-row linearGemv kernel, then the same butterfly,
//   out = y, or swiglu(T(gate), T(up)) as src/ops/swiglu/cpu/swiglu_cpu.cpp:15-20 over the
//        weight rows [0, N) (gate) and [N, 2N) (up).
//   (INT8 weights over 4096 or more channels: the skinny MFMA loop the separate linear takes
//   there, with the same K split and the same order of the waves' partials.)
// So the fused output equals rmsNorm -> linear -> swiglu launched separately, bit for bit, for
// one row (with the skinny form when the norm group is one wave, i.e. hidden <= 2048).
//
// Design (HBM-bound on the weights, one launch instead of three): a block of 4 waves; each
// wave owns one output channel (with swiglu: its gate and up rows).  The waves first
// request their weight rows' first pass, then the block forms the normalised row in LDS
// (wave 0 alone for a 64-lane norm group, all 4 waves for a 256-lane one) while those loads
// are in flight, joins on an LDS-only barrier (the weight loads stay outstanding), and
// streams the rest of the rows with the activations read from LDS.  Every block re-forms
// the row from in / residual / weight (L2 hits after the first block); block 0 stores h.
#include "common.hpp"
#include "launch.hpp"
#include "linear_common.hpp"
#include "rowplan.hpp"

#include <cmath>

namespace llaisys::kernels {

namespace {

struct NormLinArgs {
    void *out;
    void *res_out;
    const void *in;
    const void *res; // null: no residual add
    const void *norm_w;
    float eps;
    const void *w;
    const float *scale; // INT8 only
    const void *bias;   // null: no bias
    int N, K;           // outputs (swiglu: gate / up pairs), row length
};


template <typename T, bool kInt8, int G, int VMAX, bool kSwiglu, int U>
__global__ void __launch_bounds__(256)
    linearNormGemv(NormLinArgs a) {
    using F = Fmt<T>;
    constexpr int E = kInt8 ? 16 : 8;  // weight elements per 16-byte chunk
    constexpr int R = kSwiglu ? 2 : 1; // weight rows per wave; U: chunks per lane and row per pass
    static_assert(G == kWave || G == 256, "norm group: one wave or the whole block");
    extern __shared__ __align__(16) char xs[]; // the normalised row, K elements of T
    __shared__ float red[256 / kWave];
    const int lane = int(threadIdx.x) % kWave;
    const int n = int(blockIdx.x) * 4 + int(threadIdx.x) / kWave; // wave-uniform
    const bool live = n < a.N; // a wave past the last channel loads a valid row, stores nothing
    const int nc = a.K / E;    // K % E == 0
    const size_t rowB = size_t(a.K) * (kInt8 ? 1 : 2);
    const char *wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
        wrow[r] = static_cast<const char *>(a.w) + (size_t(live ? n : a.N - 1) + size_t(r) * a.N) * rowB;
    // The first pass's weight chunks are requested before the norm, so that their latency
    // overlaps it (a chunk past the row end reads chunk 0 and is skipped below).
    v4u wv[R][U];
    const auto loadPass = [&](int c0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + kWave * u < nc ? c0 + kWave * u : 0;
#pragma unroll
            for (int r = 0; r < R; ++r) wv[r][u] = *reinterpret_cast<const v4u *>(wrow[r] + size_t(c) * 16);
        }
    };
    loadPass(lane);

    if (G == 256 || threadIdx.x < G)
        lin::normRow<T, G, VMAX>(xs, a.in, a.res, a.res_out, a.norm_w, a.eps, a.K, red, blockIdx.x == 0);
    // the row in LDS is complete (LDS-only barrier: the weight loads stay in flight)
    ldsBarrier();
    if (!live) return;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    for (int c0 = lane;;) {
        v4u xv[U][E / 8];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + kWave * u < nc ? c0 + kWave * u : 0;
#pragma unroll
            for (int h = 0; h < E / 8; ++h) xv[u][h] = *reinterpret_cast<const v4u *>(xs + (size_t(c) * E + 8 * h) * 2);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + kWave * u >= nc) continue;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float wf[E];
                if constexpr (kInt8) {
                    const uint32_t ww[4] = {wv[r][u].x, wv[r][u].y, wv[r][u].z, wv[r][u].w};
#pragma unroll
                    for (int e = 0; e < E; ++e) wf[e] = float(int8_t(ww[e / 4] >> (8 * (e % 4))));
                } else {
                    F::unpack(wv[r][u], wf);
                }
#pragma unroll
                for (int h = 0; h < E / 8; ++h) {
                    float xf[8];
                    F::unpack(xv[u][h], xf);
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[r] = __builtin_fmaf(xf[e], wf[8 * h + e], acc[r]);
                }
            }
        }
        c0 += kWave * U;
        if (c0 >= nc) break;
        loadPass(c0);
    }
    float y[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int ch = n + r * a.N;
        float s = waveGroupReduce<kWave, SumOp>(acc[r]);
        if constexpr (kInt8) s = a.scale[ch] * s;
        if (a.bias) s = s + F::get(a.bias, ch);
        y[r] = s;
    }
    if (lane == 0) {
        if constexpr (kSwiglu)
            F::put(a.out, n, SwigluOp::apply(F::round(y[0]), F::round(y[1])));
        else
            F::put(a.out, n, y[0]);
    }
}

// INT8 weights with N >= 4096 (where the separate linear takes the skinny MFMA kernel): the
// same skinny loop (linear_common.hpp) over the 16 channels of the block -- and with swiglu
// their 16 up rows as a second set -- with the normalised row (formed by wave 0, a 64-lane
// norm group) as the activation operand from LDS.  Before the norm every wave requests its
// first group's weight rows, so that the loop finds them in L2; the waves' partials are then
// summed in LDS in wave order, as the separate kernel sums them.
template <typename T, int VMAX, bool kSwiglu>
__global__ void __launch_bounds__(1024)
    linearNormSkinny(NormLinArgs a) {
    constexpr int R = kSwiglu ? 2 : 1;
    constexpr int kPitch = lin::skinnyPitch(true);
    // dynamic LDS: the normalised row (K x 2 bytes), nw transpose tiles of R x 16 rows, nw
    // partial tiles of R x 256 floats
    extern __shared__ __align__(16) char smem[];
    __shared__ float red_n[256 / kWave];
    const int nw = int(blockDim.x) / kWave;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const int r16 = lane % 16, g4 = lane / 16;
    const int n0 = int(blockIdx.x) * 16;
    char *xs = smem;
    char *tile = smem + size_t(a.K) * 2 + size_t(wave) * R * 16 * kPitch;
    float *red = reinterpret_cast<float *>(smem + size_t(a.K) * 2 + size_t(nw) * R * 16 * kPitch);
    const char *wbase = static_cast<const char *>(a.w);
    int rows0[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rows0[r] = n0 + r * a.N;
    const int nrows = R * a.N;
    // the wave's first group of weights is requested before the norm and only consumed after
    // it (an empty asm use), so that the loop below finds those rows in L2; handing the
    // registers themselves to the loop measured slower
    v4u warm[R][lin::SkinnyLoads<true>::kLoads];
    lin::skinnyLoad<true, R>(warm, wbase, rows0, nrows, a.K, wave, lane);
    if (threadIdx.x < kWave)
        lin::normRow<T, kWave, VMAX>(xs, a.in, a.res, a.res_out, a.norm_w, a.eps, a.K, red_n, blockIdx.x == 0);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < lin::SkinnyLoads<true>::kLoads; ++j) asm volatile("" ::"v"(warm[r][j]));
    __syncthreads();
    const v4u z4 = {0u, 0u, 0u, 0u};
    const auto xop = [&](int k) {
        const v4u v = *reinterpret_cast<const v4u *>(xs + size_t(k < a.K ? k : 0) * 2);
        return r16 == 0 && k < a.K ? v : z4;
    };
    lin::f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = lin::f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    lin::skinnyGroups<T, true, R>(acc, wbase, rows0, nrows, a.K, tile, wave, nw, lane, xop);
    // D[m = 4 g + e][n = r16]; one activation row: m = 0
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[(size_t(wave) * R + r) * 256 + (4 * g4 + e) * 16 + r16] = acc[r][e];
    __syncthreads();
    const int t = int(threadIdx.x);
    if (t < 16 && n0 + t < a.N) {
        float y[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = rows0[r] + t;
            float s = 0.0f;
            for (int w = 0; w < nw; ++w) s += red[(size_t(w) * R + r) * 256 + t];
            s = a.scale[n] * s;
            if (a.bias) s = s + Fmt<T>::get(a.bias, n);
            y[r] = s;
        }
        if constexpr (kSwiglu)
            Fmt<T>::put(a.out, n0 + t, SwigluOp::apply(Fmt<T>::round(y[0]), Fmt<T>::round(y[1])));
        else
            Fmt<T>::put(a.out, n0 + t, y[0]);
    }
}

template <typename T, bool kInt8, bool kSwiglu, int U>
void launchU(const NormLinArgs &a, const RowPlan &plan, hipStream_t s) {
    const unsigned blocks = unsigned((a.N + 3) / 4);
    const size_t lds = size_t(a.K) * 2;
    if (plan.group == kWave)
        linearNormGemv<T, kInt8, kWave, 4, kSwiglu, U><<<blocks, 256, lds, s>>>(a);
    else if (plan.vmax == 4)
        linearNormGemv<T, kInt8, 256, 4, kSwiglu, U><<<blocks, 256, lds, s>>>(a);
    else
        linearNormGemv<T, kInt8, 256, 8, kSwiglu, U><<<blocks, 256, lds, s>>>(a);
}

// Chunks per lane and pass: a row of at most 128 chunks (INT8 K <= 2048, 16-bit K <= 1024)
// in one pass of 2, else passes of 4 (the chunk order per lane is the same either way).
template <typename T, bool kInt8, bool kSwiglu>
void launchNorm(const NormLinArgs &a, const RowPlan &plan, hipStream_t s) {
    if (a.K / (kInt8 ? 16 : 8) <= 2 * kWave)
        launchU<T, kInt8, kSwiglu, 2>(a, plan, s);
    else
        launchU<T, kInt8, kSwiglu, 4>(a, plan, s);
}

template <typename T, bool kSwiglu>
void launchSkinny(const NormLinArgs &a, const RowPlan &plan, hipStream_t s) {
    const int nw = lin::skinnyWaves(a.N, a.K), R = kSwiglu ? 2 : 1;
    const size_t lds = size_t(a.K) * 2 + size_t(nw) * R * (16 * lin::skinnyPitch(true) + 256 * sizeof(float));
    const unsigned blocks = unsigned((a.N + 15) / 16);
    if (plan.vmax == 4)
        linearNormSkinny<T, 4, kSwiglu><<<blocks, unsigned(nw * kWave), lds, s>>>(a);
    else
        linearNormSkinny<T, 8, kSwiglu><<<blocks, unsigned(nw * kWave), lds, s>>>(a);
}

template <typename T>
void dispatch(const NormLinArgs &a, const RowPlan &plan, bool int8, bool swiglu, hipStream_t s) {
    // INT8 weights over 256 or more 16-channel tiles: the skinny MFMA kernel, as the separate
    // linear of one row takes it
    if (int8 && (a.N + 15) / 16 >= 256 && plan.group == kWave) {
        swiglu ? launchSkinny<T, true>(a, plan, s) : launchSkinny<T, false>(a, plan, s);
        return;
    }
    if (int8)
        swiglu ? launchNorm<T, true, true>(a, plan, s) : launchNorm<T, true, false>(a, plan, s);
    else
        swiglu ? launchNorm<T, false, true>(a, plan, s) : launchNorm<T, false, false>(a, plan, s);
}

} // namespace

bool rmsNormLinearFused(void *out, void *residual_out, const void *in, const void *residual,
                        const void *norm_weight, float eps, const void *w, const float *w_scale,
                        const void *bias, size_t rows, size_t in_features, size_t out_features,
                        bool swiglu, llaisysDataType_t dt, hipStream_t s) {
    if (rows != 1 || (dt != LLAISYS_DTYPE_BF16 && dt != LLAISYS_DTYPE_F16) || std::isnan(eps)) return false;
    const size_t K = in_features, E = w_scale ? 16 : 8;
    // the normalised row lives in LDS: K * 2 bytes, at most 64 KB
    if (K == 0 || K % E != 0 || K > 32768 || out_features == 0 || out_features >= (size_t(1) << 30)) return false;
    if (!aligned16(in) || !aligned16(w) || !aligned16(norm_weight) ||
        (residual && (!aligned16(residual) || !aligned16(residual_out))))
        return false;
    const RowPlan plan = planRow(K / 8);
    if (plan.group != kWave && plan.group != 256) return false;
    const NormLinArgs a{out, residual_out, in, residual, norm_weight, eps, w, w_scale, bias,
                        int(out_features), int(K)};
    if (dt == LLAISYS_DTYPE_BF16)
        dispatch<BF16>(a, plan, w_scale != nullptr, swiglu, s);
    else
        dispatch<F16>(a, plan, w_scale != nullptr, swiglu, s);
    return true;
}

} // namespace llaisys::kernels
