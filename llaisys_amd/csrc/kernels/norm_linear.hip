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
// So the fused output equals rmsNorm -> linear -> swiglu launched separately, bit for bit, for
// one row (the separate linear of one row always sums this way, INT8 weights included).
//
// Design (HBM-bound on the weights, one launch instead of three): a block of 4 or 8 waves;
// each wave owns one output channel (with swiglu: its gate and up rows).  The waves first
// request their weight rows' first pass (the whole row up to 128 chunks), then the block forms the normalised row in LDS
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


template <typename T, bool kInt8, int G, int VMAX, bool kSwiglu, int U, int NW>
__global__ void __launch_bounds__(NW * kWave)
    linearNormGemv(NormLinArgs a) {
    using F = Fmt<T>;
    constexpr int E = kInt8 ? 16 : 8;  // weight elements per 16-byte chunk
    constexpr int R = kSwiglu ? 2 : 1; // weight rows per wave; U: chunks per lane and row per pass
    static_assert(G == kWave || G == 256, "norm group: one wave or 4 waves");
    // a 4-wave norm group reduces through block-wide barriers, which every wave must reach
    static_assert(G == kWave || NW == 4, "a 256-lane norm group spans the whole block");
    extern __shared__ __align__(16) char xs[]; // the normalised row, K elements of T
    __shared__ float red[256 / kWave];
    const int lane = int(threadIdx.x) % kWave;
    const int n = int(blockIdx.x) * NW + int(threadIdx.x) / kWave; // wave-uniform
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
            for (int r = 0; r < R; ++r)
                wv[r][u] = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(wrow[r] + size_t(c) * 16));
        }
    };
    loadPass(lane);

    if (threadIdx.x < G)
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
            float xf[E]; // unpacked once for the wave's R rows; each row's sum keeps its order
#pragma unroll
            for (int h = 0; h < E / 8; ++h) F::unpack(xv[u][h], xf + 8 * h);
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
                for (int e = 0; e < E; ++e) acc[r] = __builtin_fmaf(xf[e], wf[e], acc[r]);
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

// Waves per block: 8 for up to 4096 channels with a one-wave norm group (twice the channels
// per norm; q/k/v [2048, 1536] 4.01 -> 3.68 us INT8, 4.66 -> 4.00 us bf16), else 4 (with 8:
// gate/up + swiglu [2 x 8960, 1536] 9.99 -> 10.46 us INT8, 16 waves 12.67 us).
template <typename T, bool kInt8, bool kSwiglu, int U>
void launchU(const NormLinArgs &a, const RowPlan &plan, hipStream_t s) {
    const size_t lds = size_t(a.K) * 2;
    const unsigned b4 = unsigned((a.N + 3) / 4);
    if (plan.group == kWave && a.N <= 4096)
        linearNormGemv<T, kInt8, kWave, 4, kSwiglu, U, 8><<<unsigned((a.N + 7) / 8), 512, lds, s>>>(a);
    else if (plan.group == kWave)
        linearNormGemv<T, kInt8, kWave, 4, kSwiglu, U, 4><<<b4, 256, lds, s>>>(a);
    else if (plan.vmax == 4)
        linearNormGemv<T, kInt8, 256, 4, kSwiglu, U, 4><<<b4, 256, lds, s>>>(a);
    else
        linearNormGemv<T, kInt8, 256, 8, kSwiglu, U, 4><<<b4, 256, lds, s>>>(a);
}

// Chunks per lane and pass: the whole row in one pass while it is at most 4 chunks per lane
// (INT8 K <= 4096, 16-bit K <= 2048), else passes of 4 (the chunk order per lane is the
// same either way).
template <typename T, bool kInt8, bool kSwiglu>
void launchNorm(const NormLinArgs &a, const RowPlan &plan, hipStream_t s) {
    switch ((a.K / (kInt8 ? 16 : 8) + kWave - 1) / kWave) {
    case 1: launchU<T, kInt8, kSwiglu, 1>(a, plan, s); break;
    case 2: launchU<T, kInt8, kSwiglu, 2>(a, plan, s); break;
    case 3: launchU<T, kInt8, kSwiglu, 3>(a, plan, s); break;
    default: launchU<T, kInt8, kSwiglu, 4>(a, plan, s); break;
    }
}

template <typename T>
void dispatch(const NormLinArgs &a, const RowPlan &plan, bool int8, bool swiglu, hipStream_t s) {
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
