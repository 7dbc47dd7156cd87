// rms_norm and fused residual-add + rms_norm for gfx950.
//
// Semantics: reference src/ops/rms_norm/cpu/rms_norm_cpu.cpp:15-33 -- per row,
// s = sum(x^2) in f32, rms = sqrtf(s / cols + eps), inv = 1 / rms, y = T((x * w) * inv).
// The fused variant first forms h = T(x + r) exactly as src/ops/add/cpu/add_cpu.cpp:12
// (f32 add, reference rounding), stores h and normalises h.  Only the summation order
// differs from the reference (a lane-parallel tree of fused multiply-adds instead of a
// left-to-right loop).  Outputs use packQ; a NaN eps, the one caller-supplied f32 whose
// NaN payload could reach them, takes the scalar kernel, which rounds exactly.
//
// Design: HBM-bound; a row lives in registers between the reduction and the scaling so
// x (and r) are read once and y (and h) written once.  16-byte loads per lane, butterfly
// reduction within the wavefront, LDS only to join the waves of one row when G > 64.
// Activations stream (non-temporal loads and stores); the weight row uses cached loads,
// since every row of the launch reads it.
// No MFMA: there is no contraction here.
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

#include <cmath>

namespace llaisys::kernels {

namespace {

template <typename T, int G, int VMAX, bool kFused, bool kWPre>
__global__ void __launch_bounds__(blockFor<G>())
    rmsNormRows(void *__restrict__ out, void *residual_out, const void *__restrict__ in,
                const void *residual, const void *__restrict__ weight, size_t rows, int cols,
                float eps) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    constexpr int kBlock = blockFor<G>();
    __shared__ float red[kBlock / kWave];

    const int lane = threadIdx.x % G;
    const size_t row = size_t(blockIdx.x) * (kBlock / G) + threadIdx.x / G;
    const bool live = row < rows;
    const int nvec = cols / N;
    const size_t base = row * size_t(cols);

    // The lane's share of the row, kept as raw 16-byte vectors.  All loads (x and, fused,
    // the residual) are issued before any store: residual_out may alias residual, so the
    // compiler could not hoist a residual load above an earlier residual store itself, and
    // the loads would turn into a chain of dependent round trips.
    // kWPre (few rows): the weight vectors are loaded here too -- after the reduction they
    // would be one more dependent round trip, which a single row (decode) waits on; with
    // many rows the registers cost more occupancy than the latency they hide.
    v4u raw[VMAX];
    v4u res[kFused ? VMAX : 1];
    v4u wv[kWPre ? VMAX : 1];
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = lane + v * G;
        if (live && vi < nvec) {
            raw[v] = load16Stream<T>(in, base + size_t(vi) * N);
            if constexpr (kFused) res[v] = load16Stream<T>(residual, base + size_t(vi) * N);
            if constexpr (kWPre) wv[v] = load16<T>(weight, size_t(vi) * N);
        }
    }
    if constexpr (kFused) {
#pragma unroll
        for (int v = 0; v < VMAX; ++v) {
            const int vi = lane + v * G;
            if (live && vi < nvec) {
                float x[N], r[N];
                F::unpack(raw[v], x);
                F::unpack(res[v], r);
#pragma unroll
                for (int e = 0; e < N; ++e) x[e] = x[e] + r[e];
                raw[v] = F::packQ(x); // h = T(x + r), the value the reference's add stores
                store16Stream<T>(residual_out, base + size_t(vi) * N, raw[v]);
            }
        }
    }
    float ss = 0.0f;
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = lane + v * G;
        if (live && vi < nvec) {
            float x[N];
            F::unpack(raw[v], x);
#pragma unroll
            for (int e = 0; e < N; ++e) ss = fmaf(x[e], x[e], ss);
        }
    }
    ss = groupReduce<G, SumOp>(ss, red);
    const float rms = sqrtf(ss / float(cols) + eps);
    const float inv = 1.0f / rms;
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = lane + v * G;
        if (live && vi < nvec) {
            float x[N], w[N], y[N];
            F::unpack(raw[v], x);
            F::unpack(kWPre ? wv[kWPre ? v : 0] : load16<T>(weight, size_t(vi) * N), w);
#pragma unroll
            for (int e = 0; e < N; ++e) y[e] = x[e] * w[e] * inv;
            store16Stream<T>(out, base + size_t(vi) * N, F::packQ(y));
        }
    }
}

// Any shape / alignment: one 256-thread block per row, scalar accesses, two passes over
// the row (the second pass re-reads it from cache).
template <typename T, bool kFused>
__global__ void __launch_bounds__(256)
    rmsNormRowsScalar(void *out, void *residual_out, const void *in, const void *residual,
                      const void *weight, size_t rows, size_t cols, float eps) {
    using F = Fmt<T>;
    __shared__ float red[256 / kWave];
    const size_t row = blockIdx.x;
    const size_t base = row * cols;
    float ss = 0.0f;
    for (size_t j = threadIdx.x; j < cols; j += 256) {
        float x = F::get(in, base + j);
        if constexpr (kFused) {
            x = F::round(x + F::get(residual, base + j));
            F::put(residual_out, base + j, x);
        }
        ss += x * x;
    }
    ss = groupReduce<256, SumOp>(ss, red);
    const float inv = 1.0f / sqrtf(ss / float(cols) + eps);
    const void *src = kFused ? residual_out : in;
    // Each thread re-reads only the elements it wrote itself in the fused case.
    for (size_t j = threadIdx.x; j < cols; j += 256)
        F::put(out, base + j, F::get(src, base + j) * F::get(weight, j) * inv);
}

template <typename T>
void launch(void *out, void *res_out, const void *in, const void *res, const void *w,
            size_t rows, size_t cols, float eps, hipStream_t s) {
    if (rows == 0 || cols == 0) return;
    constexpr int N = Fmt<T>::kVec;
    const bool fused = res != nullptr;
    const bool vec = cols % N == 0 && cols <= size_t(INT32_MAX) && aligned16(out) &&
                     aligned16(in) && aligned16(w) &&
                     (!fused || (aligned16(res) && aligned16(res_out)));
    RowPlan plan = vec && !std::isnan(eps) ? planRow(cols / N) : RowPlan{};
    bool done = false;
    withPlan(plan, [&](auto g, auto v) {
        constexpr int G = decltype(g)::value, V = decltype(v)::value; // V: vectors per lane
        constexpr int kBlock = blockFor<G>();
        const unsigned grid = blocksFor(rows, kBlock / G);
        const bool few = rows <= 64;
        if (fused && few)
            rmsNormRows<T, G, V, true, true><<<grid, kBlock, 0, s>>>(out, res_out, in, res, w, rows,
                                                                      int(cols), eps);
        else if (fused)
            rmsNormRows<T, G, V, true, false><<<grid, kBlock, 0, s>>>(out, res_out, in, res, w, rows,
                                                                       int(cols), eps);
        else if (few)
            rmsNormRows<T, G, V, false, true><<<grid, kBlock, 0, s>>>(out, nullptr, in, nullptr, w,
                                                                       rows, int(cols), eps);
        else
            rmsNormRows<T, G, V, false, false><<<grid, kBlock, 0, s>>>(out, nullptr, in, nullptr, w,
                                                                        rows, int(cols), eps);
        done = true;
    });
    if (done) return;
    if (fused)
        rmsNormRowsScalar<T, true><<<unsigned(rows), 256, 0, s>>>(out, res_out, in, res, w,
                                                                  rows, cols, eps);
    else
        rmsNormRowsScalar<T, false><<<unsigned(rows), 256, 0, s>>>(out, nullptr, in, nullptr,
                                                                   w, rows, cols, eps);
}

} // namespace

void rmsNorm(void *out, void *residual_out, const void *in, const void *residual,
             const void *weight, size_t rows, size_t cols, float eps, llaisysDataType_t dt,
             hipStream_t s) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launch<F32>(out, residual_out, in, residual, weight, rows, cols, eps, s);
    case LLAISYS_DTYPE_BF16: return launch<BF16>(out, residual_out, in, residual, weight, rows, cols, eps, s);
    case LLAISYS_DTYPE_F16: return launch<F16>(out, residual_out, in, residual, weight, rows, cols, eps, s);
    default: return;
    }
}

} // namespace llaisys::kernels
