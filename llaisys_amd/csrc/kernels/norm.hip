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

// A row of exactly G 16-byte vectors (G a multiple of 64) per block of G threads, one
// vector per lane: the launch plan for few rows.  With the register plan above, 2048 rows
// of 1536 bf16 are 2048 single-wave rows (two waves per SIMD, each waiting on 3 KB of
// loads); here they are 6144 waves of one 1 KB load each, joined through LDS.  Measured
// on MI355X (graph-replayed medians over >= 1 GiB of rotating sets), [2048, 1536] bf16:
// add + rms_norm 5.83 -> 5.32 us, rms_norm 4.14 -> 3.57 us; [256, 1536] 3.97 -> 2.58 and
// 3.17 -> 2.46 us; f32 [128, 1536] 3.78 -> 2.57 and 3.36 -> 2.47 us.  With more data the
// register plan wins (bf16 [3072, 1536] add + rms_norm 7.69 vs 8.36 us, [2048, 4096] 11.8
// vs 13.1 us; f32 [2048, 1536] rms_norm 5.28 vs 6.58 us), so the launcher takes this
// kernel for inputs under kWideBytes.  Same arithmetic as rmsNormRows; only the lane tree
// of the sum differs.
constexpr size_t kWideBytes = size_t(8) << 20; // input bytes below which rmsNormWide runs

template <typename T, int G, bool kFused>
__global__ void __launch_bounds__(G)
    rmsNormWide(void *__restrict__ out, void *residual_out, const void *__restrict__ in,
                const void *residual, const void *__restrict__ weight, int cols, float eps) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    __shared__ float red[G / kWave];
    const size_t at = size_t(blockIdx.x) * size_t(cols) + size_t(threadIdx.x) * N;
    v4u raw = load16Stream<T>(in, at);
    float x[N];
    F::unpack(raw, x);
    if constexpr (kFused) {
        float r[N];
        F::unpack(load16Stream<T>(residual, at), r);
#pragma unroll
        for (int e = 0; e < N; ++e) x[e] = x[e] + r[e];
        raw = F::packQ(x); // h = T(x + r), the value the reference's add stores
        store16Stream<T>(residual_out, at, raw);
        F::unpack(raw, x);
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < N; ++e) ss = fmaf(x[e], x[e], ss);
    ss = groupReduce<G, SumOp>(ss, red);
    const float inv = 1.0f / sqrtf(ss / float(cols) + eps);
    float w[N], y[N];
    F::unpack(load16<T>(weight, size_t(threadIdx.x) * N), w);
#pragma unroll
    for (int e = 0; e < N; ++e) y[e] = x[e] * w[e] * inv;
    store16Stream<T>(out, at, F::packQ(y));
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

template <typename T, int G>
void launchWideG(void *out, void *res_out, const void *in, const void *res, const void *w,
                 size_t rows, size_t cols, float eps, hipStream_t s) {
    if (res)
        rmsNormWide<T, G, true><<<unsigned(rows), G, 0, s>>>(out, res_out, in, res, w, int(cols), eps);
    else
        rmsNormWide<T, G, false><<<unsigned(rows), G, 0, s>>>(out, nullptr, in, nullptr, w, int(cols), eps);
}

// The wide-row kernel for rows of 128..1024 vectors in steps of 64 that have an
// instantiation (Qwen2 1536 and Llama 4096 columns in bf16 / f16 and f32); false otherwise.
template <typename T>
bool launchWide(void *out, void *res_out, const void *in, const void *res, const void *w,
                size_t rows, size_t cols, float eps, hipStream_t s) {
    switch (cols / Fmt<T>::kVec) {
    case 192: launchWideG<T, 192>(out, res_out, in, res, w, rows, cols, eps, s); return true;
    case 384: launchWideG<T, 384>(out, res_out, in, res, w, rows, cols, eps, s); return true;
    case 512: launchWideG<T, 512>(out, res_out, in, res, w, rows, cols, eps, s); return true;
    case 1024: launchWideG<T, 1024>(out, res_out, in, res, w, rows, cols, eps, s); return true;
    default: return false;
    }
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
    if (vec && !std::isnan(eps) && rows > 64 && rows * cols * size_t(Fmt<T>::kBytes) < kWideBytes &&
        launchWide<T>(out, res_out, in, res, w, rows, cols, eps, s))
        return;
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
