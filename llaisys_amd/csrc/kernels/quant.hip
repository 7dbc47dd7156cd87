// INT8 symmetric absmax quantization for gfx950 (weights per output channel, KV cache per
// token and head).
//
// Rule (no reference kernel exists; the oracle states the same rule): per row of `cols`,
// amax = max|x| in f32 (a NaN never raises it), scale = amax / 127.0f,
// q = clamp(rint(x / scale), -127, 127) with IEEE division and round-half-even, and
// q = 0 for an all-zero row or a NaN quotient.  The codes are bit-exact with the oracle:
// max is order-independent and every other step is a single correctly rounded operation.
//
// Design: the row lives in registers (same lane-group plan as rms_norm), so x is read
// once; amax is an integer max over the packed magnitude bits and the codes come from the
// division-free correctly rounded quotient of quantize.hpp, ~7 VALU operations per bf16
// element in all; codes are written as 8-byte (bf16/f16 input) or 4-byte (f32) stores per lane and
// the scale by the group's first lane.  A KV-cache append is this kernel pointed at the
// cache rows pos .. pos + n_tok, so the codes go straight into the cache.
#include "common.hpp"
#include "launch.hpp"
#include "quantize.hpp"
#include "rowplan.hpp"

#include <type_traits>

namespace llaisys::kernels {

namespace {

template <typename T, int G, int VMAX>
__global__ void __launch_bounds__(blockFor<G>())
    quantRows(int8_t *__restrict__ q, float *__restrict__ scale, const void *__restrict__ in,
              size_t rows, int cols) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    constexpr int kBlock = blockFor<G>();
    __shared__ float red[kBlock / kWave];

    const int lane = threadIdx.x % G;
    const size_t row = size_t(blockIdx.x) * (kBlock / G) + threadIdx.x / G;
    const bool live = row < rows;
    const int nvec = cols / N;
    const size_t base = row * size_t(cols);

    v4u raw[VMAX];
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = lane + v * G;
        if (live && vi < nvec) raw[v] = load16Stream<T>(in, base + size_t(vi) * N);
    }
    // amax: integer max of the magnitude bits; the float rule only for a row with a NaN
    // (the test is uniform over the group, so the group's lanes all take it)
    using A = AbsBits<T>;
    uint32_t bits = 0;
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = lane + v * G;
        if (live && vi < nvec) bits = A::fold(bits, raw[v]);
    }
    bits = groupReduce<G, MaxU32Op>(A::finish(bits), reinterpret_cast<uint32_t *>(red));
    float amax = A::value(bits);
    if (__builtin_expect(bits > A::kInf, 0)) {
        amax = 0.0f;
#pragma unroll
        for (int v = 0; v < VMAX; ++v) {
            const int vi = lane + v * G;
            if (live && vi < nvec) {
                float x[N];
                F::unpack(raw[v], x);
#pragma unroll
                for (int e = 0; e < N; ++e) amax = MaxOp::apply(amax, fabsf(x[e]));
            }
        }
        amax = groupReduce<G, MaxOp>(amax, red);
    }
    const RowQuantizer qz(amax);
    if (live && lane == 0) scale[row] = qz.scale;
    if (__builtin_expect(qz.exact_only, 0)) {
        // scale < 2^-96 (or an all-zero row): IEEE quotients, re-reading the row's elements
        // so that this rare path adds no per-vector code to the common one
        for (int j = lane; live && j < cols; j += G)
            q[base + j] = int8_t(codeOf(F::get(in, base + j), amax, qz.scale));
        return;
    }
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = lane + v * G;
        if (live && vi < nvec) {
            float x[N];
            uint32_t c[N];
            F::unpack(raw[v], x);
            qz.fastCodes<N, std::is_same_v<T, F32>>(x, c);
            storeCodes<N>(q, base + size_t(vi) * N, c);
        }
    }
}

template <typename T>
__global__ void __launch_bounds__(256)
    quantRowsScalar(int8_t *q, float *scale, const void *in, size_t rows, size_t cols) {
    using F = Fmt<T>;
    __shared__ float red[256 / kWave];
    const size_t base = size_t(blockIdx.x) * cols;
    float amax = 0.0f;
    for (size_t j = threadIdx.x; j < cols; j += 256) amax = MaxOp::apply(amax, fabsf(F::get(in, base + j)));
    amax = groupReduce<256, MaxOp>(amax, red);
    const float sc = amax / 127.0f;
    if (threadIdx.x == 0) scale[blockIdx.x] = sc;
    for (size_t j = threadIdx.x; j < cols; j += 256)
        q[base + j] = int8_t(codeOf(F::get(in, base + j), amax, sc));
}

template <typename T>
void launch(int8_t *q, float *scale, const void *in, size_t rows, size_t cols, hipStream_t s) {
    if (rows == 0) return;
    constexpr int N = Fmt<T>::kVec;
    const bool vec = cols > 0 && cols % N == 0 && cols <= size_t(INT32_MAX) && aligned16(in) &&
                     reinterpret_cast<uintptr_t>(q) % N == 0;
    RowPlan plan = vec ? planRow(cols / N) : RowPlan{};
    bool done = false;
    withPlan(plan, [&](auto g, auto v) {
        constexpr int G = decltype(g)::value, V = decltype(v)::value;
        constexpr int kBlock = blockFor<G>();
        quantRows<T, G, V><<<blocksFor(rows, kBlock / G), kBlock, 0, s>>>(q, scale, in, rows,
                                                                          int(cols));
        done = true;
    });
    if (!done) quantRowsScalar<T><<<unsigned(rows), 256, 0, s>>>(q, scale, in, rows, cols);
}

} // namespace

void quantizeInt8(int8_t *q, float *scale, const void *in, size_t rows, size_t cols,
                  llaisysDataType_t dt, hipStream_t s) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launch<F32>(q, scale, in, rows, cols, s);
    case LLAISYS_DTYPE_BF16: return launch<BF16>(q, scale, in, rows, cols, s);
    case LLAISYS_DTYPE_F16: return launch<F16>(q, scale, in, rows, cols, s);
    default: return;
    }
}

} // namespace llaisys::kernels
