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
// once; codes are written as 8-byte (bf16/f16 input) or 4-byte (f32) stores per lane and
// the scale by the group's first lane.  A KV-cache append is this kernel pointed at the
// cache rows pos .. pos + n_tok, so the codes go straight into the cache.
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

namespace llaisys::kernels {

namespace {

__device__ __forceinline__ uint32_t codeOf(float x, float amax, float scale) {
    if (amax == 0.0f) return 0;
    float t = x / scale;
    if (t != t) return 0;
    t = rintf(t);
    t = t > 127.0f ? 127.0f : (t < -127.0f ? -127.0f : t);
    return uint32_t(int32_t(t)) & 0xFFu;
}

// Codes of one 16-byte vector of a row.  q = clamp(rint(x / s), -127, 127) needs the
// correctly rounded quotient only to decide which side of a half-integer it falls on, so
// the common path multiplies by r = 1/s (both IEEE, once per row) and rounds:
//  * |x| <= 127 s, so |x*r - x/s| <= 127 (2^-24 + 2^-24 + 2^-48) < 1.52e-5 and the
//    correctly rounded x/s is within another 127 * 2^-25 < 3.8e-6 of x/s: together
//    < 1.9e-5 < 2^-15, so when x*r is farther than 2^-15 from every half-integer both
//    quotients round to the same integer (and the clamp is a no-op: |x*r| <= 127.00001);
//  * when s is a power of two, x*r == x/s exactly, so x*r is always right;
//  * x = +-amax/2 lands within 63.5 * 2^-24 of the tie 63.5 in every row: its code is
//    computed once per row with the IEEE quotient;
//  * anything else near a half-integer (random near-ties, ~6e-5 of the elements) or NaN
//    redoes the vector with IEEE quotients.
// 16-bit data makes exact ties common (a row whose amax has mantissa 127 has a power-of-two
// scale, and x = amax/2 recurs in most rows): handling them without the IEEE path took the
// quantizer from a divergent slow path on ~60 % of wavefront-vectors to ~3 %.
struct RowQuantizer {
    float amax, scale, recip, half;
    uint32_t half_code;
    bool pow2, exact_only;
    __device__ explicit RowQuantizer(float a) : amax(a), scale(a / 127.0f) {
        recip = 1.0f / scale;
        exact_only = !(scale >= 0x1p-120f);
        pow2 = (__float_as_uint(scale) & 0x7FFFFFu) == 0;
        half = a * 0.5f;
        half_code = codeOf(half, amax, scale);
    }
    template <int N>
    __device__ __forceinline__ void codes(const float *x, uint32_t *c) const {
        bool slow = exact_only;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float t = x[e] * recip;
            const float q = rintf(t);
            const bool is_half = fabsf(x[e]) == half;
            const bool near = !(fabsf(t - q) < 0.5f - 0x1p-15f); // also true for NaN
            slow |= near && !is_half && !(pow2 && t == t);
            const uint32_t hc = x[e] < 0.0f ? (0u - half_code) : half_code;
            c[e] = (is_half ? hc : uint32_t(int32_t(q))) & 0xFFu;
        }
        if (__builtin_expect(slow, 0)) {
#pragma unroll
            for (int e = 0; e < N; ++e) c[e] = codeOf(x[e], amax, scale);
        }
    }
};

template <int N>
__device__ __forceinline__ void storeCodes(int8_t *q, size_t i, const uint32_t *c) {
    if constexpr (N == 8) {
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        const v2u r{c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24),
                    c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24)};
        __builtin_nontemporal_store(r, reinterpret_cast<v2u *>(q + i));
    } else {
        __builtin_nontemporal_store(c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24),
                                    reinterpret_cast<uint32_t *>(q + i));
    }
}

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
    float amax = 0.0f;
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = lane + v * G;
        if (live && vi < nvec) raw[v] = load16Stream<T>(in, base + size_t(vi) * N);
    }
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
    const RowQuantizer qz(amax);
    if (live && lane == 0) scale[row] = qz.scale;
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = lane + v * G;
        if (live && vi < nvec) {
            float x[N];
            uint32_t c[N];
            F::unpack(raw[v], x);
            qz.codes<N>(x, c);
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
