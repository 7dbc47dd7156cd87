// Streaming element-wise kernels for gfx950: swiglu, add, INT8 dequantize, dtype cast.
//
// swiglu follows src/ops/swiglu/cpu/swiglu_cpu.cpp:15-20: out = T(u * (g / (1 + exp(-g))))
// in f32.  exp is the hardware exp2 of -g*log2(e) and the quotient is the hardware
// reciprocal refined by one Newton step (within an ulp of the IEEE quotient); against
// glibc expf and IEEE division that is a few f32 ulps, inside the 1e-5 relative (f32) and
// 2-ulp (bf16) parity bounds, and it keeps the kernel at the HBM rate (the libm exp plus
// IEEE division cost ~30 VALU ops per element, as much time as the HBM traffic).
// add follows src/ops/add/cpu/add_cpu.cpp:9-16.  dequantize is out = T(float(q) * scale[row]).
//
// Design: pure HBM streaming.  Each lane moves U 16-byte vectors per input (all loads
// issued before any math); vector k of a block is (blockIdx * U + k) * B + thread for B threads, so
// every wavefront access is one contiguous 1 KB segment.  Loads and stores are
// non-temporal.  A scalar kernel handles lengths / addresses that are not multiples of
// 16 bytes.
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

#include <algorithm>

namespace llaisys::kernels {

namespace {

// 16-byte vectors per input per lane, measured per kernel on MI355X: the binary ops
// (two streamed inputs) are fastest with one (swiglu [8192, 8960]: 69.3 us vs 71.2 with
// two, 75.1 with four); dequantize writes two output vectors per lane from 8-byte code
// loads, in 64-thread blocks (see dequantVec).
constexpr int kBinaryU = 1;
constexpr int kDequantU = 2;
constexpr int kDequantBlock = 64;
// Threads per block of the binary ops: one wavefront.  Same work per lane, only smaller
// blocks: swiglu [8192, 8960] 67.3 us vs 69.2 with 256 threads (a plain 2-in / 1-out
// stream measured the same way: 65.1 vs 66.0 us).
constexpr int kBinaryBlock = 64;

struct AddOp {
    __device__ static float apply(float a, float b) { return a + b; }
};

template <typename T, typename Op, int kU>
__global__ void __launch_bounds__(kBinaryBlock)
    binaryVec(void *__restrict__ out, const void *__restrict__ a, const void *__restrict__ b,
              size_t nvec) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    const size_t first = size_t(blockIdx.x) * kBinaryBlock * kU + threadIdx.x;
    v4u ra[kU], rb[kU];
#pragma unroll
    for (int k = 0; k < kU; ++k) {
        const size_t i = first + size_t(k) * kBinaryBlock;
        if (i < nvec) {
            ra[k] = load16Stream<T>(a, i * N);
            rb[k] = load16Stream<T>(b, i * N);
        }
    }
#pragma unroll
    for (int k = 0; k < kU; ++k) {
        const size_t i = first + size_t(k) * kBinaryBlock;
        if (i < nvec) {
            float x[N], y[N];
            F::unpack(ra[k], x);
            F::unpack(rb[k], y);
#pragma unroll
            for (int e = 0; e < N; ++e) x[e] = Op::apply(x[e], y[e]);
            store16Stream<T>(out, i * N, F::packQ(x));
        }
    }
}

template <typename T, typename Op>
__global__ void __launch_bounds__(256)
    binaryScalar(void *out, const void *a, const void *b, size_t n) {
    using F = Fmt<T>;
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256)
        F::put(out, i, Op::apply(F::get(a, i), F::get(b, i)));
}

template <typename T, typename Op>
void launchBinary(void *out, const void *a, const void *b, size_t n, hipStream_t s) {
    if (n == 0) return;
    constexpr int N = Fmt<T>::kVec;
    if (n % N == 0 && aligned16(out) && aligned16(a) && aligned16(b)) {
        const size_t nvec = n / N;
        binaryVec<T, Op, kBinaryU><<<blocksFor(nvec, kBinaryBlock * kBinaryU), kBinaryBlock, 0, s>>>(out, a, b, nvec);
        return;
    }
    const unsigned grid = unsigned(std::min<size_t>(blocksFor(n, 256), 1u << 20));
    binaryScalar<T, Op><<<grid, 256, 0, s>>>(out, a, b, n);
}

template <typename Op>
void dispatchBinary(void *out, const void *a, const void *b, size_t n, llaisysDataType_t dt,
                    hipStream_t s) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launchBinary<F32, Op>(out, a, b, n, s);
    case LLAISYS_DTYPE_BF16: return launchBinary<BF16, Op>(out, a, b, n, s);
    case LLAISYS_DTYPE_F16: return launchBinary<F16, Op>(out, a, b, n, s);
    default: return;
    }
}

// ---- INT8 dequantize --------------------------------------------------------------------

// One output vector of code * sc.  packQ rounds every non-NaN product like the reference;
// with a NaN scale (caller data) every product is the same quieted NaN, whose reference
// rounding (pack) is one value per lane, selected word by word.  Branch-free on purpose: a
// divergent branch around the stores measured 40 % slower on the whole kernel (13.9 vs
// 9.8 us, W[8960, 1536]).
template <typename T>
__device__ __forceinline__ v4u packScaled(const float *f, float sc) {
    using F = Fmt<T>;
    v4u r = F::packQ(f);
    if constexpr (F::kBytes == 2) {
        const uint32_t h = F::pack(f).x & 0xFFFFu; // the exact rounding of the lane's NaN
        const uint32_t nanw = h | (h << 16);
        const bool nan = sc != sc;
        r.x = nan ? nanw : r.x;
        r.y = nan ? nanw : r.y;
        r.z = nan ? nanw : r.z;
        r.w = nan ? nanw : r.w;
    }
    return r;
}

// N codes (one output vector) per lane: 8 bytes of codes for 16-bit outputs, 4 for f32.
template <int N>
__device__ __forceinline__ void loadCodes(const int8_t *q, size_t i, float *f) {
    if constexpr (N == 8) {
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        const v2u r = __builtin_nontemporal_load(reinterpret_cast<const v2u *>(q + i));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            f[e] = float(int8_t(r.x >> (8 * e)));
            f[4 + e] = float(int8_t(r.y >> (8 * e)));
        }
    } else {
        const uint32_t r = __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(q + i));
#pragma unroll
        for (int e = 0; e < 4; ++e) f[e] = float(int8_t(r >> (8 * e)));
    }
}

// Up to two dequantizations with the same row length and type in one launch (k and v of a
// cache read): blocks [0, nb0) take job 0, the rest job 1.
struct DequantJob {
    void *out;
    const int8_t *q;
    const float *scale;
    size_t nvec;
};
struct DequantJobs {
    DequantJob job[2];
    unsigned nb0;
};

// kU output vectors per lane, vector k of a lane at (blk * kU + k) * B + thread, so every
// store instruction of a wavefront writes one contiguous 1 KB and every code load reads
// one contiguous 256 / 512 B.  All loads (codes and the row scales) are issued before any
// arithmetic, unconditionally (a lane past the end reads vector 0 and stores nothing).
// Measured on MI355X (W[8960, 1536] bf16, graph-replayed medians over >= 1 GiB of rotating
// sets): 8.27 us with two vectors per lane in 64-thread blocks, against 9.30 us for 16
// codes per lane (one 16-byte code load, two stores 32 bytes apart per lane) in 256-thread
// blocks and 8.44 us for the same layout in 256-thread blocks.
template <typename T, int kU, int B>
__global__ void __launch_bounds__(B)
    dequantVec(DequantJobs jobs, DivU64 rowdiv) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    const bool second = blockIdx.x >= jobs.nb0; // block-uniform
    void *__restrict__ out = second ? jobs.job[1].out : jobs.job[0].out;
    const int8_t *__restrict__ q = second ? jobs.job[1].q : jobs.job[0].q;
    const float *__restrict__ scale = second ? jobs.job[1].scale : jobs.job[0].scale;
    const size_t nvec = second ? jobs.job[1].nvec : jobs.job[0].nvec;
    const unsigned blk = second ? blockIdx.x - jobs.nb0 : blockIdx.x;
    const size_t first = size_t(blk) * B * kU + threadIdx.x;
    float f[kU][N], sc[kU];
#pragma unroll
    for (int k = 0; k < kU; ++k) {
        const size_t i = first + size_t(k) * B;
        const size_t ic = i < nvec ? i : 0;
        loadCodes<N>(q, ic * N, f[k]);
        sc[k] = scale[rowdiv.div(ic)];
    }
#pragma unroll
    for (int k = 0; k < kU; ++k) {
        const size_t i = first + size_t(k) * B;
#pragma unroll
        for (int e = 0; e < N; ++e) f[k][e] = f[k][e] * sc[k];
        if (i < nvec) store16Stream<T>(out, i * N, packScaled<T>(f[k], sc[k]));
    }
}

template <typename T>
__global__ void __launch_bounds__(256)
    dequantScalar(void *out, const int8_t *q, const float *scale, size_t n, size_t cols) {
    using F = Fmt<T>;
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256)
        F::put(out, i, float(q[i]) * scale[i / cols]);
}

struct DequantArgs {
    void *out;
    const int8_t *q;
    const float *scale;
    size_t rows;
};

template <typename T>
void launchDequant(const DequantArgs &a0, const DequantArgs &a1, size_t cols, hipStream_t s) {
    constexpr int N = Fmt<T>::kVec;
    constexpr size_t kPerBlock = size_t(kDequantBlock) * kDequantU;
    const auto vecOk = [&](const DequantArgs &a) {
        return a.rows == 0 || (aligned16(a.out) && reinterpret_cast<uintptr_t>(a.q) % N == 0);
    };
    const size_t nv0 = cols % N == 0 ? a0.rows * cols / N : 0;
    const size_t nv1 = cols % N == 0 ? a1.rows * cols / N : 0;
    const size_t nb0 = (nv0 + kPerBlock - 1) / kPerBlock, nb1 = (nv1 + kPerBlock - 1) / kPerBlock;
    if (cols % N == 0 && vecOk(a0) && vecOk(a1) && nb0 + nb1 < (size_t(1) << 31)) {
        if (nb0 + nb1 == 0) return;
        const DequantJobs jobs{{DequantJob{a0.out, a0.q, a0.scale, nv0}, DequantJob{a1.out, a1.q, a1.scale, nv1}},
                               unsigned(nb0)};
        dequantVec<T, kDequantU, kDequantBlock><<<unsigned(nb0 + nb1), kDequantBlock, 0, s>>>(jobs, DivU64(cols / N));
        return;
    }
    for (const DequantArgs *a : {&a0, &a1}) {
        const size_t n = a->rows * cols;
        if (n == 0) continue;
        const unsigned grid = unsigned(std::min<size_t>(blocksFor(n, 256), 1u << 20));
        dequantScalar<T><<<grid, 256, 0, s>>>(a->out, a->q, a->scale, n, cols);
    }
}

// ---- dtype conversion ---------------------------------------------------------------------
// out[i] = cast<To>(in[i]) as the reference's types.hpp:116-139: through f32, with the
// reference rules (Fmt<T>::unpack / pack: bf16 round-half-even without a NaN case, f16
// truncation).  pack, not packQ: the inputs are caller data whose NaN payloads the
// hardware converter would not round like the reference.  Eight elements per lane: one
// or two 16-byte loads, one or two 16-byte stores.

template <typename T>
__device__ __forceinline__ void load8(const void *p, size_t i, float *f) {
    if constexpr (Fmt<T>::kVec == 8) {
        Fmt<T>::unpack(load16Stream<T>(p, i), f);
    } else {
        Fmt<T>::unpack(load16Stream<T>(p, i), f);
        Fmt<T>::unpack(load16Stream<T>(p, i + 4), f + 4);
    }
}

template <typename T>
__device__ __forceinline__ void store8(void *p, size_t i, const float *f) {
    if constexpr (Fmt<T>::kVec == 8) {
        store16Stream<T>(p, i, Fmt<T>::pack(f));
    } else {
        store16Stream<T>(p, i, Fmt<T>::pack(f));
        store16Stream<T>(p, i + 4, Fmt<T>::pack(f + 4));
    }
}

template <typename To, typename From>
__global__ void __launch_bounds__(256) castVec(void *__restrict__ out, const void *__restrict__ in, size_t n8) {
    const size_t k = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (k >= n8) return;
    float f[8];
    load8<From>(in, k * 8, f);
    store8<To>(out, k * 8, f);
}

template <typename To, typename From>
__global__ void __launch_bounds__(256) castScalar(void *out, const void *in, size_t n) {
    for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256)
        Fmt<To>::put(out, i, Fmt<From>::get(in, i));
}

template <typename To, typename From>
void launchCast(void *out, const void *in, size_t n, hipStream_t s) {
    if (n == 0) return;
    if (n % 8 == 0 && aligned16(out) && aligned16(in)) {
        castVec<To, From><<<blocksFor(n / 8, 256), 256, 0, s>>>(out, in, n / 8);
        return;
    }
    const unsigned grid = unsigned(std::min<size_t>(blocksFor(n, 256), 1u << 20));
    castScalar<To, From><<<grid, 256, 0, s>>>(out, in, n);
}

template <typename To>
void castFrom(void *out, const void *in, llaisysDataType_t in_dt, size_t n, hipStream_t s) {
    switch (in_dt) {
    case LLAISYS_DTYPE_F32: return launchCast<To, F32>(out, in, n, s);
    case LLAISYS_DTYPE_BF16: return launchCast<To, BF16>(out, in, n, s);
    case LLAISYS_DTYPE_F16: return launchCast<To, F16>(out, in, n, s);
    default: return;
    }
}

} // namespace

void swiglu(void *out, const void *gate, const void *up, size_t n, llaisysDataType_t dt,
            hipStream_t s) {
    dispatchBinary<SwigluOp>(out, gate, up, n, dt, s);
}

void add(void *c, const void *a, const void *b, size_t n, llaisysDataType_t dt, hipStream_t s) {
    dispatchBinary<AddOp>(c, a, b, n, dt, s);
}

void dequantizeInt8Pair(void *out0, const int8_t *q0, const float *scale0, size_t rows0,
                        void *out1, const int8_t *q1, const float *scale1, size_t rows1,
                        size_t cols, llaisysDataType_t dt, hipStream_t s) {
    const DequantArgs a0{out0, q0, scale0, rows0}, a1{out1, q1, scale1, rows1};
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launchDequant<F32>(a0, a1, cols, s);
    case LLAISYS_DTYPE_BF16: return launchDequant<BF16>(a0, a1, cols, s);
    case LLAISYS_DTYPE_F16: return launchDequant<F16>(a0, a1, cols, s);
    default: return;
    }
}

void dequantizeInt8(void *out, const int8_t *q, const float *scale, size_t rows, size_t cols,
                    llaisysDataType_t dt, hipStream_t s) {
    dequantizeInt8Pair(out, q, scale, rows, nullptr, nullptr, nullptr, 0, cols, dt, s);
}

void cast(void *out, llaisysDataType_t out_dt, const void *in, llaisysDataType_t in_dt, size_t n,
          hipStream_t s) {
    switch (out_dt) {
    case LLAISYS_DTYPE_F32: return castFrom<F32>(out, in, in_dt, n, s);
    case LLAISYS_DTYPE_BF16: return castFrom<BF16>(out, in, in_dt, n, s);
    case LLAISYS_DTYPE_F16: return castFrom<F16>(out, in, in_dt, n, s);
    default: return;
    }
}

} // namespace llaisys::kernels
