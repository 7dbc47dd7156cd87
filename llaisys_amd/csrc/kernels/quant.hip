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
// the scale by the group's first lane.  Rows of at most 32 vectors (KV cache rows) take
// quantGroup (one vector per lane, one-wavefront blocks), rows of 65..1152 vectors
// quantWave (one wavefront per row), others quantRows.  A KV-cache append is this kernel
// pointed at the cache rows pos .. pos + n_tok, so the codes go straight into the cache; k and v of an
// append go through one launch (two jobs), which saves a launch's fixed cost of about
// 2 us (fill, first-load latency, drain) on a 25 MB job.
#include "common.hpp"
#include "launch.hpp"
#include "quantize.hpp"
#include "rowplan.hpp"

#include <algorithm>
#include <type_traits>

namespace llaisys::kernels {

namespace {

// Up to two quantizations of rows of the same length and type in one launch (k and v of a
// KV append): blocks [0, nb0) take job 0, the rest job 1.
struct QuantJob {
    int8_t *q;
    float *scale;
    const void *in;
    size_t rows;
};
struct QuantJobs {
    QuantJob job[2];
    unsigned nb0;
};

template <typename T, int G, int VMAX>
__global__ void __launch_bounds__(blockFor<G>())
    quantRows(QuantJobs jobs, int cols) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    constexpr int kBlock = blockFor<G>();
    __shared__ float red[kBlock / kWave];

    const bool second = blockIdx.x >= jobs.nb0; // block-uniform
    int8_t *__restrict__ q = second ? jobs.job[1].q : jobs.job[0].q;
    float *__restrict__ scale = second ? jobs.job[1].scale : jobs.job[0].scale;
    const void *__restrict__ in = second ? jobs.job[1].in : jobs.job[0].in;
    const size_t rows = second ? jobs.job[1].rows : jobs.job[0].rows;
    const unsigned blk = second ? blockIdx.x - jobs.nb0 : blockIdx.x;
    const int lane = threadIdx.x % G;
    const size_t row = size_t(blk) * (kBlock / G) + threadIdx.x / G;
    const bool live = row < rows;
    const int nvec = cols / N;
    const size_t base = row * size_t(cols);

    // unconditional loads (a dead row or a slot past the row end reads the row's first
    // vector; the folds below skip those): loads under a per-lane branch were issued one
    // round trip at a time (MI355X, bf16: W[1536, 8960] 9.61 -> 9.09 us, KV pair
    // [32768, 2, 128] 11.79 -> 11.58 us).  The fold keeps its branch: a select there
    // measured slower on the 8960-wide rows.
    const size_t lbase = live ? base : 0;
    v4u raw[VMAX];
#pragma unroll
    for (int v = 0; v < VMAX; ++v) {
        const int vi = lane + v * G;
        raw[v] = load16Stream<T>(in, lbase + size_t(vi < nvec ? vi : 0) * N);
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

// Rows of at most 64 * V vectors: one wavefront per row, four rows per block, the row's
// vectors lane + 64 v in registers; amax by wave butterflies only (no LDS, no block
// barrier).  Same results as quantRows.  Measured on MI355X (W[8960, 1536] bf16, graph-
// replayed medians over >= 1 GiB of rotating sets): 8.64 us against 9.0 us for quantRows
// with the same lane plan; V = 4 ran faster than V = 3 (8.94 us) on these 192-vector rows
// while both masked the slots past the row end.  kFull (rows of exactly V * 64 vectors,
// the wave index wave-uniform): no masks, no dead slot; the launcher takes it at V = 3 for
// 192-vector rows, 8.70-8.82 -> 8.57-8.73 us (same-box A/B, 3 runs each; the uniform wave
// index alone, at V = 4, measured slower: 9.26-9.44 us), V = 4 for other rows of 65..256
// vectors.  Rows of 257..1152 vectors take
// V = 8 / 12 / 18 in one-wavefront blocks: W[1536, 8960] 8.74 us against 9.15 us for
// quantRows (256 lanes per row) and 9.01 / 10.18 us for 2 / 4 rows per block (at
// W[8960, 1536] one-wavefront blocks made no difference: 8.63 against 8.67 us).
template <typename T, int V, int B, bool kFull = false>
__global__ void __launch_bounds__(B)
    quantWave(QuantJobs jobs, int nvec_arg) {
    const int nvec = kFull ? V * kWave : nvec_arg;
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    const bool second = blockIdx.x >= jobs.nb0; // block-uniform
    int8_t *__restrict__ q = second ? jobs.job[1].q : jobs.job[0].q;
    float *__restrict__ scale = second ? jobs.job[1].scale : jobs.job[0].scale;
    const v4u *__restrict__ in = static_cast<const v4u *>(second ? jobs.job[1].in : jobs.job[0].in);
    const size_t rows = second ? jobs.job[1].rows : jobs.job[0].rows;
    const unsigned blk = second ? blockIdx.x - jobs.nb0 : blockIdx.x;
    const int lane = int(threadIdx.x) % kWave;
    // kFull: the wave index as a wave-uniform value (with the masked slots it measured slower)
    const int wv = kFull ? __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave) : int(threadIdx.x) / kWave;
    const size_t row = size_t(blk) * (B / kWave) + size_t(wv);
    const bool live = row < rows;
    const size_t base = (live ? row : 0) * size_t(nvec); // in vectors
    v4u raw[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int vi = lane + v * kWave;
        raw[v] = __builtin_nontemporal_load(in + base + (vi < nvec ? vi : 0));
    }
    // vectors past the row end fold as zeros: a select, not a branch (a branch here made
    // the compiler wait for every load before the first fold)
    using A = AbsBits<T>;
    uint32_t bits = 0;
#pragma unroll
    for (int v = 0; v < V; ++v)
        bits = A::fold(bits, lane + v * kWave < nvec ? raw[v] : v4u{0u, 0u, 0u, 0u});
    bits = waveGroupReduce<kWave, MaxU32Op>(A::finish(bits));
    float amax = A::value(bits);
    if (__builtin_expect(bits > A::kInf, 0)) { // a NaN in the row: the float rule
        amax = 0.0f;
#pragma unroll
        for (int v = 0; v < V; ++v) {
            float x[N];
            F::unpack(lane + v * kWave < nvec ? raw[v] : v4u{0u, 0u, 0u, 0u}, x);
#pragma unroll
            for (int e = 0; e < N; ++e) amax = MaxOp::apply(amax, fabsf(x[e]));
        }
        amax = waveGroupReduce<kWave, MaxOp>(amax);
    }
    const RowQuantizer qz(amax);
    if (live && lane == 0) scale[row] = qz.scale;
    const size_t cbase = base * N; // in codes
    if (__builtin_expect(qz.exact_only, 0)) {
        for (int j = lane; live && j < nvec * N; j += kWave)
            q[cbase + j] = int8_t(codeOf(F::get(in, cbase + j), amax, qz.scale));
        return;
    }
#pragma unroll
    for (int v = 0; v < V; ++v) {
        const int vi = lane + v * kWave;
        if (live && vi < nvec) {
            float x[N];
            uint32_t c[N];
            F::unpack(raw[v], x);
            qz.fastCodes<N, std::is_same_v<T, F32>>(x, c);
            storeCodes<N>(q, cbase + size_t(vi) * N, c);
        }
    }
}

// Rows of at most G <= 32 vectors (KV cache rows: head_dim 64 / 128 / 256 in 16-bit
// types): G lanes per row, one vector per lane, blocks of one wavefront (64 / G rows).
// Same results as quantRows.  Measured on MI355X (KV append pair [32768, 2, 128] bf16,
// graph-replayed medians over >= 1 GiB of rotating sets): 10.27 us against 11.65 us for
// quantRows (G = 16 in 256-thread blocks); the same kernel in blocks of 128 / 256 / 512
// threads took 11.05 / 11.08 / 11.25 us, and 2 or 4 rows per lane group 11.09 / 11.34 us.
template <typename T, int G>
__global__ void __launch_bounds__(kWave)
    quantGroup(QuantJobs jobs, int nvec) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    const bool second = blockIdx.x >= jobs.nb0; // block-uniform
    int8_t *__restrict__ q = second ? jobs.job[1].q : jobs.job[0].q;
    float *__restrict__ scale = second ? jobs.job[1].scale : jobs.job[0].scale;
    const v4u *__restrict__ in = static_cast<const v4u *>(second ? jobs.job[1].in : jobs.job[0].in);
    const size_t rows = second ? jobs.job[1].rows : jobs.job[0].rows;
    const unsigned blk = second ? blockIdx.x - jobs.nb0 : blockIdx.x;
    const int lane = int(threadIdx.x) % G;
    const size_t row = size_t(blk) * (kWave / G) + threadIdx.x / G;
    const bool live = row < rows;
    const bool inrow = lane < nvec;
    const size_t base = (live ? row : 0) * size_t(nvec); // in vectors
    // unconditional load (a dead row or a lane past the row end reads a valid vector and
    // folds as zero)
    const v4u raw = __builtin_nontemporal_load(in + base + (inrow ? lane : 0));
    const v4u val = inrow ? raw : v4u{0u, 0u, 0u, 0u};
    using A = AbsBits<T>;
    const uint32_t bits = waveGroupReduce<G, MaxU32Op>(A::finish(A::fold(0u, val)));
    float amax = A::value(bits);
    if (__builtin_expect(bits > A::kInf, 0)) { // a NaN in the row: the float rule
        float x[N];
        F::unpack(val, x);
        amax = 0.0f;
#pragma unroll
        for (int e = 0; e < N; ++e) amax = MaxOp::apply(amax, fabsf(x[e]));
        amax = waveGroupReduce<G, MaxOp>(amax);
    }
    const RowQuantizer qz(amax);
    if (live && lane == 0) scale[row] = qz.scale;
    const size_t cbase = base * N; // in codes
    if (__builtin_expect(qz.exact_only, 0)) {
        for (int j = lane; live && j < nvec * N; j += G)
            q[cbase + j] = int8_t(codeOf(F::get(in, cbase + j), amax, qz.scale));
        return;
    }
    if (live && inrow) {
        float x[N];
        uint32_t c[N];
        F::unpack(raw, x);
        qz.fastCodes<N, std::is_same_v<T, F32>>(x, c);
        storeCodes<N>(q, cbase + size_t(lane) * N, c);
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
void launch(const QuantJob &j0, const QuantJob &j1, size_t cols, hipStream_t s) {
    constexpr int N = Fmt<T>::kVec;
    const auto vecOk = [&](const QuantJob &j) {
        return j.rows == 0 || (aligned16(j.in) && reinterpret_cast<uintptr_t>(j.q) % N == 0);
    };
    const bool vec = cols > 0 && cols % N == 0 && cols <= size_t(INT32_MAX) && vecOk(j0) && vecOk(j1);
    if (vec && cols / N <= 32) {
        const int nvec = int(cols / N);
        const auto go = [&](auto g) {
            constexpr int G = decltype(g)::value;
            const unsigned nb0 = blocksFor(j0.rows, kWave / G), nb1 = blocksFor(j1.rows, kWave / G);
            if (nb0 + nb1 == 0) return;
            quantGroup<T, G><<<nb0 + nb1, kWave, 0, s>>>(QuantJobs{{j0, j1}, nb0}, nvec);
        };
        if (nvec <= 4) go(std::integral_constant<int, 4>{});
        else if (nvec <= 8) go(std::integral_constant<int, 8>{});
        else if (nvec <= 16) go(std::integral_constant<int, 16>{});
        else go(std::integral_constant<int, 32>{});
        return;
    }
    if (vec && cols / N > 64 && cols / N <= 256) {
        const unsigned nb0 = blocksFor(j0.rows, 256 / kWave), nb1 = blocksFor(j1.rows, 256 / kWave);
        if (nb0 + nb1 == 0) return;
        if (cols / N == 192)
            quantWave<T, 3, 256, true><<<nb0 + nb1, 256, 0, s>>>(QuantJobs{{j0, j1}, nb0}, int(cols / N));
        else
            quantWave<T, 4, 256><<<nb0 + nb1, 256, 0, s>>>(QuantJobs{{j0, j1}, nb0}, int(cols / N));
        return;
    }
    if (vec && cols / N > 256 && cols / N <= 18 * 64) {
        const int nvec = int(cols / N);
        const unsigned nb0 = unsigned(j0.rows), nb1 = unsigned(j1.rows); // rows < 2^30
        if (nb0 + nb1 == 0) return;
        const QuantJobs jobs{{j0, j1}, nb0};
        if (nvec <= 8 * 64)
            quantWave<T, 8, kWave><<<nb0 + nb1, kWave, 0, s>>>(jobs, nvec);
        else if (nvec <= 12 * 64)
            quantWave<T, 12, kWave><<<nb0 + nb1, kWave, 0, s>>>(jobs, nvec);
        else
            quantWave<T, 18, kWave><<<nb0 + nb1, kWave, 0, s>>>(jobs, nvec);
        return;
    }
    RowPlan plan = vec ? planRow(cols / N) : RowPlan{};
    bool done = false;
    withPlan(plan, [&](auto g, auto v) {
        constexpr int G = decltype(g)::value, V = decltype(v)::value;
        constexpr int kBlock = blockFor<G>();
        const unsigned nb0 = blocksFor(j0.rows, kBlock / G), nb1 = blocksFor(j1.rows, kBlock / G);
        if (nb0 + nb1 == 0) return;
        quantRows<T, G, V><<<nb0 + nb1, kBlock, 0, s>>>(QuantJobs{{j0, j1}, nb0}, int(cols));
        done = true;
    });
    if (done) return;
    for (const QuantJob *j : {&j0, &j1})
        if (j->rows)
            quantRowsScalar<T><<<unsigned(j->rows), 256, 0, s>>>(j->q, j->scale, j->in, j->rows, cols);
}

template <typename T>
void launchAny(const QuantJob &j0, const QuantJob &j1, size_t cols, hipStream_t s) {
    // a job too large for the block index space is split; real KV / weight shapes never are
    constexpr size_t kMaxRows = size_t(1) << 29; // both jobs' blocks fit a 31-bit grid
    if (j0.rows > kMaxRows || j1.rows > kMaxRows) {
        for (const QuantJob *j : {&j0, &j1})
            for (size_t r = 0; r < j->rows; r += kMaxRows) {
                const QuantJob part{j->q + r * cols, j->scale + r,
                                    static_cast<const char *>(j->in) + r * cols * Fmt<T>::kBytes,
                                    std::min(kMaxRows, j->rows - r)};
                launch<T>(part, QuantJob{}, cols, s);
            }
        return;
    }
    launch<T>(j0, j1, cols, s);
}

} // namespace

void quantizeInt8Pair(int8_t *q0, float *scale0, const void *in0, size_t rows0, int8_t *q1,
                      float *scale1, const void *in1, size_t rows1, size_t cols,
                      llaisysDataType_t dt, hipStream_t s) {
    const QuantJob j0{q0, scale0, in0, rows0}, j1{q1, scale1, in1, rows1};
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launchAny<F32>(j0, j1, cols, s);
    case LLAISYS_DTYPE_BF16: return launchAny<BF16>(j0, j1, cols, s);
    case LLAISYS_DTYPE_F16: return launchAny<F16>(j0, j1, cols, s);
    default: return;
    }
}

void quantizeInt8(int8_t *q, float *scale, const void *in, size_t rows, size_t cols,
                  llaisysDataType_t dt, hipStream_t s) {
    quantizeInt8Pair(q, scale, in, rows, nullptr, nullptr, nullptr, 0, cols, dt, s);
}

} // namespace llaisys::kernels
