// Argmax for gfx950: flat (the reference op) and per row (logits [rows, vocab]).
//
// Semantics: reference src/ops/argmax/cpu/argmax_cpu.cpp:14-27 -- seed with element 0,
// replace only on a strictly greater f32 value.  Equivalently: the lowest index whose
// value is the maximum over the non-NaN elements; index 0 when element 0 is NaN or when no
// element is greater than -inf.  max_val is T(f32 value of that element).
//
// Design: HBM-bound reduction.  Each lane scans its own 16-byte vectors in ascending
// order (the max of a vector is found with compares first; the index is searched only
// when that max beats the lane's best, which is rare on real logits), then (value, index)
// pairs are merged across the wavefront with butterflies and across wavefronts through
// LDS, ties going to the lower index.  Rows: one 256-thread block per row.  Flat: the
// vector is cut into segments, one block each; every block folds its best into one
// device-scope 64-bit atomic maximum of (value bits, ~index) and the last block to arrive
// (a device-scope counter) reads it, all in one launch and with no L2 write-back fence
// (above 2^32 elements: partials behind a fence, merged by the last block).
// The final write uses the values the scans already hold (element 0 and the winner), so
// no input element is re-read after the merge.
//
// Latency (MI355X, [1, 151936] bf16): 5.6 us with the atomic maximum (6.6-7.0 us when
// every block stored a partial behind an agent-scope fence, which writes back the L2);
// a near-empty launch is 1.6 us and one HBM round trip about 1.2 us.  One 1024-thread block issuing all its
// loads at once took 17 us: a single CU keeps too few misses in flight to stream 300 KB,
// so the vector is spread over 19 blocks and the cross-block merge stays.
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

#include <climits>

namespace llaisys::kernels {

namespace {

constexpr int kBlock = 256;     // flat argmax: many blocks over one vector
// Rows: one block per row.  512 threads measured 92.1 us against 94.0 us with 256 on
// [2048, 151936] bf16 (MI355X, rotating sets; a read-only kernel over the same bytes takes
// 89.2 us).
constexpr int kRowBlock = 512;
constexpr int kU = 4;
constexpr int64_t kNone = INT64_MAX;

struct Best {
    float v;
    int64_t i;
};

__device__ __forceinline__ void take(Best &b, float v, int64_t i) {
    if (v > b.v || (v == b.v && i < b.i)) {
        b.v = v;
        b.i = i;
    }
}

// Merge of the whole block of B threads; the result is valid in thread 0.
template <int B = kBlock>
__device__ Best blockMerge(Best b) {
    __shared__ float sv[B / kWave];
    __shared__ int64_t si[B / kWave];
#pragma unroll
    for (int m = kWave / 2; m > 0; m >>= 1) {
        const float ov = __shfl_xor(b.v, m, kWave);
        const int64_t oi = __shfl_xor(b.i, m, kWave);
        take(b, ov, oi);
    }
    const int wave = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) {
        sv[wave] = b.v;
        si[wave] = b.i;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < B / kWave; ++w) take(b, sv[w], si[w]);
    return b;
}

// Scan of [begin, end) by the block; thread-local order is ascending.
// Thread 0 reads element `begin` first (the first vector's element 0, or the first tail
// element when there is no vector); its value is returned in *x0 for that thread.
template <typename T, int B = kBlock>
__device__ Best scan(const void *vals, size_t begin, size_t end, bool vec, float *x0) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    Best b{-INFINITY, kNone};
    size_t tail = begin;
    if (vec) {
        const size_t nv = (end - begin) / N;
        tail = begin + nv * N;
        for (size_t k = threadIdx.x; k < nv; k += B * kU) {
            v4u r[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u)
                if (k + u * B < nv) r[u] = load16Stream<T>(vals, begin + (k + u * B) * N);
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                if (k + u * B < nv) {
                    float f[N];
                    F::unpack(r[u], f);
                    if (k + u * B == 0) *x0 = f[0];
                    float m = -INFINITY;
#pragma unroll
                    for (int e = 0; e < N; ++e) m = f[e] > m ? f[e] : m;
                    if (m > b.v) {
                        int first = N - 1;
#pragma unroll
                        for (int e = N - 1; e >= 0; --e) first = f[e] == m ? e : first;
                        b.v = m;
                        b.i = int64_t(begin + (k + u * B) * N + first);
                    }
                }
            }
        }
    }
    for (size_t j = tail + threadIdx.x; j < end; j += B) {
        const float x = F::get(vals, j);
        if (j == begin) *x0 = x;
        if (x > b.v) {
            b.v = x;
            b.i = int64_t(j);
        }
    }
    return b;
}

// Writes the final answer (thread 0 only) without re-reading the input: x0 is the range's
// first element and b.v the winner's f32 value, which converts back to T exactly (T -> f32
// -> T is the identity for bf16 / f16 / f32 under the reference rounding, NaNs included).
template <typename T>
__device__ void finish(Best b, float x0, void *idx, bool i64, void *val, size_t slot) {
    using F = Fmt<T>;
    const bool at0 = b.i == kNone || x0 != x0;
    if (i64)
        static_cast<int64_t *>(idx)[slot] = at0 ? 0 : b.i;
    else
        static_cast<int32_t *>(idx)[slot] = at0 ? 0 : int32_t(b.i);
    F::put(val, slot, at0 ? x0 : b.v);
}

template <typename T>
__global__ void __launch_bounds__(kRowBlock)
    argmaxRowsKernel(void *idx, bool i64, void *val, const void *__restrict__ vals, size_t cols,
                     bool vec) {
    const size_t first = size_t(blockIdx.x) * cols;
    float x0 = 0.0f;
    Best b = blockMerge<kRowBlock>(scan<T, kRowBlock>(vals, first, first + cols, vec, &x0));
    if (b.i != kNone) b.i -= int64_t(first);
    if (threadIdx.x == 0) finish<T>(b, x0, idx, i64, val, blockIdx.x);
}

struct Partial {
    uint32_t vbits;
    uint32_t x0bits; // element 0 (block 0's partial only)
    int64_t i;
};

template <typename T>
__global__ void __launch_bounds__(kBlock)
    argmaxFlatKernel(void *idx, bool i64, void *val, const void *__restrict__ vals, size_t n,
                     size_t seg, bool vec, unsigned *counter, Partial *part) {
    __shared__ bool last;
    const size_t begin = size_t(blockIdx.x) * seg;
    const size_t end = begin + seg < n ? begin + seg : n;
    float x0 = 0.0f;
    Best b = blockMerge(scan<T>(vals, begin, end, vec, &x0));
    if (threadIdx.x == 0) {
        part[blockIdx.x].vbits = __float_as_uint(b.v);
        part[blockIdx.x].x0bits = __float_as_uint(x0);
        part[blockIdx.x].i = b.i;
        __threadfence();
        last = atomicAdd(counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence();
    Best m{-INFINITY, kNone};
    float x0_all = 0.0f; // thread 0 reads partial 0
    for (unsigned p = threadIdx.x; p < gridDim.x; p += kBlock) {
        // Device-scope loads: other blocks' partials must not come from a stale L1 line.
        const uint32_t vb = __hip_atomic_load(&part[p].vbits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int64_t pi = __hip_atomic_load(&part[p].i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (p == 0)
            x0_all = __uint_as_float(__hip_atomic_load(&part[0].x0bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        take(m, __uint_as_float(vb), pi);
    }
    m = blockMerge(m);
    if (threadIdx.x == 0) {
        finish<T>(m, x0_all, idx, i64, val, 0);
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Flat argmax for n < 2^32 without partials or fences: every block folds its best
// (value, index) into one device-scope 64-bit atomic maximum of the key
// (order-preserving bits of the value) << 32 | ~index -- a larger value, then a lower
// index, makes a larger key; a block with no candidate (all -inf / NaN) skips it.  The
// atomic returns its old value, and the wait for it orders the maximum before the block's
// arrival count; the last block to arrive reads the key (and element 0) with device-scope
// loads, finishes, and leaves key and counter zero.  Device-scope atomics are performed at
// the device's coherence point, so no L2 write-back fence is needed between blocks.
struct FlatSlots {
    unsigned counter; // the launch's arrival count (offset 0 of the scratch)
    unsigned x0bits;  // element 0, stored by block 0 before it arrives
    unsigned long long key;
};

__device__ __forceinline__ uint32_t orderBits(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <typename T>
__global__ void __launch_bounds__(kBlock)
    argmaxFlatAtomic(void *idx, bool i64, void *val, const void *__restrict__ vals, size_t n,
                     size_t seg, bool vec, FlatSlots *sl) {
    const size_t begin = size_t(blockIdx.x) * seg;
    const size_t end = begin + seg < n ? begin + seg : n;
    float x0 = 0.0f;
    Best b = blockMerge(scan<T>(vals, begin, end, vec, &x0));
    if (threadIdx.x != 0) return;
    unsigned long long seen = 0;
    if (blockIdx.x == 0)
        seen += __hip_atomic_exchange(&sl->x0bits, __float_as_uint(x0), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (b.i != kNone) {
        const unsigned long long key = (uint64_t(orderBits(b.v)) << 32) | uint64_t(~uint32_t(b.i));
        seen += __hip_atomic_fetch_max(&sl->key, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Consuming the returned values keeps both atomics in their returning form, and the
    // wait completes them before the arrival is counted.
    asm volatile("s_waitcnt vmcnt(0)" : "+v"(seen)::"memory");
    if (__hip_atomic_fetch_add(&sl->counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != gridDim.x - 1)
        return;
    const unsigned long long key = __hip_atomic_load(&sl->key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float x0_all = __uint_as_float(__hip_atomic_load(&sl->x0bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    Best m{-INFINITY, kNone};
    if (key != 0) {
        const uint32_t ob = uint32_t(key >> 32);
        m.v = __uint_as_float((ob & 0x80000000u) ? (ob & 0x7FFFFFFFu) : ~ob);
        m.i = int64_t(~uint32_t(key));
    }
    finish<T>(m, x0_all, idx, i64, val, 0);
    __hip_atomic_store(&sl->key, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&sl->counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

constexpr size_t kCounterBytes = kScratchReserved;

template <typename T>
size_t segmentOf() {
    return size_t(kBlock) * kU * Fmt<T>::kVec;
}

size_t segmentFor(llaisysDataType_t dt) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return segmentOf<F32>();
    default: return segmentOf<BF16>();
    }
}

template <typename T>
void launchRows(void *idx, bool i64, void *val, const void *vals, size_t rows, size_t cols,
                hipStream_t s) {
    if (rows == 0 || cols == 0) return;
    const bool vec = aligned16(vals) && (cols * Fmt<T>::kBytes) % 16 == 0;
    argmaxRowsKernel<T><<<unsigned(rows), kRowBlock, 0, s>>>(idx, i64, val, vals, cols, vec);
}

template <typename T>
void launchFlat(void *idx, bool i64, void *val, const void *vals, size_t n, void *ws,
                hipStream_t s) {
    if (n == 0) return;
    const size_t seg = segmentOf<T>();
    const unsigned blocks = unsigned((n + seg - 1) / seg);
    if (n < (size_t(1) << 32)) {
        argmaxFlatAtomic<T><<<blocks, kBlock, 0, s>>>(idx, i64, val, vals, n, seg, aligned16(vals),
                                                      static_cast<FlatSlots *>(ws));
        return;
    }
    auto *counter = static_cast<unsigned *>(ws);
    auto *part = reinterpret_cast<Partial *>(static_cast<char *>(ws) + kCounterBytes);
    argmaxFlatKernel<T><<<blocks, kBlock, 0, s>>>(idx, i64, val, vals, n, seg, aligned16(vals),
                                                  counter, part);
}

} // namespace

size_t argmaxWorkspaceBytes(size_t n, llaisysDataType_t dt) {
    const size_t seg = segmentFor(dt);
    return kCounterBytes + ((n + seg - 1) / seg) * sizeof(Partial);
}

void argmaxRows(void *idx, bool i64, void *val, const void *vals, size_t rows, size_t cols,
                llaisysDataType_t dt, hipStream_t s) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launchRows<F32>(idx, i64, val, vals, rows, cols, s);
    case LLAISYS_DTYPE_BF16: return launchRows<BF16>(idx, i64, val, vals, rows, cols, s);
    case LLAISYS_DTYPE_F16: return launchRows<F16>(idx, i64, val, vals, rows, cols, s);
    default: return;
    }
}

void argmax(void *idx, bool i64, void *val, const void *vals, size_t n, llaisysDataType_t dt,
            void *ws, hipStream_t s) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launchFlat<F32>(idx, i64, val, vals, n, ws, s);
    case LLAISYS_DTYPE_BF16: return launchFlat<BF16>(idx, i64, val, vals, n, ws, s);
    case LLAISYS_DTYPE_F16: return launchFlat<F16>(idx, i64, val, vals, n, ws, s);
    default: return;
    }
}

} // namespace llaisys::kernels
