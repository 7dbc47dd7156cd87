// Random sampling after argmax: temperature, top-k and top-p over rows of logits.
//
// No reference kernel: README.md:397-399 asks for a random sample operator with
// temperature, top-k and top-p, and python/llaisys/models/qwen2.py:216-218 takes the three
// parameters.  The rule (z = x * (1/T); order by (z desc, index asc); keep the top k;
// integer weights w = floor(2^31 * 2^((z - zmax) log2 e)) from a fixed exp2 polynomial, with
// (z - zmax) taken as 0 for candidates tied with the top one (infinite ties included) and a
// NaN z ordered as -inf;
// top-p prefix by integer weight sum; inverse-CDF draw with a splitmix64 uniform) is made of
// integer work and IEEE single multiplies / adds in a fixed order, so every GPU result is
// bit-identical to the CPU statement of the rule whatever the thread order.
//
// Kernels per launch of up to kSampleRows rows (all on the context stream):
//   sampleHist<1..2> : top-k radix select over the order-preserving u32 key of z -- each
//                      level histograms one 11-bit digit of the keys that match the digits
//                      chosen so far; the choice of every earlier digit is recomputed by
//                      each block from the previous histograms (integer atomics: exact and
//                      order-free).  HBM / L2-bound, one read of the row.
//   sampleGather     : after the two digits, the 22-bit prefix P of the k-th largest key:
//                      the keys whose prefix is above P (< k of them) and the "bucket" of
//                      keys with prefix P (about one on real logits), both stored as sort
//                      items (~key << 32) | index.
//   sampleFinish     : one 256-thread block per row (512 when k > 256): the best `need`
//                      bucket members by (key desc, index asc) -- sorted in LDS, or, for a
//                      bucket larger than its list, by the key's last 10 bits resolved in a
//                      scan of the row --; then the k candidates sorted by (key desc, index
//                      asc) in LDS, weights, prefix sums, the top-p cut, the draw; then
//                      re-zeroes the row's histograms and counters.
// The selection is that of a full 32-bit radix select: the same k candidates.
#include "common.hpp"
#include "launch.hpp"

#include <algorithm>

namespace llaisys::kernels {

namespace {

// histogram / gather blocks: 1024 threads, 2 keys each (75 blocks over 151936 logits):
// top_k 50 22.9 -> 20.6 us against 256 threads x 8 keys (512 x 4: 21.3 us; 1024 x 1: 20.9 us)
constexpr int kSmpBlock = 1024;
constexpr int kSmpChunk = kSmpBlock * 2; // elements per histogram block
constexpr int kMaxK = 1024;
constexpr int kTieCap = 4096;

// Order-preserving key of z; a NaN z (either sign) takes the key of -inf, so it is never
// preferred to a number and ties with -inf by index.
__device__ __forceinline__ uint32_t keyOf(float z) {
    const uint32_t b = z != z ? 0xFF800000u : __float_as_uint(z);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float unkey(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// 2^t for t <= 0: degree-7 Taylor polynomial of e^(g ln 2) on g = frac(t) - 1/2, times
// sqrt(2), scaled by 2^floor(t); each step one IEEE single multiply or add (_rn: never
// contracted), so CPU and GPU agree bit for bit.
__device__ __forceinline__ float sampleExp2(float t) {
    if (!(t > -126.0f)) return 0.0f;
    const float n = floorf(t);
    const float g = __fsub_rn(__fsub_rn(t, n), 0.5f);
    float y = 1.525273380405984e-05f;
    y = __fadd_rn(__fmul_rn(y, g), 0.00015403530393381608f);
    y = __fadd_rn(__fmul_rn(y, g), 0.0013333558146428443f);
    y = __fadd_rn(__fmul_rn(y, g), 0.009618129107628477f);
    y = __fadd_rn(__fmul_rn(y, g), 0.05550410866482158f);
    y = __fadd_rn(__fmul_rn(y, g), 0.2402265069591007f);
    y = __fadd_rn(__fmul_rn(y, g), 0.6931471805599453f);
    y = __fadd_rn(__fmul_rn(y, g), 1.0f);
    return ldexpf(__fmul_rn(y, 1.4142135623730951f), int(n));
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// per-row state in the reserved (zero between launches) scratch
struct SmpRow {
    uint32_t h1[2048];
    uint32_t h2[2048];
    uint32_t nGt, nTie, theta, need; // counters; the 22-bit prefix P and the bucket members it takes
};
static_assert(sizeof(SmpRow) == kSampleRowStateBytes, "sampler state layout");

struct SmpArgs {
    const void *x;
    void *out;
    bool i64;
    int V, k, rows;
    float inv, topP;
    uint64_t seed;
    SmpRow *st;      // rows entries, reserved scratch
    uint64_t *gt;    // rows x kMaxK candidates with a prefix above P: (~key << 32) | index
    uint64_t *ties;  // rows x kTieCap bucket members (prefix P), as the same items
};

// Inclusive suffix sum within the wavefront (lane l: the sum over lanes l .. 63).
__device__ __forceinline__ uint32_t waveSuffix(uint32_t v) {
    const int lane = int(threadIdx.x) % kWave;
#pragma unroll
    for (int d = 1; d < kWave; d *= 2) {
        const uint32_t o = __shfl_down(v, d, kWave);
        if (lane + d < kWave) v += o;
    }
    return v;
}

// LDS scratch of one radix decision: the wave totals and the (bin, inside) result.
struct BinScratch {
    uint32_t wtot[1024 / kWave];
    uint32_t bin, in;
};

// Largest bin b of lh[0..n) (a histogram already in LDS) whose suffix count reaches `need`;
// returns b and, in *inside, need minus the count above b.  All kSmpBlock threads call it.
// Thread t owns bins [t*per, (t+1)*per); the suffix sums over the threads come from wave
// shuffles and one exchange of the wave totals (two block barriers in all).
template <int NB = kSmpBlock>
__device__ int chooseBin(const uint32_t *lh, int n, uint32_t need, uint32_t *inside, BinScratch &bs) {
    static_assert(NB / kWave <= int(sizeof(BinScratch::wtot) / sizeof(uint32_t)), "wave totals");
    const int t = int(threadIdx.x), w = t / kWave;
    const int per = n / NB;
    uint32_t s = 0;
    for (int j = 0; j < per; ++j) s += lh[t * per + j];
    const uint32_t v = waveSuffix(s);
    if (t % kWave == 0) bs.wtot[w] = v;
    __syncthreads();
    uint32_t suf = v; // count in bins >= t*per
    for (int x = w + 1; x < NB / kWave; ++x) suf += bs.wtot[x];
    const uint32_t above = suf - s; // count in bins >= (t+1)*per
    // the thread whose range holds the crossing resolves it
    if (above < need && suf >= need) {
        uint32_t acc = above;
        for (int j = per - 1; j >= 0; --j) {
            const uint32_t c = lh[t * per + j];
            if (acc + c >= need) {
                bs.bin = uint32_t(t * per + j);
                bs.in = need - acc;
                break;
            }
            acc += c;
        }
    }
    __syncthreads();
    *inside = bs.in;
    return int(bs.bin);
}

// LDS for decide(): the row's two histograms and one BinScratch per level
struct DecideLds {
    uint32_t h[2048 + 2048];
    BinScratch bs[2];
};

// the digits chosen after `level` histograms: prefix (the key's top bits) and the count
// still needed among keys with that prefix.  The histograms are final when this runs, so
// all the levels' are staged in one round of loads.
__device__ void decide(const SmpRow &st, int level, uint32_t k, uint32_t *prefix, uint32_t *need,
                       DecideLds &L) {
    const int t = int(threadIdx.x);
    for (int b = t; b < 2048; b += kSmpBlock) L.h[b] = st.h1[b];
    if (level >= 2)
        for (int b = t; b < 2048; b += kSmpBlock) L.h[2048 + b] = st.h2[b];
    __syncthreads();
    uint32_t nd = k, p = 0;
    if (level >= 1) p = uint32_t(chooseBin(L.h, 2048, nd, &nd, L.bs[0]));
    if (level >= 2) p = (p << 11) | uint32_t(chooseBin(L.h + 2048, 2048, nd, &nd, L.bs[1]));
    *prefix = p;
    *need = nd;
}

template <typename T>
__device__ __forceinline__ uint32_t keyAt(const SmpArgs &a, int row, int i) {
    return keyOf(__fmul_rn(Fmt<T>::get(a.x, size_t(row) * a.V + i), a.inv));
}

// LEVEL 1..3: histogram of digit LEVEL of the keys matching the chosen prefix
template <typename T, int LEVEL>
__global__ void __launch_bounds__(kSmpBlock)
    sampleHist(SmpArgs a) {
    __shared__ uint32_t hist[2048];
    const int row = int(blockIdx.y);
    SmpRow &st = a.st[row];
    // the block's keys first: their loads and the histogram staging of decide() share one
    // round trip
    const int base = int(blockIdx.x) * kSmpChunk;
    constexpr int kPer = kSmpChunk / kSmpBlock;
    uint32_t keys[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = base + j * kSmpBlock + int(threadIdx.x);
        keys[j] = keyAt<T>(a, row, i < a.V ? i : a.V - 1);
    }
    uint32_t prefix = 0, need = 0;
    if constexpr (LEVEL > 1) {
        __shared__ DecideLds dl;
        decide(st, LEVEL - 1, uint32_t(a.k), &prefix, &need, dl);
    }
    static_assert(LEVEL == 1 || LEVEL == 2, "two 11-bit digits");
    constexpr int kBins = 2048;
    for (int b = int(threadIdx.x); b < kBins; b += kSmpBlock) hist[b] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = base + j * kSmpBlock + int(threadIdx.x);
        if (i >= a.V) break;
        const uint32_t key = keys[j];
        if constexpr (LEVEL == 1)
            atomicAdd(&hist[key >> 21], 1u);
        else if ((key >> 21) == prefix)
            atomicAdd(&hist[(key >> 10) & 0x7FFu], 1u);
    }
    __syncthreads();
    uint32_t *g = LEVEL == 1 ? st.h1 : st.h2;
    for (int b = int(threadIdx.x); b < kBins; b += kSmpBlock)
        if (hist[b]) atomicAdd(g + b, hist[b]);
}

// the candidates: keys above the k-th largest key, and the ties at it
template <typename T>
__global__ void __launch_bounds__(kSmpBlock)
    sampleGather(SmpArgs a) {
    __shared__ DecideLds dl;
    const int row = int(blockIdx.y);
    SmpRow &st = a.st[row];
    const int base = int(blockIdx.x) * kSmpChunk;
    constexpr int kPer = kSmpChunk / kSmpBlock;
    uint32_t keys[kPer]; // loaded before the decision (one round trip with its staging)
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = base + j * kSmpBlock + int(threadIdx.x);
        keys[j] = keyAt<T>(a, row, i < a.V ? i : a.V - 1);
    }
    uint32_t theta = 0, need = 0;
    decide(st, 2, uint32_t(a.k), &theta, &need, dl); // theta: the 22-bit prefix P
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        st.theta = theta;
        st.need = need;
    }
    // positions are reserved per block (LDS counters, then one global atomic per list), so a
    // thousand candidates do not queue on one global counter
    __shared__ uint32_t nG, nT, baseG, baseT;
    if (threadIdx.x == 0) nG = nT = 0;
    __syncthreads();
    uint32_t slot[kPer]; // bit 31: tie; else candidate; position within the block's list
    int cls[kPer];       // 0 none, 1 prefix above P, 2 prefix P (the bucket)
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int i = base + j * kSmpBlock + int(threadIdx.x);
        cls[j] = 0;
        if (i < a.V) {
            const uint32_t pre = keys[j] >> 10;
            if (pre > theta) {
                cls[j] = 1;
                slot[j] = atomicAdd(&nG, 1u);
            } else if (pre == theta) {
                cls[j] = 2;
                slot[j] = atomicAdd(&nT, 1u);
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        baseG = nG ? atomicAdd(&st.nGt, nG) : 0u;
        baseT = nT ? atomicAdd(&st.nTie, nT) : 0u;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const uint32_t i = uint32_t(base + j * kSmpBlock + int(threadIdx.x));
        if (cls[j] == 1) {
            const uint32_t pos = baseG + slot[j];
            if (pos < uint32_t(kMaxK)) a.gt[size_t(row) * kMaxK + pos] = (uint64_t(~keys[j]) << 32) | i;
        } else if (cls[j] == 2) {
            const uint32_t pos = baseT + slot[j];
            if (pos < uint32_t(kTieCap)) a.ties[size_t(row) * kTieCap + pos] = (uint64_t(~keys[j]) << 32) | i;
        }
    }
}

// ascending bitonic sort of n (power of two) 64-bit items in LDS by all threads
__device__ void bitonic(uint64_t *v, int n) {
    for (int size = 2; size <= n; size *= 2)
        for (int stride = size / 2; stride > 0; stride /= 2) {
            for (int i = int(threadIdx.x); i < n / 2; i += int(blockDim.x)) {
                const int lo = 2 * i - (i & (stride - 1)), hi = lo + stride;
                const bool up = (lo & size) == 0;
                const uint64_t x = v[lo], y = v[hi];
                if ((x > y) == up) {
                    v[lo] = y;
                    v[hi] = x;
                }
            }
            __syncthreads();
        }
}

// finish block: 256 threads, 512 when k > 256 (one compare-exchange per thread and stage
// of the 1024-item sort: top_k 1024 26.1 -> 22.0 us; 256 threads are faster up to k = 64,
// 8.1 against 9.2 us)
constexpr int kFinThreads = 256;
constexpr int kFinThreadsWide = 512;
static_assert(kMaxK <= 4 * kFinThreads, "the finish sorts k candidates as 4 per thread");

// exclusive prefix sums of v (one value per thread, NT threads): inclusive scans within
// each wavefront by shuffles, the wave totals through `buf` (NT / 64 words);
// returns this thread's exclusive sum and, in *total, the block total
template <int NT>
__device__ uint64_t blockExclusive(uint64_t v, uint64_t *buf, uint64_t *total) {
    const int t = int(threadIdx.x), lane = t % kWave, w = t / kWave;
    uint64_t inc = v;
#pragma unroll
    for (int d = 1; d < kWave; d *= 2) {
        const uint64_t o = __shfl_up(inc, d, kWave);
        if (lane >= d) inc += o;
    }
    if (lane == kWave - 1) buf[w] = inc;
    __syncthreads();
    uint64_t before = 0, all = 0;
    for (int x = 0; x < NT / kWave; ++x) {
        if (x < w) before += buf[x];
        all += buf[x];
    }
    *total = all;
    __syncthreads(); // buf is free for the next call
    return before + inc - v;
}

template <typename T, int NT>
__global__ void __launch_bounds__(NT)
    sampleFinish(SmpArgs a) {
    __shared__ uint64_t item[kTieCap];
    __shared__ uint64_t cum[kMaxK];
    __shared__ uint64_t sbuf[NT];
    __shared__ uint64_t sel[kMaxK]; // the bucket members taken, as sort items
    __shared__ int kept, pick;
    const int row = int(blockIdx.x);
    const int t = int(threadIdx.x);
    SmpRow &st = a.st[row];
    const uint32_t prefix = st.theta, need = st.need, nB = st.nTie;
    const uint32_t nGt = min(st.nGt, uint32_t(kMaxK));
    const int k = a.k; // == nGt + need
    // 1. the `need` best bucket members (prefix P) by (key desc, index asc)
    if (nB <= uint32_t(kTieCap)) {
        int n2 = 2;
        while (n2 < int(nB)) n2 *= 2;
        for (int i = t; i < n2; i += NT) item[i] = i < int(nB) ? a.ties[size_t(row) * kTieCap + i] : ~0ull;
        __syncthreads();
        bitonic(item, n2);
        for (int i = t; i < int(need); i += NT) sel[i] = item[i];
    } else {
        // more bucket members than the list holds: the last 10 bits of the k-th largest key
        // from a histogram of the bucket over a scan of the row, then the members above that
        // key (any order) and the smallest indices of its ties (contiguous segments)
        __shared__ uint32_t h3[1024];
        __shared__ BinScratch bs;
        __shared__ uint32_t nAbove;
        for (int b = t; b < 1024; b += NT) h3[b] = 0;
        if (t == 0) nAbove = 0;
        __syncthreads();
        const int seg = (a.V + NT - 1) / NT, lo = t * seg, hi = min(a.V, lo + seg);
        for (int i = lo; i < hi; ++i) {
            const uint32_t key = keyAt<T>(a, row, i);
            if ((key >> 10) == prefix) atomicAdd(&h3[key & 0x3FFu], 1u);
        }
        __syncthreads();
        uint32_t need3 = 0;
        const uint32_t theta = (prefix << 10) | uint32_t(chooseBin<NT>(h3, 1024, need, &need3, bs));
        for (int i = lo; i < hi; ++i) {
            const uint32_t key = keyAt<T>(a, row, i);
            if ((key >> 10) == prefix && key > theta) sel[atomicAdd(&nAbove, 1u)] = (uint64_t(~key) << 32) | uint32_t(i);
        }
        uint32_t c = 0;
        for (int i = lo; i < hi; ++i) c += keyAt<T>(a, row, i) == theta;
        uint64_t tot;
        uint32_t r = uint32_t(blockExclusive<NT>(c, sbuf, &tot)); // (its barriers also order nAbove)
        const uint32_t above = need - need3;
        for (int i = lo; i < hi && r < need3; ++i)
            if (keyAt<T>(a, row, i) == theta) sel[above + r++] = (uint64_t(~theta) << 32) | uint32_t(i);
    }
    __syncthreads();
    // 2. the k candidates sorted by (key desc, index asc): ascending on (~key, index)
    int nk = 2;
    while (nk < k) nk *= 2;
    // the gather stored the candidates as sort items.  Loads unconditional (clamped), the padding selected after them: loads under per-lane
    // branches were issued one round trip at a time.
    uint64_t x4[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = min(4 * t + e, k - 1);
        const uint64_t g = a.gt[size_t(row) * kMaxK + min(j, kMaxK - 1)];
        const uint64_t b = sel[max(j - int(nGt), 0)];
        x4[e] = 4 * t + e < k ? (j < int(nGt) ? g : b) : ~0ull;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) item[4 * t + e] = x4[e];
    __syncthreads();
    bitonic(item, nk);
    // 3. integer weights and their running sums (thread t owns elements [4t, 4t + 4))
    const float zmax = unkey(~uint32_t(item[0] >> 32));
    uint64_t w4[4], run = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int j = 4 * t + e;
        w4[e] = 0;
        if (j < k) {
            const float z = unkey(~uint32_t(item[j] >> 32));
            // a candidate tied with the top key weighs 2^0 also when both are infinite
            const bool top = uint32_t(item[j] >> 32) == uint32_t(item[0] >> 32);
            const float p = sampleExp2(top ? 0.0f : __fmul_rn(__fsub_rn(z, zmax), 1.4426950408889634f));
            w4[e] = uint32_t(__fmul_rn(p, 2147483648.0f));
        }
        run += w4[e];
    }
    uint64_t tot;
    uint64_t pre = blockExclusive<NT>(run, sbuf, &tot);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        pre += w4[e];
        if (4 * t + e < kMaxK) cum[4 * t + e] = pre;
    }
    __syncthreads();
    // 4. the top-p cut and the draw
    const uint64_t W = cum[k - 1];
    uint64_t target = 0; // 0: no top-p cut
    if (a.topP < 1.0f) {
        target = 1;
        if (a.topP > 0.0f) {
            target = uint64_t(double(a.topP) * double(W));
            if (target == 0) target = 1;
        }
    }
    if (t == 0) {
        kept = k;
        pick = 0; // overwritten below: r < the kept weight sum, so the crossing exists
    }
    __syncthreads();
    if (target)
        for (int j = t; j < k; j += NT)
            if (cum[j] >= target && (j == 0 || cum[j - 1] < target)) kept = j + 1;
    __syncthreads();
    const uint64_t wk = cum[kept - 1];
    const uint64_t u24 = splitmix64(a.seed + uint64_t(row)) >> 40;
    const uint64_t rr = (__umul64hi(u24, wk) << 40) | ((u24 * wk) >> 24);
    for (int j = t; j < kept; j += NT)
        if (cum[j] > rr && (j == 0 || cum[j - 1] <= rr)) pick = j;
    __syncthreads();
    if (t == 0) {
        const int64_t idx = int64_t(uint32_t(item[pick]));
        if (a.i64)
            static_cast<int64_t *>(a.out)[row] = idx;
        else
            static_cast<int32_t *>(a.out)[row] = int32_t(idx);
    }
    // 5. leave the row's state zero for the next launch
    for (int b = t; b < 2048; b += NT) {
        st.h1[b] = 0;
        st.h2[b] = 0;
    }
    if (t == 0) st.nGt = st.nTie = st.theta = st.need = 0;
}

} // namespace

} // namespace llaisys::kernels

namespace llaisys::kernels {

// greedy: the flat argmax's partials (after kScratchReserved), then one value per row
size_t greedyValueOffset(size_t V, llaisysDataType_t dt) {
    return (argmaxWorkspaceBytes(V, dt) + 15) / 16 * 16;
}

size_t randomSampleWorkspaceBytes(size_t rows, size_t V, llaisysDataType_t dt) {
    // sampling: candidate and tie lists of up to kSampleRows rows
    const size_t lists = kSampleRows * (size_t(kMaxK) + size_t(kTieCap)) * sizeof(uint64_t);
    const size_t greedy = greedyValueOffset(V, dt) - kScratchReserved + rows * sizeof(float);
    return std::max(lists, greedy);
}

void randomSample(void *out_idx, bool i64, const void *logits, size_t rows, size_t V,
                  llaisysDataType_t dt, float temperature, int64_t top_k, float top_p,
                  uint64_t seed, void *ws, hipStream_t s) {
    if (rows == 0 || V == 0) return;
    char *base = static_cast<char *>(ws);
    if (!(temperature > 0.0f) || top_k == 1) { // greedy: the row's argmax
        char *val = base + greedyValueOffset(V, dt); // the argmax kernels want a value output too
        if (rows == 1) // one row: the multi-block flat argmax (its workspace: base, counter at 0)
            argmax(out_idx, i64, val, logits, V, dt, base, s);
        else
            argmaxRows(out_idx, i64, val, logits, rows, V, dt, s);
        return;
    }
    const float inv = 1.0f / temperature;
    const int k = int(std::min<int64_t>(top_k, int64_t(V)));
    const size_t esz = dt == LLAISYS_DTYPE_F32 ? 4 : 2;
    for (size_t r0 = 0; r0 < rows; r0 += kSampleRows) {
        const size_t nr = std::min(kSampleRows, rows - r0);
        SmpArgs a;
        a.x = static_cast<const char *>(logits) + r0 * V * esz;
        a.out = static_cast<char *>(out_idx) + r0 * (i64 ? 8 : 4);
        a.i64 = i64;
        a.V = int(V);
        a.k = k;
        a.rows = int(nr);
        a.inv = inv;
        a.topP = top_p;
        a.seed = seed + r0;
        a.st = reinterpret_cast<SmpRow *>(base + kSampleStateOffset);
        a.gt = reinterpret_cast<uint64_t *>(base + kScratchReserved);
        a.ties = a.gt + kSampleRows * kMaxK;
        const dim3 grid(unsigned((V + kSmpChunk - 1) / kSmpChunk), unsigned(nr));
        switch (dt) {
        case LLAISYS_DTYPE_F32:
            sampleHist<F32, 1><<<grid, kSmpBlock, 0, s>>>(a);
            sampleHist<F32, 2><<<grid, kSmpBlock, 0, s>>>(a);
            sampleGather<F32><<<grid, kSmpBlock, 0, s>>>(a);
            if (k > 256)
                sampleFinish<F32, kFinThreadsWide><<<unsigned(nr), kFinThreadsWide, 0, s>>>(a);
            else
                sampleFinish<F32, kFinThreads><<<unsigned(nr), kFinThreads, 0, s>>>(a);
            break;
        case LLAISYS_DTYPE_BF16:
            sampleHist<BF16, 1><<<grid, kSmpBlock, 0, s>>>(a);
            sampleHist<BF16, 2><<<grid, kSmpBlock, 0, s>>>(a);
            sampleGather<BF16><<<grid, kSmpBlock, 0, s>>>(a);
            if (k > 256)
                sampleFinish<BF16, kFinThreadsWide><<<unsigned(nr), kFinThreadsWide, 0, s>>>(a);
            else
                sampleFinish<BF16, kFinThreads><<<unsigned(nr), kFinThreads, 0, s>>>(a);
            break;
        case LLAISYS_DTYPE_F16:
            sampleHist<F16, 1><<<grid, kSmpBlock, 0, s>>>(a);
            sampleHist<F16, 2><<<grid, kSmpBlock, 0, s>>>(a);
            sampleGather<F16><<<grid, kSmpBlock, 0, s>>>(a);
            if (k > 256)
                sampleFinish<F16, kFinThreadsWide><<<unsigned(nr), kFinThreadsWide, 0, s>>>(a);
            else
                sampleFinish<F16, kFinThreads><<<unsigned(nr), kFinThreads, 0, s>>>(a);
            break;
        default: return;
        }
    }
}

} // namespace llaisys::kernels
