// Causal GQA self-attention for gfx950, over a cache in the element type or in INT8.
//
// Semantics: reference src/ops/self_attention/cpu/self_attention_cpu.cpp:13-115.  q [seq,
// nh, d], k [total, nkvh, d], v [total, nkvh, dv], out [seq, nh, dv]; q head h reads kv
// head h / (nh / nkvh); query i sits at current_pos = total - seq + i in size_t arithmetic
// (so seq > total wraps and the early queries see every key) and sees keys t <=
// current_pos; scores are (q . k) * scale in f32, softmax in f32, out = sum_t p_t v_t
// rounded to the element type; total == 0 gives zeros.  The INT8 form reads k and v as
// codes [total, nkvh, d] I8 plus scales [total, nkvh] F32 and rounds code * scale to the
// element type first, i.e. it is attention over llaisysDequantizeInt8 of the caches.
//
// Arithmetic differs from the reference in order only: fused multiply-adds in a lane tree
// for q . k, an online softmax (running max, rescaled sum and output) over batches of keys,
// exp through the hardware exp2, and (sum p v) / (sum p) instead of sum (p / sum) v.  The
// tests bound the difference by the f32 accumulation error of the reference itself.
//
// Design, three kernels (the launcher at the end picks one):
//  - attnMfmaLds / attnMfma (bf16, head_dim 128, >= 16 queries: prefill): MFMA-bound; 16
//    queries x one kv head's q heads per block, S^T = K Q^T and O^T += V^T P^T on
//    v_mfma_f32_16x16x32_bf16 with K / V tiles in LDS one tile ahead; with few blocks per CU,
//    two wave sets per block split the key tiles (kSplit).  attnMfmaLds moves bf16 tiles
//    HBM -> LDS directly; an INT8 cache whose bf16 form fits the workspace is dequantized
//    once into it and attended by it as bf16 (the same operands), and attnMfma stages other
//    INT8 caches through registers, converting the codes on the way.
//  - attnDecodeMfma (bf16 q, head_dim 128, fewer queries: decode, cache in bf16 or INT8):
//    HBM-bound; the key range is cut into chunks, one block per (query, kv head, chunk) with
//    the kv head's q heads as the MFMA columns; attnCombine merges the chunk partials.
//  - attnGroup (other dtypes, head_dim 64): one wavefront per q head, the waves of a block
//    being q heads of one kv head (they read the same K / V rows).  A key row of D elements
//    is spread over R = D / 8 lanes, 8 elements per lane, so one load instruction covers
//    64 / R keys; per batch of U instructions the wave forms its scores (8 FMAs, a butterfly
//    over R lanes), updates the running max once and folds p * v into per-lane
//    accumulators.  Long key ranges with few (query, head) pairs are split and merged by
//    attnCombine as well.
//  - attnScalar: any other head_dim / v_head_dim, one wave per (query, head).
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

#include <algorithm>
#include <cstdio>
#include <mutex>
#include <cmath>
#include <type_traits>

namespace llaisys::kernels {

namespace {


// Row reader: 8 consecutive elements of a K or V row as f32.
template <typename T, bool kInt8>
struct RowIO;

template <typename T>
struct RowIO<T, false> {
    static constexpr int kRegs = Fmt<T>::kBytes == 2 ? 1 : 2; // 16-byte loads per lane
    struct Raw {
        v4u r[kRegs];
    };
    __device__ static Raw load(const void *base, size_t row, int d, int col) {
        const char *p = static_cast<const char *>(base) + (row * size_t(d) + col) * Fmt<T>::kBytes;
        Raw x;
#pragma unroll
        for (int k = 0; k < kRegs; ++k) x.r[k] = *reinterpret_cast<const v4u *>(p + 16 * k);
        return x;
    }
    __device__ static void unpack(const Raw &x, float sc, float *f) {
        (void)sc;
        if constexpr (kRegs == 1) {
            Fmt<T>::unpack(x.r[0], f);
        } else {
            Fmt<T>::unpack(x.r[0], f);
            Fmt<T>::unpack(x.r[1], f + 4);
        }
    }
};

template <typename T>
struct RowIO<T, true> {
    typedef uint32_t v2u __attribute__((ext_vector_type(2)));
    struct Raw {
        v2u r;
    };
    __device__ static Raw load(const void *base, size_t row, int d, int col) {
        const int8_t *p = static_cast<const int8_t *>(base) + row * size_t(d) + col;
        return Raw{*reinterpret_cast<const v2u *>(p)};
    }
    // code * scale rounded to the element type, as llaisysDequantizeInt8 stores it
    __device__ static void unpack(const Raw &x, float sc, float *f) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            f[e] = Fmt<T>::round(float(int8_t(x.r.x >> (8 * e))) * sc);
            f[4 + e] = Fmt<T>::round(float(int8_t(x.r.y >> (8 * e))) * sc);
        }
    }
};

struct AttnArgs {
    void *out;
    const void *q;
    const void *k;  // elements, or codes
    const void *v;
    const float *ks; // scales (INT8 only)
    const float *vs;
    float *part;     // partials of a split launch: [(i * nh + h) * nchunks + c][D + 2]
    size_t seq, total;
    int nh, nkvh, group, slices, nchunks, chunk;
    float scale;
};

// Visible keys of query i: [0, vis).
__device__ __forceinline__ size_t visibleKeys(size_t total, size_t seq, size_t i) {
    const size_t cur = total - seq + i; // size_t arithmetic, as the reference
    return cur >= total ? total : cur + 1;
}

constexpr int kWaves = 8; // waves per block of the vector kernel

// One block per (query, kv head, slice of G q heads, key chunk); its kWaves waves take the
// chunk's key tiles (KPW * U keys) in turn, every wave holding the G heads' q, running max,
// sum and output columns in registers, so each K / V row is loaded once per block.  The
// waves' states merge through LDS; the block then writes the output (one chunk) or the
// chunk's partial (split launch).
template <typename T, bool kInt8, int D, int G, int U>
__global__ void __launch_bounds__(kWave * kWaves)
    attnGroup(AttnArgs a) {
    using IO = RowIO<T, kInt8>;
    constexpr int R = D / 8;       // lanes per key row
    constexpr int KPW = kWave / R; // keys per load instruction
    constexpr int TILE = KPW * U;  // keys per wave per step
    __shared__ float st[kWaves][G][D + 2];

    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const int rs = lane / R, col = (lane % R) * 8;

    // block -> (query, kv head, head slice, chunk); the latest queries (most keys) first
    unsigned b = blockIdx.x;
    const int c = int(b % unsigned(a.nchunks));
    b /= unsigned(a.nchunks);
    const int sl = int(b % unsigned(a.slices));
    b /= unsigned(a.slices);
    const int g = int(b % unsigned(a.nkvh));
    const size_t i = a.seq - 1 - size_t(b / unsigned(a.nkvh));
    const int h0 = g * a.group + sl * G; // first q head of the slice

    const size_t vis = visibleKeys(a.total, a.seq, i);
    const size_t k0 = size_t(c) * size_t(a.chunk);
    const size_t k1 = min(vis, k0 + size_t(a.chunk));

    float qv[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const char *qp = static_cast<const char *>(a.q) + ((i * a.nh + h0 + j) * D + col) * Fmt<T>::kBytes;
        typename RowIO<T, false>::Raw r;
#pragma unroll
        for (int k = 0; k < RowIO<T, false>::kRegs; ++k) r.r[k] = *reinterpret_cast<const v4u *>(qp + 16 * k);
        RowIO<T, false>::unpack(r, 0.0f, qv[j]);
    }
    float m[G], l[G], o[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        m[j] = -INFINITY;
        l[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[j][e] = 0.0f;
    }

    for (size_t kb = k0 + size_t(wave) * TILE; kb < k1; kb += size_t(kWaves) * TILE) {
        typename IO::Raw kr[U], vr[U];
        float ksc[U], vsc[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t key = kb + size_t(u * KPW + rs);
            ok[u] = key < k1;
            const size_t row = (ok[u] ? key : k0) * size_t(a.nkvh) + size_t(g);
            kr[u] = IO::load(a.k, row, D, col);
            vr[u] = IO::load(a.v, row, D, col);
            if constexpr (kInt8) {
                ksc[u] = a.ks[row];
                vsc[u] = a.vs[row];
            } else {
                ksc[u] = vsc[u] = 0.0f;
            }
        }
        float s[G][U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float kf[8];
            IO::unpack(kr[u], ksc[u], kf);
#pragma unroll
            for (int j = 0; j < G; ++j) {
                float dot = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) dot = __builtin_fmaf(qv[j][e], kf[e], dot);
                dot = waveGroupReduce<R, SumOp>(dot);
                s[j][u] = ok[u] ? dot * a.scale : -INFINITY;
            }
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
            float mx = m[j];
#pragma unroll
            for (int u = 0; u < U; ++u) mx = fmaxf(mx, s[j][u]);
            // a -inf score is weight 0 (reference :111-113); m == mx keeps the state as is
            const float corr = mx == m[j] ? 1.0f : __expf(m[j] - mx);
            l[j] *= corr;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[j][e] *= corr;
            m[j] = mx;
#pragma unroll
            for (int u = 0; u < U; ++u) s[j][u] = s[j][u] == -INFINITY ? 0.0f : __expf(s[j][u] - mx);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float vf[8];
            IO::unpack(vr[u], vsc[u], vf);
#pragma unroll
            for (int j = 0; j < G; ++j) {
                l[j] += s[j][u];
#pragma unroll
                for (int e = 0; e < 8; ++e) o[j][e] = __builtin_fmaf(s[j][u], vf[e], o[j][e]);
            }
        }
    }

    // merge the KPW key slots of the wave (lanes R, 2R, ... apart hold the same columns)
#pragma unroll
    for (int off = R; off < kWave; off *= 2) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const float mo = __shfl_xor(m[j], off, kWave), lo = __shfl_xor(l[j], off, kWave);
            const float M = fmaxf(m[j], mo);
            // a slot that saw no key has m = -inf, l = 0, o = 0; its factor is 1 only when M
            // is -inf too, and then every term is 0
            const float fa = m[j] == M ? 1.0f : __expf(m[j] - M);
            const float fb = mo == M ? 1.0f : __expf(mo - M);
            l[j] = l[j] * fa + lo * fb;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float oo = __shfl_xor(o[j][e], off, kWave);
                o[j][e] = o[j][e] * fa + oo * fb;
            }
            m[j] = M;
        }
    }
    if (lane < R) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
#pragma unroll
            for (int e = 0; e < 8; ++e) st[wave][j][col + e] = o[j][e];
            if (lane == 0) {
                st[wave][j][D] = m[j];
                st[wave][j][D + 1] = l[j];
            }
        }
    }
    __syncthreads();
    // merge the waves: thread t -> (head j, column e) pairs
    for (int p = threadIdx.x; p < G * D; p += kWave * kWaves) {
        const int j = p / D, e = p % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, st[w][j][D]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = st[w][j][D];
            const float f = mw == M ? 1.0f : __expf(mw - M); // 1 for M = -inf, where l = o = 0
            L += st[w][j][D + 1] * f;
            O += st[w][j][e] * f;
        }
        const size_t ih = i * a.nh + size_t(h0 + j);
        if (a.nchunks == 1) {
            // put: the reference rounding, also for a NaN carrying the caller's scale payload
            Fmt<T>::put(a.out, ih * D + e, L > 0.0f ? O / L : 0.0f);
        } else {
            float *pp = a.part + (ih * size_t(a.nchunks) + c) * (D + 2);
            pp[e] = O;
            if (e == 0) {
                pp[D] = M;
                pp[D + 1] = L;
            }
        }
    }
}

// Merge of the chunk partials of a split launch: one 1024-thread block per (query, head,
// slab of 32 output columns); thread t takes column t % 32 of the slab for the chunks c =
// t / 32 (mod 32), so a thread reads at most nchunks / 32 partial values and the (query,
// head) pairs of a decode launch spread over D / 32 times as many blocks.  Every block of a
// pair forms the same maximum and sum from the chunks' (m, l).  Up to 256 chunks (kPer = 8
// per thread) the partial values are requested together with the (m, l) loads, so the
// merge waits for one round of loads rather than two; the sum runs in the same order
// either way.
constexpr int kCombineThreads = 1024;
constexpr int kCombineCols = 32; // output columns per block (head_dim is 64 or 128)

template <typename T, int kPer>
__global__ void __launch_bounds__(kCombineThreads)
    attnCombine(void *out, const float *part, int nchunks, int D) {
    __shared__ float w[1024];  // per-chunk factor exp(m_c - M), nchunks <= 1024
    __shared__ float red[kCombineThreads];
    __shared__ float wred[kCombineThreads / kWave];
    constexpr int kGroups = kCombineThreads / kCombineCols;
    const int slabs = D / kCombineCols;
    const size_t ih = blockIdx.x / unsigned(slabs); // i * nh + h
    const int col0 = int(blockIdx.x % unsigned(slabs)) * kCombineCols;
    const float *pp = part + ih * size_t(nchunks) * (D + 2);
    const int t = threadIdx.x;
    const int e = col0 + t % kCombineCols, grp = t / kCombineCols;
    const float mc = t < nchunks ? pp[size_t(t) * (D + 2) + D] : -INFINITY;
    const float lc = t < nchunks ? pp[size_t(t) * (D + 2) + D + 1] : 0.0f;
    float v[kPer > 0 ? kPer : 1];
#pragma unroll
    for (int j = 0; j < kPer; ++j) { // unconditional (clamped) loads, used only for k < nchunks
        const int k = grp + j * kGroups;
        v[j] = pp[size_t(k < nchunks ? k : 0) * (D + 2) + e];
    }
    const float M = groupReduce<kCombineThreads, MaxOp>(mc, wred); // every thread gets it
    const float f = mc == M ? 1.0f : __expf(mc - M);                // mc = -inf: l = o = 0
    if (t < nchunks) w[t] = f;
    const float L = groupReduce<kCombineThreads, SumOp>(t < nchunks ? lc * f : 0.0f, wred);
    __syncthreads();
    float acc = 0.0f;
    if constexpr (kPer > 0) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int k = grp + j * kGroups;
            if (k < nchunks) acc += v[j] * w[k];
        }
    } else {
#pragma unroll 8
        for (int k = grp; k < nchunks; k += kGroups) acc += pp[size_t(k) * (D + 2) + e] * w[k];
    }
    red[t] = acc;
    __syncthreads();
    if (t < kCombineCols) {
        float O = 0.0f;
        for (int g = 0; g < kGroups; ++g) O += red[g * kCombineCols + t];
        Fmt<T>::put(out, ih * D + col0 + t, L > 0.0f ? O / L : 0.0f);
    }
}

template <typename T>
void launchCombine(void *out, const float *part, int nchunks, int D, size_t pairs, hipStream_t s) {
    const unsigned blocks = unsigned(pairs) * unsigned(D / kCombineCols);
    if (nchunks <= 8 * (kCombineThreads / kCombineCols))
        attnCombine<T, 8><<<blocks, kCombineThreads, 0, s>>>(out, part, nchunks, D);
    else
        attnCombine<T, 0><<<blocks, kCombineThreads, 0, s>>>(out, part, nchunks, D);
}

// Any head_dim / v_head_dim / group: one wave per (query, head), keys one at a time with an
// online softmax; the output accumulates in LDS (dv floats per wave, lane j owns the
// columns j, j + 64, ...).  For the shapes the vector kernel does not take.
template <typename T, bool kInt8>
__global__ void __launch_bounds__(kWave)
    attnScalar(AttnArgs a, int d, int dv) {
    extern __shared__ float acc[]; // dv
    const size_t ih = blockIdx.x;
    const size_t i = ih / size_t(a.nh);
    const int h = int(ih % size_t(a.nh));
    const int g = h / a.group;
    const int lane = threadIdx.x;
    const size_t vis = visibleKeys(a.total, a.seq, i);
    const auto kval = [&](size_t t, int e) {
        const size_t row = t * size_t(a.nkvh) + size_t(g);
        if constexpr (kInt8)
            return Fmt<T>::round(float(static_cast<const int8_t *>(a.k)[row * d + e]) * a.ks[row]);
        else
            return Fmt<T>::get(a.k, row * d + e);
    };
    const auto vval = [&](size_t t, int e) {
        const size_t row = t * size_t(a.nkvh) + size_t(g);
        if constexpr (kInt8)
            return Fmt<T>::round(float(static_cast<const int8_t *>(a.v)[row * dv + e]) * a.vs[row]);
        else
            return Fmt<T>::get(a.v, row * dv + e);
    };
    for (int e = lane; e < dv; e += kWave) acc[e] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    for (size_t t = 0; t < vis; ++t) {
        float dot = 0.0f;
        for (int e = lane; e < d; e += kWave) dot = __builtin_fmaf(Fmt<T>::get(a.q, (i * a.nh + h) * d + e), kval(t, e), dot);
        dot = waveGroupReduce<kWave, SumOp>(dot);
        const float s = dot * a.scale;
        if (s == -INFINITY) continue; // weight 0
        const float mx = fmaxf(m, s);
        const float corr = mx == m ? 1.0f : __expf(m - mx);
        const float p = __expf(s - mx);
        l = l * corr + p;
        for (int e = lane; e < dv; e += kWave) acc[e] = acc[e] * corr + p * vval(t, e);
        m = mx;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    for (int e = lane; e < dv; e += kWave) Fmt<T>::put(a.out, ih * dv + e, acc[e] * inv);
}

// 8 consecutive elements of a cache row (128 per row) as raw bits: bf16 (16 bytes) or INT8
// codes (8 bytes, in .x / .y).
template <bool kInt8>
__device__ __forceinline__ v4u loadRow8(const void *base, size_t row, int col) {
    if constexpr (kInt8) {
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        const v2u c = *reinterpret_cast<const v2u *>(static_cast<const int8_t *>(base) + row * 128 + col);
        return v4u{c.x, c.y, 0u, 0u};
    } else {
        return *reinterpret_cast<const v4u *>(static_cast<const uint16_t *>(base) + row * 128 + col);
    }
}

// 8 INT8 codes -> bf16(code * sc) as 4 packed words.  code = u - 128 for the unsigned byte
// u of code ^ 0x80, and fma(u, sc, -128 sc) rounds u * sc - 128 sc = code * sc once (-128 sc
// is exact), i.e. exactly float(code) * sc; the pair conversion then rounds to bf16 as the
// reference does for every non-NaN value.
__device__ __forceinline__ v4u codesToBf16(const v4u &raw, float sc) {
    const uint32_t ux = raw.x ^ 0x80808080u, uy = raw.y ^ 0x80808080u;
    const float off = -128.0f * sc;
    const auto cv = [&](uint32_t u, int k) {
        const float b = float((u >> (8 * k)) & 0xFFu); // v_cvt_f32_ubyte{k}
        return __builtin_fmaf(b, sc, off);
    };
    return v4u{Bf16Cvt::narrow2Q(cv(ux, 0), cv(ux, 1)), Bf16Cvt::narrow2Q(cv(ux, 2), cv(ux, 3)),
               Bf16Cvt::narrow2Q(cv(uy, 0), cv(uy, 1)), Bf16Cvt::narrow2Q(cv(uy, 2), cv(uy, 3))};
}

// ---- prefill on MFMA (bf16 q / out, head_dim 128, cache in bf16 or INT8) --------------
// One block per (16 queries, kv head, slice of W q heads), one wave per q head.  Per tile
// of 64 keys a wave forms S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (A = 16 key rows of
// the tile, B = the wave's 16 queries kept in registers), so each lane holds the scores of
// one query (column l % 16) for 16 of the keys and the softmax needs only an exchange
// between the 4 lanes of that column; then O^T += V^T P^T with the same instruction.
// Operand layouts (measured on MI355X): A[m = l % 16][k = 8(l / 16) + j],
// B[k = 8(l / 16) + j][n = l % 16], D[m = 4(l / 16) + i][n = l % 16].
// Key order: row m of score tile t (of 4) is key 32(t / 2) + 8(m / 4) + 4(t % 2) + m % 4,
// so lane group g holds keys 32p + 8g .. + 7 of tiles 2p and 2p + 1 -- exactly the 8
// consecutive k-slots 8g + j of the P V product for keys 32p .. 32p + 31, and the V^T
// operand of those slots is one 16-byte LDS read.  P enters as bf16 hi + lo parts (2^-17
// relative), so the output keeps f32 accuracy.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfmaQ = 16;  // queries per block
constexpr int kMfmaKT = 64; // keys per tile
constexpr int kKtLd = 136;  // K tile row stride (bf16): 16-byte rows, rows 4 banks apart
constexpr int kVtLd = 72;   // V^T row stride (bf16): 16-byte reads; rows 8 apart 32 banks apart

__device__ __forceinline__ bf16x8 asBf16x8(const v4u &r) { return __builtin_bit_cast(bf16x8, r); }

// Tiles move HBM -> registers -> LDS with one tile of lookahead: while the waves compute on
// tile t (in LDS buffer t % 2), every thread holds its share of tile t + 1 in registers and
// writes it to the other buffer at the start of the next step, so the loads overlap the
// MFMA work and a step needs one barrier.  K is stored as loaded (row-major); V is stored
// transposed from pairs of consecutive keys, one 4-byte write per column and pair (the 32
// lanes of a pair of rows write 32 consecutive words, the other 32 lanes rows 32 banks on).
// kSplit: the block holds two waves per q head, and the key tiles are cut in two halves that
// the two wave sets walk in lockstep (one barrier per step for both), each staging its own
// tiles; at the end the second half's (max, sum, output) is merged into the first's through
// LDS.  It halves the longest block's chain of tiles -- the causal imbalance that bounds
// a prefill with about one block per CU.
template <int W, bool kSplit, bool kInt8>
__global__ void __launch_bounds__(kWave * W * (kSplit ? 2 : 1))
    attnMfma(AttnArgs a) {
    constexpr int D = 128, KB = D / 32, DT = D / 16;
    constexpr int NHALF = kSplit ? 2 : 1;
    constexpr int kKItems = kMfmaKT * (D / 8);           // 16-byte K pieces per tile
    constexpr int kVItems = (kMfmaKT / 2) * (D / 8);     // V pieces: 2 keys x 8 columns
    constexpr int kKPer = (kKItems + kWave * W - 1) / (kWave * W);
    constexpr int kVPer = (kVItems + kWave * W - 1) / (kWave * W);
    __shared__ uint16_t kt_all[NHALF][2][kMfmaKT][kKtLd];
    __shared__ uint16_t vt_all[NHALF][2][D][kVtLd];
    const int wave_all = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int half = kSplit ? wave_all / W : 0;   // key half this wave walks
    const int wave = wave_all % W;                 // q head of the slice
    const int ltid = int(threadIdx.x) % (kWave * W); // thread index within the half
    auto &kt = kt_all[half];
    auto &vt = vt_all[half];
    const int lane = int(threadIdx.x) % kWave;
    const int n = lane % 16, g4 = lane / 16;

    const size_t nqb = (a.seq + kMfmaQ - 1) / kMfmaQ;
    unsigned b = blockIdx.x;
    const int sl = int(b % unsigned(a.slices));
    b /= unsigned(a.slices);
    const int g = int(b % unsigned(a.nkvh));
    const size_t qb = nqb - 1 - size_t(b / unsigned(a.nkvh)); // latest queries first
    const int h = g * a.group + sl * W + wave;
    const size_t q0 = qb * kMfmaQ;
    const size_t qi = min(q0 + size_t(n), a.seq - 1); // this lane's query (clamped for loads)
    const size_t vis_q = visibleKeys(a.total, a.seq, qi);
    const size_t vis_blk = visibleKeys(a.total, a.seq, min(q0 + kMfmaQ - 1, a.seq - 1));
    const size_t vis_first = visibleKeys(a.total, a.seq, q0); // the fewest keys any query sees
    const size_t ntiles = (vis_blk + kMfmaKT - 1) / kMfmaKT;
    const float c2 = a.scale * 1.4426950408889634f; // scores to base-2 exponents

    bf16x8 qreg[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        const uint16_t *qp = static_cast<const uint16_t *>(a.q) + (qi * a.nh + h) * D + 32 * kb + 8 * g4;
        qreg[kb] = asBf16x8(*reinterpret_cast<const v4u *>(qp));
    }
    float m = -INFINITY, lsum = 0.0f; // m: running max of the raw dots (scaled by c2 in use)
    f32x4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // cache rows of the kv head: row t at element (t * nkvh + g) * D; INT8 codes with one
    // scale per (t, g), turned into bf16(code * scale) (codesToBf16) when staged into LDS
    const size_t rstride = size_t(a.nkvh);
    v4u kraw[kKPer], vraw[kVPer][2];
    float ksc[kInt8 ? kKPer : 1], vsc[kInt8 ? kVPer : 1][2];
    const auto loadTile = [&](size_t t0) {
        const size_t left = a.total - t0; // keys of the cache from t0 on (> 0)
#pragma unroll
        for (int r = 0; r < kKPer; ++r) {
            const int idx = ltid + r * kWave * W;
            const int kk = idx / (D / 8), col = 8 * (idx % (D / 8));
            kraw[r] = v4u{0u, 0u, 0u, 0u}; // keys past the cache: zeros
            if constexpr (kInt8) ksc[r] = 0.0f;
            if (idx < kKItems && size_t(kk) < left) {
                kraw[r] = loadRow8<kInt8>(a.k, (t0 + kk) * rstride + g, col);
                if constexpr (kInt8) ksc[r] = a.ks[(t0 + kk) * rstride + g];
            }
        }
#pragma unroll
        for (int r = 0; r < kVPer; ++r) {
            const int idx = ltid + r * kWave * W;
            const int kp = idx % (kMfmaKT / 2), col = 8 * (idx / (kMfmaKT / 2));
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                vraw[r][e] = v4u{0u, 0u, 0u, 0u};
                if constexpr (kInt8) vsc[r][e] = 0.0f;
                if (idx < kVItems && size_t(2 * kp + e) < left) {
                    vraw[r][e] = loadRow8<kInt8>(a.v, (t0 + 2 * kp + e) * rstride + g, col);
                    if constexpr (kInt8) vsc[r][e] = a.vs[(t0 + 2 * kp + e) * rstride + g];
                }
            }
        }
    };
    const auto storeTile = [&](int buf) {
        if constexpr (kInt8) {
#pragma unroll
            for (int r = 0; r < kKPer; ++r) kraw[r] = codesToBf16(kraw[r], ksc[r]);
#pragma unroll
            for (int r = 0; r < kVPer; ++r)
#pragma unroll
                for (int e = 0; e < 2; ++e) vraw[r][e] = codesToBf16(vraw[r][e], vsc[r][e]);
        }
#pragma unroll
        for (int r = 0; r < kKPer; ++r) {
            const int idx = ltid + r * kWave * W;
            if (idx < kKItems)
                *reinterpret_cast<v4u *>(&kt[buf][idx / (D / 8)][8 * (idx % (D / 8))]) = kraw[r];
        }
#pragma unroll
        for (int r = 0; r < kVPer; ++r) {
            const int idx = ltid + r * kWave * W;
            if (idx >= kVItems) continue;
            const int kp = idx % (kMfmaKT / 2), col = 8 * (idx / (kMfmaKT / 2));
            const uint32_t w0[4] = {vraw[r][0].x, vraw[r][0].y, vraw[r][0].z, vraw[r][0].w};
            const uint32_t w1[4] = {vraw[r][1].x, vraw[r][1].y, vraw[r][1].z, vraw[r][1].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // columns col + 2e (low halves) and col + 2e + 1 (high halves) of keys 2kp, 2kp + 1
                *reinterpret_cast<uint32_t *>(&vt[buf][col + 2 * e][2 * kp]) =
                    __builtin_amdgcn_perm(w1[e], w0[e], 0x05040100u);
                *reinterpret_cast<uint32_t *>(&vt[buf][col + 2 * e + 1][2 * kp]) =
                    __builtin_amdgcn_perm(w1[e], w0[e], 0x07060302u);
            }
        }
    };

    // this half's tiles: [tbeg, tbeg + tcount); both halves step nsteps times
    const size_t nsteps = kSplit ? (ntiles + 1) / 2 : ntiles;
    const size_t tbeg = half ? nsteps : 0;
    const size_t tcount = half ? ntiles - nsteps : nsteps;
    if (tcount > 0) loadTile(tbeg * kMfmaKT);
    for (size_t it = 0; it < nsteps; ++it) {
        const int buf = int(it & 1);
        const size_t ti = tbeg + it;
        const size_t kt0 = ti * kMfmaKT;
        storeTile(buf);
        if (it + 1 < tcount) loadTile(kt0 + kMfmaKT); // in flight during this step's math
        __syncthreads(); // tile ti in LDS; every wave is past the step that read buf last
        if (kSplit && it >= tcount) continue; // the shorter half idles through its last step
        // keys of this lane's query visible in the tile: offsets < nvis.  A tile every query
        // of the block sees whole (all but the causal diagonal) skips the masking.
        const bool whole = kt0 + kMfmaKT <= vis_first; // block-uniform
        const int nvis = int(min(vis_q - min(vis_q, kt0), size_t(kMfmaKT)));
        float p[4][4];
        float mx = m;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int krow = 32 * (t / 2) + 8 * (n / 4) + 4 * (t % 2) + n % 4; // A row n
            f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const v4u kv = *reinterpret_cast<const v4u *>(&kt[buf][krow][32 * kb + 8 * g4]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(kv), qreg[kb], acc, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) p[t][i] = acc[i];
        }
        if (!whole) { // the causal diagonal: keys past this lane's query are masked
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int off = 32 * (t / 2) + 8 * g4 + 4 * (t % 2) + i; // key of D row 4g + i
                    p[t][i] = off < nvis ? p[t][i] : -INFINITY;
                }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, p[t][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        // exp(scale * (s - max)) as 2^(s * c2 - max * c2); a masked key (-inf) gets weight 0.
        // Key 0 is visible to every query, so mx = -inf only when every score so far is -inf;
        // mc = 0 then keeps 2^(-inf - mc) at 0 instead of NaN, with no per-score select.
        const float mc = mx == -INFINITY ? 0.0f : mx * c2;
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[t][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(p[t][i], c2, -mc));
                ps += p[t][i];
            }
        if (__builtin_expect(__any(mx != m), 0)) { // rescale only when a max moved
            const float corr = mx == m ? 1.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(m, c2, -mc));
            lsum *= corr;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] *= corr;
        }
        m = mx;
        lsum += ps;
#pragma unroll
        for (int p2 = 0; p2 < 2; ++p2) {
            // P as bf16 hi + lo, two keys per conversion: key 32 p2 + 8g + j is p[2 p2 + j / 4][j % 4]
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float x0 = p[2 * p2 + w / 2][2 * (w % 2)], x1 = p[2 * p2 + w / 2][2 * (w % 2) + 1];
                hw[w] = Bf16Cvt::narrow2Q(x0, x1);
                lw[w] = Bf16Cvt::narrow2Q(x0 - __uint_as_float(hw[w] << 16), x1 - __uint_as_float(hw[w] & 0xFFFF0000u));
            }
            const bf16x8 bhi = asBf16x8(v4u{hw[0], hw[1], hw[2], hw[3]});
            const bf16x8 blo = asBf16x8(v4u{lw[0], lw[1], lw[2], lw[3]});
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const v4u vv = *reinterpret_cast<const v4u *>(&vt[buf][16 * dt + n][32 * p2 + 8 * g4]);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vv), bhi, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vv), blo, o[dt], 0, 0, 0);
            }
        }
    }
    float lt = lsum + __shfl_xor(lsum, 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
    if constexpr (kSplit) {
        // the second half hands (max, sum, output) to its partner wave through LDS (the
        // tiles' storage, free once every wave is past its last step)
        float *xch = reinterpret_cast<float *>(&kt_all[0][0][0][0]) + size_t(wave) * kWave * (2 + 4 * DT);
        __syncthreads();
        if (half == 1) {
            xch[lane] = m;
            xch[kWave + lane] = lt;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) xch[(2 + 4 * dt + i) * kWave + lane] = o[dt][i];
        }
        __syncthreads();
        if (half == 1) return;
        const float m1 = xch[lane], l1 = xch[kWave + lane];
        const float M = fmaxf(m, m1);
        // a half with no visible key has m = -inf: weight 0 (the other half holds key 0)
        const float f0 = m == M ? 1.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(m, c2, -M * c2));
        const float f1 = m1 == M ? 1.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(m1, c2, -M * c2));
        lt = lt * f0 + l1 * f1;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[dt][i] = o[dt][i] * f0 + xch[(2 + 4 * dt + i) * kWave + lane] * f1;
    }
    if (q0 + size_t(n) >= a.seq) return;
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    uint16_t *op = static_cast<uint16_t *>(a.out) + (qi * a.nh + h) * D + 4 * g4;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        // O^T[d = 16dt + 4g + i][query n]; the reference rounding
        const uint32_t w0 = f32ToBf16(o[dt][0] * inv) | (f32ToBf16(o[dt][1] * inv) << 16);
        const uint32_t w1 = f32ToBf16(o[dt][2] * inv) | (f32ToBf16(o[dt][3] * inv) << 16);
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        *reinterpret_cast<v2u *>(op + 16 * dt) = v2u{w0, w1};
    }
}

// ---- prefill on MFMA over a bf16 cache: tiles HBM -> LDS with no register staging -------
// The arithmetic of attnMfma (same operands, same MFMA order, same bits), with the K and V
// tiles moved by global_load_lds_dwordx4: one instruction fills 1 KB of LDS (4 key rows of
// 256 bytes) straight from memory, so a step spends no VALU on staging and holds no tile in
// registers.  V stays row-major in LDS and the Vᵀ operand of O^T += V^T P^T comes from two
// ds_read_b64_tr_b16: within each 16 lanes, lane j's element e is element j % 4 of the 8
// bytes lane 4e + j / 4 addresses (measured on MI355X), so lanes i reading 4 columns
// 4(i % 4) .. of key row 8g + i / 4 (then + 4) hand lane j of group g the 8 consecutive keys
// 8g .. 8g + 7 of column j.  Rows cannot be padded (the load fills LDS contiguously), so
// the 16-byte chunks of each row are XOR-swizzled by row bits: K by (r & 3) | (r >> 3 & 3) << 2,
// which spreads the 16 rows one ds_read_b128 of an A operand touches over all banks, V by
// 2 ((r & 3) | (r >> 3 & 1) << 2), which spreads the 8 rows of 32 lanes' transposing reads.
// Two LDS stages: the loads of tile t + 1 are issued after the barrier that ends every
// wave's reads of tile t - 1 and land while tile t is computed.  Keys past the cache load
// row 0 (finite wherever the reference's own output is; masked keys weigh 0).
typedef short v4s __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int swzK(int r) { return (r & 3) | (((r >> 3) & 3) << 2); }
__device__ __forceinline__ int swzV(int r) { return ((r & 3) | (((r >> 3) & 1) << 2)) << 1; }
__device__ __forceinline__ uint64_t ldsReadTr16(const char *p) {
    const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s *)(p));
    return __builtin_bit_cast(uint64_t, r);
}

template <int W, bool kSplit>
__global__ void __launch_bounds__(kWave * W * (kSplit ? 2 : 1))
    attnMfmaLds(AttnArgs a) {
    constexpr int D = 128, KB = D / 32, DT = D / 16;
    constexpr int NHALF = kSplit ? 2 : 1;
    constexpr int kRowB = 2 * D;              // bytes of a key row
    constexpr int kTileB = kMfmaKT * kRowB;   // one K or V tile
    constexpr int kLoads = 2 * kTileB / 1024; // 1 KB load instructions per stage
    constexpr int kPer = (kLoads + W - 1) / W;
    __shared__ __align__(16) char lds_all[NHALF][2][2 * kTileB]; // [half][stage][K tile | V tile]
    const int wave_all = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int half = kSplit ? wave_all / W : 0;
    const int wave = wave_all % W;
    const int lane = int(threadIdx.x) % kWave;
    const int n = lane % 16, g4 = lane / 16;

    const size_t nqb = (a.seq + kMfmaQ - 1) / kMfmaQ;
    unsigned b = blockIdx.x;
    const int sl = int(b % unsigned(a.slices));
    b /= unsigned(a.slices);
    const int g = int(b % unsigned(a.nkvh));
    const size_t qb = nqb - 1 - size_t(b / unsigned(a.nkvh)); // latest queries first
    const int h = g * a.group + sl * W + wave;
    const size_t q0 = qb * kMfmaQ;
    const size_t qi = min(q0 + size_t(n), a.seq - 1);
    const size_t vis_q = visibleKeys(a.total, a.seq, qi);
    const size_t vis_blk = visibleKeys(a.total, a.seq, min(q0 + kMfmaQ - 1, a.seq - 1));
    const size_t vis_first = visibleKeys(a.total, a.seq, q0);
    const size_t ntiles = (vis_blk + kMfmaKT - 1) / kMfmaKT;
    const float c2 = a.scale * 1.4426950408889634f;

    bf16x8 qreg[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        const uint16_t *qp = static_cast<const uint16_t *>(a.q) + (qi * a.nh + h) * D + 32 * kb + 8 * g4;
        qreg[kb] = asBf16x8(*reinterpret_cast<const v4u *>(qp));
    }
    float m = -INFINITY, lsum = 0.0f;
    f32x4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // load instruction j of this wave is stage load q = wave + W j (K rows for q < 16, then
    // V rows): rows 4 (q % 16) + lane / 16 of the tile, LDS slot lane % 16 receiving chunk
    // slot ^ swizzle(row) of the kv head's row
    const size_t rowB = size_t(a.nkvh) * kRowB; // bytes between consecutive keys
    const char *cache[2] = {static_cast<const char *>(a.k), static_cast<const char *>(a.v)};
    // (byte offsets within a tile fit 32 bits: the launcher checks 64 rows * rowB < 2^31)
    int lrow[kPer];
    uint32_t loff[kPer], lcol[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int q = wave + W * j;
        const int row = 4 * (q % 16) + lane / 16, slot = lane % 16;
        const int chunk = slot ^ (q < 16 ? swzK(row) : swzV(row));
        lrow[j] = row;
        lcol[j] = uint32_t(g * kRowB + chunk * 16);
        loff[j] = uint32_t(row) * uint32_t(rowB) + lcol[j];
    }
    const auto issue = [&](size_t t0, int stage) {
        char *dst = &lds_all[half][stage][0];
        const size_t left = a.total - t0; // keys of the cache from t0 on (> 0)
        const bool full = left >= size_t(kMfmaKT);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int q = wave + W * j;
            if (q >= kLoads) break;
            // the tile's rows from the tile base; in the cache's last tile, rows past it read row 0
            const char *src = full || size_t(lrow[j]) < left ? cache[q / 16] + t0 * rowB + loff[j]
                                                            : cache[q / 16] + lcol[j];
            __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1))) *)(src),
                                             (void __attribute__((address_space(3))) *)(dst + q * 1024), 16, 0, 0);
        }
    };

    const size_t nsteps = kSplit ? (ntiles + 1) / 2 : ntiles;
    const size_t tbeg = half ? nsteps : 0;
    const size_t tcount = half ? ntiles - nsteps : nsteps;
    if (tcount > 0) issue(tbeg * kMfmaKT, 0);
    for (size_t it = 0; it < nsteps; ++it) {
        const int buf = int(it & 1);
        const size_t kt0 = (tbeg + it) * kMfmaKT;
        waitVmcnt<0>(); // this wave's loads of tile it have landed
        ldsBarrier();   // every wave's have; every wave is past the step that read the other stage
        if (it + 1 < tcount) issue(kt0 + kMfmaKT, buf ^ 1);
        if (kSplit && it >= tcount) continue;
        const char *kt = &lds_all[half][buf][0], *vt = kt + kTileB;
        const bool whole = kt0 + kMfmaKT <= vis_first;
        const int nvis = int(min(vis_q - min(vis_q, kt0), size_t(kMfmaKT)));
        float p[4][4];
        float mx = m;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int krow = 32 * (t / 2) + 8 * (n / 4) + 4 * (t % 2) + n % 4; // A row n
            const char *kr = kt + krow * kRowB;
            const int sw = swzK(krow);
            f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) {
                const v4u kv = *reinterpret_cast<const v4u *>(kr + 16 * ((4 * kb + g4) ^ sw));
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(kv), qreg[kb], acc, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) p[t][i] = acc[i];
        }
        if (!whole) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int off = 32 * (t / 2) + 8 * g4 + 4 * (t % 2) + i;
                    p[t][i] = off < nvis ? p[t][i] : -INFINITY;
                }
        }
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, p[t][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float mc = mx == -INFINITY ? 0.0f : mx * c2;
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[t][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(p[t][i], c2, -mc));
                ps += p[t][i];
            }
        if (__builtin_expect(__any(mx != m), 0)) {
            const float corr = mx == m ? 1.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(m, c2, -mc));
            lsum *= corr;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] *= corr;
        }
        m = mx;
        lsum += ps;
        // the transposing reads' rows and column offset: keys 32 p2 + 8 g + n / 4 (and + 4),
        // columns 16 dt + 4 (n % 4) .. + 3, i.e. half n % 2 of chunk 2 dt + (n % 4) / 2
#pragma unroll
        for (int p2 = 0; p2 < 2; ++p2) {
            uint32_t hw[4], lw[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float x0 = p[2 * p2 + w / 2][2 * (w % 2)], x1 = p[2 * p2 + w / 2][2 * (w % 2) + 1];
                hw[w] = Bf16Cvt::narrow2Q(x0, x1);
                lw[w] = Bf16Cvt::narrow2Q(x0 - __uint_as_float(hw[w] << 16), x1 - __uint_as_float(hw[w] & 0xFFFF0000u));
            }
            const bf16x8 bhi = asBf16x8(v4u{hw[0], hw[1], hw[2], hw[3]});
            const bf16x8 blo = asBf16x8(v4u{lw[0], lw[1], lw[2], lw[3]});
            const int r0 = 32 * p2 + 8 * g4 + n / 4;
            const char *v0 = vt + r0 * kRowB + 8 * (n % 2), *v1 = v0 + 4 * kRowB;
            const int sw = swzV(r0); // rows r0 and r0 + 4 share it
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int cofs = 16 * ((2 * dt + (n % 4) / 2) ^ sw);
                const uint64_t e0 = ldsReadTr16(v0 + cofs), e1 = ldsReadTr16(v1 + cofs);
                const v4u vv = v4u{uint32_t(e0), uint32_t(e0 >> 32), uint32_t(e1), uint32_t(e1 >> 32)};
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vv), bhi, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vv), blo, o[dt], 0, 0, 0);
            }
        }
    }
    float lt = lsum + __shfl_xor(lsum, 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
    if constexpr (kSplit) {
        float *xch = reinterpret_cast<float *>(&lds_all[0][0][0]) + size_t(wave) * kWave * (2 + 4 * DT);
        __syncthreads();
        if (half == 1) {
            xch[lane] = m;
            xch[kWave + lane] = lt;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) xch[(2 + 4 * dt + i) * kWave + lane] = o[dt][i];
        }
        __syncthreads();
        if (half == 1) return;
        const float m1 = xch[lane], l1 = xch[kWave + lane];
        const float M = fmaxf(m, m1);
        const float f0 = m == M ? 1.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(m, c2, -M * c2));
        const float f1 = m1 == M ? 1.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(m1, c2, -M * c2));
        lt = lt * f0 + l1 * f1;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) o[dt][i] = o[dt][i] * f0 + xch[(2 + 4 * dt + i) * kWave + lane] * f1;
    }
    if (q0 + size_t(n) >= a.seq) return;
    const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
    uint16_t *op = static_cast<uint16_t *>(a.out) + (qi * a.nh + h) * D + 4 * g4;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        const uint32_t w0 = f32ToBf16(o[dt][0] * inv) | (f32ToBf16(o[dt][1] * inv) << 16);
        const uint32_t w1 = f32ToBf16(o[dt][2] * inv) | (f32ToBf16(o[dt][3] * inv) << 16);
        typedef uint32_t v2u __attribute__((ext_vector_type(2)));
        *reinterpret_cast<v2u *>(op + 16 * dt) = v2u{w0, w1};
    }
}

// ---- decode on MFMA (bf16 q / out, head_dim 128, cache in bf16 or INT8) ---------------
// Few queries, long cache.  Block = (query, kv head, key chunk), NW waves; each wave takes
// 32-key steps of the chunk on its own.  The MFMA columns are the G (<= 16) q heads of the
// kv head (columns past G hold zero queries and are never written): S^T = K Q^T over 2
// tiles of 16 keys (row m of tile t is key 8(m / 4) + 4t + m % 4, so lane group g holds keys
// 8g .. 8g + 7 and P^T is the B operand of one 32-key P V product as the lanes hold it),
// then O^T += V^T P^T with the V rows staged through the wave's own LDS slice and read
// back transposed (no block barrier inside the loop).  K enters the A operand straight
// from memory: bf16 rows, or INT8 codes turned into bf16(code * scale) (codesToBf16) with
// the step's scales shared by shuffles.  The waves merge in LDS; a split launch writes
// chunk partials in the layout attnCombine merges (max in scaled units).
constexpr int kDecWaves = 2;
constexpr int kDecKT = 32;   // keys per wave step

template <bool kInt8, int NW>
__global__ void __launch_bounds__(kWave * NW)
    attnDecodeMfma(AttnArgs a) {
    constexpr int D = 128, KB = D / 32, DT = D / 16;
    __shared__ __align__(16) char vrow[NW][kDecKT * 2 * D]; // the wave's V rows, chunks swizzled (swzV)
    __shared__ float st[NW][16][D + 2];
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const int n = lane % 16, g4 = lane / 16;

    unsigned b = blockIdx.x;
    const int c = int(b % unsigned(a.nchunks));
    b /= unsigned(a.nchunks);
    const int g = int(b % unsigned(a.nkvh));
    const size_t i = a.seq - 1 - size_t(b / unsigned(a.nkvh));
    const size_t vis = visibleKeys(a.total, a.seq, i);
    const size_t k0 = size_t(c) * size_t(a.chunk);
    const size_t k1 = min(vis, k0 + size_t(a.chunk));
    const bool col_ok = n < a.group;
    const int hq = g * a.group + (col_ok ? n : 0); // this column's q head (clamped)
    const float c2 = a.scale * 1.4426950408889634f;
    const size_t rstride = size_t(a.nkvh);          // rows between keys

    bf16x8 qreg[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        v4u r = v4u{0u, 0u, 0u, 0u};
        if (col_ok)
            r = *reinterpret_cast<const v4u *>(static_cast<const uint16_t *>(a.q) + (i * a.nh + hq) * D + 32 * kb + 8 * g4);
        qreg[kb] = asBf16x8(r);
    }
    float m = -INFINITY, lsum = 0.0f; // m: max of the raw dots
    f32x4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    for (size_t kt0 = k0 + size_t(wave) * kDecKT; kt0 < k1; kt0 += size_t(NW) * kDecKT) {
        const int nk = int(min(k1 - kt0, size_t(kDecKT)));
        const bool part = nk < kDecKT; // the chunk's last, partial step (wave-uniform)
        // Loads are unconditional: a key past the step reads the step's first key and is
        // zeroed after the load (partial steps only).  Loads under per-lane branches were
        // issued one round trip at a time.
        // V pieces: piece r of a lane is key 4r + lane / 16, columns 8 (lane % 16) .. + 7, so
        // 16 lanes read one row contiguously
        v4u vr[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int kr = 4 * r + lane / 16;
            const int key = kr < nk ? kr : 0;
            vr[r] = loadRow8<kInt8>(a.v, (kt0 + key) * rstride + g, 8 * (lane % 16));
        }
        // K operands: tile t, row n -> key 8(n / 4) + 4t + n % 4
        v4u ka[2][KB];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int off = 8 * (n / 4) + 4 * t + n % 4;
            const int key = off < nk ? off : 0;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
                ka[t][kb] = loadRow8<kInt8>(a.k, (kt0 + key) * rstride + g, 32 * kb + 8 * g4);
        }
        if (part) {
#pragma unroll
            for (int r = 0; r < 8; ++r)
                if (4 * r + lane / 16 >= nk) vr[r] = v4u{0u, 0u, 0u, 0u};
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int kb = 0; kb < KB; ++kb)
                    if (8 * (n / 4) + 4 * t + n % 4 >= nk) ka[t][kb] = v4u{0u, 0u, 0u, 0u};
        }
        if constexpr (kInt8) {
            // the step's scales, one load per lane (K for lanes 0-31, V for 32-63), handed
            // to the lanes that convert a row by lane shuffles
            const int sk = lane % kDecKT;
            float sreg = (lane < kDecKT ? a.ks : a.vs)[(kt0 + (sk < nk ? sk : 0)) * rstride + g];
            if (sk >= nk) sreg = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float sc = __shfl(sreg, 8 * (n / 4) + 4 * t + n % 4, kWave);
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) ka[t][kb] = codesToBf16(ka[t][kb], sc);
            }
#pragma unroll
            for (int r = 0; r < 8; ++r) vr[r] = codesToBf16(vr[r], __shfl(sreg, kDecKT + 4 * r + lane / 16, kWave));
        }
        float p[2][4];
        float mx = m;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(ka[t][kb]), qreg[kb], acc, 0, 0, 0);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) p[t][ii] = acc[ii];
        }
        if (nk < kDecKT) { // the chunk's last, partial step: keys past its end are masked
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) // key of D row 4g + ii
                    p[t][ii] = 8 * g4 + 4 * t + ii < nk ? p[t][ii] : -INFINITY;
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) mx = fmaxf(mx, p[t][ii]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        // a masked key (-inf) gets weight 0; mc = 0 while every score is -inf keeps it 0
        // rather than NaN, with no per-score select
        const float mc = mx == -INFINITY ? 0.0f : mx * c2;
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                p[t][ii] = __builtin_amdgcn_exp2f(__builtin_fmaf(p[t][ii], c2, -mc));
                ps += p[t][ii];
            }
        if (__builtin_expect(__any(mx != m), 0)) {
            const float corr = mx == m ? 1.0f : __builtin_amdgcn_exp2f(__builtin_fmaf(m, c2, -mc));
            lsum *= corr;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt] *= corr;
        }
        m = mx;
        lsum += ps;
        // V rows into this wave's slice as loaded (the previous step's reads of it are done:
        // one wave, in order; the fences keep the compiler from moving accesses across); 16
        // lanes write one row's 16 chunks, whatever the swizzle: no bank conflicts
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int kr = 4 * r + lane / 16;
            *reinterpret_cast<v4u *>(&vrow[wave][kr * 2 * D + 16 * ((lane % 16) ^ swzV(kr))]) = vr[r];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // P as bf16 hi + lo, two keys per conversion (key 8g + j is p[j / 4][j % 4])
        uint32_t hw[4], lw[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float x0 = p[w / 2][2 * (w % 2)], x1 = p[w / 2][2 * (w % 2) + 1];
            hw[w] = Bf16Cvt::narrow2Q(x0, x1);
            lw[w] = Bf16Cvt::narrow2Q(x0 - __uint_as_float(hw[w] << 16), x1 - __uint_as_float(hw[w] & 0xFFFF0000u));
        }
        const bf16x8 bhi = asBf16x8(v4u{hw[0], hw[1], hw[2], hw[3]});
        const bf16x8 blo = asBf16x8(v4u{lw[0], lw[1], lw[2], lw[3]});
        // V^T operands by transposing reads: lane n of group g gets keys 8g .. 8g + 7 of column
        // 16 dt + n from lanes reading key rows 8g + n / 4 (and + 4), columns 16 dt + 4 (n % 4) ..
        const int r0 = 8 * g4 + n / 4;
        const char *v0 = &vrow[wave][r0 * 2 * D + 8 * (n % 2)], *v1 = v0 + 4 * 2 * D;
        const int vsw = swzV(r0); // rows r0 and r0 + 4 share it
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int cofs = 16 * ((2 * dt + (n % 4) / 2) ^ vsw);
            const uint64_t e0 = ldsReadTr16(v0 + cofs), e1 = ldsReadTr16(v1 + cofs);
            const v4u vv = v4u{uint32_t(e0), uint32_t(e0 >> 32), uint32_t(e1), uint32_t(e1 >> 32)};
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vv), bhi, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(vv), blo, o[dt], 0, 0, 0);
        }
    }
    float lt = lsum + __shfl_xor(lsum, 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
    if (col_ok) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) st[wave][n][16 * dt + 4 * g4 + ii] = o[dt][ii];
        if (g4 == 0) {
            st[wave][n][D] = m;
            st[wave][n][D + 1] = lt;
        }
    }
    __syncthreads();
    for (int pi = threadIdx.x; pi < a.group * D; pi += kWave * NW) {
        const int j = pi / D, e = pi % D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, st[w][j][D]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = st[w][j][D];
            const float f = mw == M ? 1.0f : __builtin_amdgcn_exp2f((mw - M) * c2); // 1 for M = -inf, where l = o = 0
            L += st[w][j][D + 1] * f;
            O += st[w][j][e] * f;
        }
        const size_t ih = i * a.nh + size_t(g * a.group + j);
        if (a.nchunks == 1) {
            Fmt<BF16>::put(a.out, ih * D + e, L > 0.0f ? O / L : 0.0f);
        } else {
            float *pp = a.part + (ih * size_t(a.nchunks) + c) * (D + 2);
            pp[e] = O;
            if (e == 0) {
                pp[D] = M * a.scale; // the scaled units attnCombine works in
                pp[D + 1] = L;
            }
        }
    }
}

// Heads per wave for a kv group: the largest supported count that divides it.
int sliceOf(int group) {
    for (int g : {8, 6, 4, 2})
        if (group % g == 0) return g;
    return 1;
}

template <typename T, bool kInt8, int D, int G>
void launchGroup(const AttnArgs &a, size_t blocks, hipStream_t s) {
    constexpr int U = kInt8 ? 8 : 4; // 16 bytes of K and V codes per lane per step, or 32 of elements
    attnGroup<T, kInt8, D, G, U><<<unsigned(blocks), kWave * kWaves, 0, s>>>(a);
}

template <typename T, bool kInt8, int D>
void launchD(const AttnArgs &a, int G, size_t blocks, hipStream_t s) {
    switch (G) {
    case 8: return launchGroup<T, kInt8, D, 8>(a, blocks, s);
    case 6: return launchGroup<T, kInt8, D, 6>(a, blocks, s);
    case 4: return launchGroup<T, kInt8, D, 4>(a, blocks, s);
    case 2: return launchGroup<T, kInt8, D, 2>(a, blocks, s);
    default: return launchGroup<T, kInt8, D, 1>(a, blocks, s);
    }
}

// The vector kernels' shape and alignment condition.
bool vecShape(const AttnArgs &a, int d, int dv, bool int8) {
    const auto aligned = [](const void *p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; };
    return d == dv && (d == 64 || d == 128) && aligned(a.q, 16) && aligned(a.out, 16) &&
           (int8 ? aligned(a.k, 8) && aligned(a.v, 8) : aligned(a.k, 16) && aligned(a.v, 16));
}

// The bf16 prefill on MFMA: head_dim 128, 16 or more queries, a non-empty cache and a
// positive finite scale (the kernel tracks the max of the raw dot products).
bool prefillMfma(const AttnArgs &a, int d, int dv, bool int8, bool bf16) {
    if (!bf16 || !vecShape(a, d, dv, int8)) return false;
    const size_t mblocks = (a.seq + kMfmaQ - 1) / kMfmaQ * size_t(a.nkvh) * size_t(a.group / sliceOf(a.group));
    return d == 128 && a.total > 0 && a.seq >= size_t(kMfmaQ) && mblocks < (size_t(1) << 31) &&
           a.scale > 0.0f && std::isfinite(a.scale);
}

template <typename T, bool kInt8>
void launch(AttnArgs a, int d, int dv, void *ws, size_t ws_bytes, hipStream_t s) {
    if (a.seq == 0 || a.nh == 0) return;
    const bool vec = vecShape(a, d, dv, kInt8);
    if (!vec) {
        a.nchunks = 1;
        attnScalar<T, kInt8><<<unsigned(a.seq * size_t(a.nh)), kWave, size_t(dv) * sizeof(float), s>>>(a, d, dv);
        return;
    }
    const int G = sliceOf(a.group);
    a.slices = a.group / G;
    // bf16 prefill (16 or more queries, cache in bf16 or INT8) goes to the MFMA kernel;
    // decode and the other types stay on the vector kernel
    if constexpr (std::is_same_v<T, BF16>) {
        const size_t mblocks = (a.seq + kMfmaQ - 1) / kMfmaQ * size_t(a.nkvh) * size_t(a.slices);
        if (prefillMfma(a, d, dv, kInt8, true)) {
            a.nchunks = 1;
            if constexpr (kInt8) {
                // An INT8 cache whose bf16 form fits the workspace is dequantized once (both
                // caches in one launch, bf16(code * scale) as the tiles would be staged) and
                // attended as bf16: the tile staging of every query block no longer converts
                // the same codes again.  Same operands, so the same bits.
                const size_t cache_el = a.total * size_t(a.nkvh) * size_t(d);
                if (2 * cache_el * sizeof(uint16_t) <= ws_bytes) {
                    uint16_t *kd = static_cast<uint16_t *>(ws), *vd = kd + cache_el;
                    dequantizeInt8Pair(kd, static_cast<const int8_t *>(a.k), a.ks, a.total * size_t(a.nkvh), vd,
                                       static_cast<const int8_t *>(a.v), a.vs, a.total * size_t(a.nkvh),
                                       size_t(d), LLAISYS_DTYPE_BF16, s);
                    AttnArgs b = a;
                    b.k = kd;
                    b.v = vd;
                    b.ks = b.vs = nullptr;
                    return launch<T, false>(b, d, dv, nullptr, 0, s);
                }
            }
            // few blocks per CU: the causal imbalance is not averaged out across blocks, so
            // the key tiles of each block are split over two wave sets
            // (groups of 8 keep one wave per head: 16 waves of 8 heads would spill registers).
            // A bf16 cache's tiles go HBM -> LDS directly (attnMfmaLds; its byte offsets
            // within a tile take 32 bits, so beyond 2^17 kv heads the register-staged kernel).
            if (!kInt8 && size_t(a.nkvh) * 256 * kMfmaKT < (size_t(1) << 31)) {
                if (mblocks <= 512 && G <= 6) {
                    switch (G) {
                    case 6: attnMfmaLds<6, true><<<unsigned(mblocks), kWave * 12, 0, s>>>(a); return;
                    case 4: attnMfmaLds<4, true><<<unsigned(mblocks), kWave * 8, 0, s>>>(a); return;
                    case 2: attnMfmaLds<2, true><<<unsigned(mblocks), kWave * 4, 0, s>>>(a); return;
                    default: attnMfmaLds<1, true><<<unsigned(mblocks), kWave * 2, 0, s>>>(a); return;
                    }
                }
                switch (G) {
                case 8: attnMfmaLds<8, false><<<unsigned(mblocks), kWave * 8, 0, s>>>(a); return;
                case 6: attnMfmaLds<6, false><<<unsigned(mblocks), kWave * 6, 0, s>>>(a); return;
                case 4: attnMfmaLds<4, false><<<unsigned(mblocks), kWave * 4, 0, s>>>(a); return;
                case 2: attnMfmaLds<2, false><<<unsigned(mblocks), kWave * 2, 0, s>>>(a); return;
                default: attnMfmaLds<1, false><<<unsigned(mblocks), kWave, 0, s>>>(a); return;
                }
            }
            if (mblocks <= 512 && G <= 6) {
                switch (G) {
                case 6: attnMfma<6, true, kInt8><<<unsigned(mblocks), kWave * 12, 0, s>>>(a); return;
                case 4: attnMfma<4, true, kInt8><<<unsigned(mblocks), kWave * 8, 0, s>>>(a); return;
                case 2: attnMfma<2, true, kInt8><<<unsigned(mblocks), kWave * 4, 0, s>>>(a); return;
                default: attnMfma<1, true, kInt8><<<unsigned(mblocks), kWave * 2, 0, s>>>(a); return;
                }
            }
            switch (G) {
            case 8: attnMfma<8, false, kInt8><<<unsigned(mblocks), kWave * 8, 0, s>>>(a); return;
            case 6: attnMfma<6, false, kInt8><<<unsigned(mblocks), kWave * 6, 0, s>>>(a); return;
            case 4: attnMfma<4, false, kInt8><<<unsigned(mblocks), kWave * 4, 0, s>>>(a); return;
            case 2: attnMfma<2, false, kInt8><<<unsigned(mblocks), kWave * 2, 0, s>>>(a); return;
            default: attnMfma<1, false, kInt8><<<unsigned(mblocks), kWave, 0, s>>>(a); return;
            }
        }
    }
    // bf16 decode (fewer than 16 queries): the MFMA decode kernel, one 32-key step per wave
    // when the chunks allow (up to 1024 per (query, head), partials within the workspace)
    if constexpr (std::is_same_v<T, BF16>) {
        if (d == 128 && a.total > 0 && a.seq < size_t(kMfmaQ) && a.group <= 16 && a.scale > 0.0f &&
            std::isfinite(a.scale)) {
            // waves per block: 8 for caches of 16K+ keys (half the partials to merge: 32K
            // decode 14.6 -> 13.3 us INT8 KV, 14.4 -> 13.8 us bf16 KV), 2 below (more blocks
            // for the shorter chains: the 4096-key decode step took 1.157 ms with 4, 1.122 ms
            // with 2, 1.144 ms with 1; it lost with 8)
            const int nw = a.total >= 16384 ? 8 : kDecWaves;
            const size_t bk = size_t(nw) * kDecKT; // keys per block step
            const size_t pairs = a.seq * size_t(a.nh);
            size_t nchunks = std::min<size_t>((a.total + bk - 1) / bk, 1024);
            nchunks = std::max<size_t>(1, std::min(nchunks, ws_bytes / (size_t(d + 2) * sizeof(float) * pairs)));
            a.nchunks = int(nchunks);
            a.chunk = int(std::min<size_t>((a.total + nchunks - 1) / nchunks, size_t(INT32_MAX)));
            a.part = static_cast<float *>(ws);
            const unsigned blocks = unsigned(a.seq * size_t(a.nkvh) * nchunks);
            if (nw == 8)
                attnDecodeMfma<kInt8, 8><<<blocks, kWave * 8, 0, s>>>(a);
            else
                attnDecodeMfma<kInt8, kDecWaves><<<blocks, kWave * kDecWaves, 0, s>>>(a);
            if (nchunks > 1)
                launchCombine<T>(a.out, a.part, a.nchunks, d, pairs, s);
            return;
        }
    }
    // A block's waves each take one step of keys per chunk when the launch is split: about
    // 2048 waves for decode, partials within the workspace and at most 1024 per (query, head).
    const int U = kInt8 ? 8 : 4;
    const size_t tile = size_t(kWave / (d / 8)) * U * kWaves; // keys per block step
    const size_t groups = a.seq * size_t(a.nkvh) * size_t(a.slices);
    size_t nchunks = 1;
    if (groups < 512 && a.total > tile) {
        nchunks = std::min<size_t>((a.total + tile - 1) / tile, 1024);
        const size_t per = size_t(d + 2) * sizeof(float) * a.seq * size_t(a.nh);
        nchunks = std::max<size_t>(1, std::min(nchunks, ws_bytes / per));
    }
    a.nchunks = int(nchunks);
    a.chunk = int(std::min<size_t>(nchunks == 1 ? std::max<size_t>(a.total, 1)
                                                : (a.total + nchunks - 1) / nchunks,
                                   size_t(INT32_MAX)));
    a.part = static_cast<float *>(ws);
    const size_t blocks = groups * nchunks;
    if (d == 64)
        launchD<T, kInt8, 64>(a, G, blocks, s);
    else
        launchD<T, kInt8, 128>(a, G, blocks, s);
    if (nchunks > 1)
        launchCombine<T>(a.out, a.part, a.nchunks, d, a.seq * size_t(a.nh), s);
}

template <bool kInt8>
void dispatch(AttnArgs a, int d, int dv, llaisysDataType_t dt, void *ws, size_t ws_bytes, hipStream_t s) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launch<F32, kInt8>(a, d, dv, ws, ws_bytes, s);
    case LLAISYS_DTYPE_BF16: return launch<BF16, kInt8>(a, d, dv, ws, ws_bytes, s);
    case LLAISYS_DTYPE_F16: return launch<F16, kInt8>(a, d, dv, ws, ws_bytes, s);
    default: return;
    }
}

} // namespace

// ---- scratch of the allocation-free entry point -----------------------------------------
// File-scope device array holding the split attention's partials for
// llaisysSelfAttentionInt8KVNoAlloc.  Each GPU the library runs on holds its own copy (at its
// own address) until the process ends.  In host code the name `scratch` is only a stand-in:
// its device address comes from hipGetSymbolAddress, resolved once per device with that
// device current, and only that address is ever handed to kernels.  Nothing in it needs to
// start at zero: every partial a launch reads was written earlier in the same launch pair.
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kScratchDevices] = {};
} // namespace

void *noAllocScratch(int device, char *err, size_t err_len) {
    if (device < 0 || device >= kScratchDevices) {
        snprintf(err, err_len, "device id %d out of range", device);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *ptr = nullptr;
        const hipError_t st = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (st != hipSuccess || ptr == nullptr) {
            snprintf(err, err_len, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(st));
            return nullptr;
        }
        g_scratch_ptr[device] = ptr;
    }
    return g_scratch_ptr[device];
}

size_t selfAttentionInt8KVScratchBytes(const void *out, const void *q, const void *k, const void *v,
                                       size_t seq, size_t total, size_t nh, size_t nkvh, size_t d,
                                       size_t dv, float scale, llaisysDataType_t dt, size_t cap) {
    AttnArgs a{};
    a.out = const_cast<void *>(out);
    a.q = q;
    a.k = k;
    a.v = v;
    a.seq = seq;
    a.total = total;
    a.nh = int(nh);
    a.nkvh = int(nkvh);
    a.group = int(nh / nkvh);
    a.scale = scale;
    if (seq > 0 && nh > 0 && prefillMfma(a, int(d), int(dv), true, dt == LLAISYS_DTYPE_BF16)) {
        const size_t cache = 2 * total * nkvh * d * sizeof(uint16_t);
        return cache <= cap ? cache : 0;
    }
    return selfAttentionWorkspaceBytes(seq, nh, d);
}

size_t selfAttentionWorkspaceBytes(size_t seq, size_t nh, size_t head_dim) {
    // up to 1024 partials of head_dim + 2 floats per (query, head), capped at 64 MiB: a
    // smaller workspace only lowers the chunk count (decode: 12 heads x 1024 x 520 B)
    return std::min<size_t>(std::min<size_t>(seq * nh, 4096) * 1024 * (head_dim + 2) * sizeof(float),
                            size_t(64) << 20);
}

void selfAttention(void *out, const void *q, const void *k, const void *v, const float *k_scale,
                   const float *v_scale, size_t seq, size_t total, size_t nh, size_t nkvh,
                   size_t d, size_t dv, float scale, llaisysDataType_t dt, void *ws,
                   size_t ws_bytes, hipStream_t s) {
    AttnArgs a{};
    a.out = out;
    a.q = q;
    a.k = k;
    a.v = v;
    a.ks = k_scale;
    a.vs = v_scale;
    a.seq = seq;
    a.total = total;
    a.nh = int(nh);
    a.nkvh = int(nkvh);
    a.group = int(nh / nkvh);
    a.scale = scale;
    if (k_scale)
        dispatch<true>(a, int(d), int(dv), dt, ws, ws_bytes, s);
    else
        dispatch<false>(a, int(d), int(dv), dt, ws, ws_bytes, s);
}

} // namespace llaisys::kernels
