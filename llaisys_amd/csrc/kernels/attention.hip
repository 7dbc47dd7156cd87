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
// Design (HBM-bound for decode, VALU-bound for long prefill): one wavefront per q head; the
// waves of a block are q heads of one kv head, so they read the same K / V rows (the
// later waves hit the lines the first brought in).  A key row of D elements is spread over
// R = D / 8 lanes, 8 elements per lane (one 16-byte load for bf16 / f16, 8 bytes of codes
// for INT8), so one load instruction covers 64 / R keys.  Per batch of U instructions the
// wave forms its scores (8 FMAs, a butterfly over R lanes), updates the running max once,
// and folds p * v into per-lane accumulators.  Long key ranges with few (query, head) pairs
// (decode) are cut into chunks whose partial (max, sum, output) a second kernel merges.
// No MFMA here: a decode step is a matrix-vector product per head.
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

#include <algorithm>
#include <cmath>

namespace llaisys::kernels {

namespace {

constexpr int kU = 4;              // load instructions of K (and V) per batch
constexpr int kMaxWavesPerBlock = 8;
constexpr int kChunkKeys = 256;    // smallest key chunk of a split launch

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
    int nh, nkvh, group, head_blocks, nchunks, chunk;
    float scale;
};

// Visible keys of query i: [0, vis).
__device__ __forceinline__ size_t visibleKeys(size_t total, size_t seq, size_t i) {
    const size_t cur = total - seq + i; // size_t arithmetic, as the reference
    return cur >= total ? total : cur + 1;
}

template <typename T, bool kInt8, int D>
__global__ void __launch_bounds__(kWave * kMaxWavesPerBlock)
    attnWave(AttnArgs a) {
    using IO = RowIO<T, kInt8>;
    constexpr int R = D / 8;          // lanes per key row
    constexpr int KPW = kWave / R;    // keys per load instruction
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const int rs = lane / R, col = (lane % R) * 8;

    // block -> (query, kv head, head block, chunk); the latest queries (most keys) first
    unsigned b = blockIdx.x;
    const int c = int(b % unsigned(a.nchunks));
    b /= unsigned(a.nchunks);
    const int hb = int(b % unsigned(a.head_blocks));
    b /= unsigned(a.head_blocks);
    const int g = int(b % unsigned(a.nkvh));
    const size_t i = a.seq - 1 - size_t(b / unsigned(a.nkvh));
    const int hg = hb * kMaxWavesPerBlock + wave; // head within the kv group
    if (hg >= a.group) return;                    // wave-uniform; no block barrier below
    const int h = g * a.group + hg;

    const size_t vis = visibleKeys(a.total, a.seq, i);
    const size_t k0 = size_t(c) * size_t(a.chunk);
    const size_t k1 = min(vis, k0 + size_t(a.chunk));

    float qv[8];
    {
        const char *qp = static_cast<const char *>(a.q) + ((i * a.nh + h) * D + col) * Fmt<T>::kBytes;
        typename RowIO<T, false>::Raw r;
#pragma unroll
        for (int k = 0; k < RowIO<T, false>::kRegs; ++k) r.r[k] = *reinterpret_cast<const v4u *>(qp + 16 * k);
        RowIO<T, false>::unpack(r, 0.0f, qv);
    }
    float m = -INFINITY, l = 0.0f, o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;

    for (size_t kb = k0; kb < k1; kb += size_t(KPW) * kU) {
        typename IO::Raw kr[kU], vr[kU];
        float ksc[kU], vsc[kU];
        bool ok[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
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
        float s[kU];
        float mx = m;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            float kf[8];
            IO::unpack(kr[u], ksc[u], kf);
            float dot = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) dot = __builtin_fmaf(qv[e], kf[e], dot);
            dot = waveGroupReduce<R, SumOp>(dot);
            s[u] = ok[u] ? dot * a.scale : -INFINITY;
            mx = fmaxf(mx, s[u]);
        }
        // a -inf score is weight 0 (reference :111-113); m == mx keeps the state as is
        const float corr = mx == m ? 1.0f : __expf(m - mx);
        l *= corr;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] *= corr;
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const float p = s[u] == -INFINITY ? 0.0f : __expf(s[u] - mx);
            float vf[8];
            IO::unpack(vr[u], vsc[u], vf);
            l += p;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(p, vf[e], o[e]);
        }
        m = mx;
    }

    // merge the KPW key slots of the wave (lanes R, 2R, ... apart hold the same columns)
#pragma unroll
    for (int off = R; off < kWave; off *= 2) {
        const float mo = __shfl_xor(m, off, kWave), lo = __shfl_xor(l, off, kWave);
        const float M = fmaxf(m, mo);
        const float fa = m == M ? 1.0f : __expf(m - M);
        const float fb = mo == M ? 1.0f : __expf(mo - M);
        // (a slot that saw no key has m = -inf and l = 0, o = 0: its factor may be 1 only
        // when M is -inf too, and then every term is 0)
        l = l * fa + lo * fb;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float oo = __shfl_xor(o[e], off, kWave);
            o[e] = o[e] * fa + oo * fb;
        }
        m = M;
    }
    if (lane >= R) return;
    if (a.nchunks == 1) {
        float y[8];
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = o[e] * inv;
        char *op = static_cast<char *>(a.out) + ((i * a.nh + h) * D + col) * Fmt<T>::kBytes;
        // pack: the reference rounding also for a NaN carrying the caller's scale payload
        if constexpr (Fmt<T>::kBytes == 2) {
            *reinterpret_cast<v4u *>(op) = Fmt<T>::pack(y);
        } else {
            *reinterpret_cast<v4u *>(op) = Fmt<T>::pack(y);
            *reinterpret_cast<v4u *>(op + 16) = Fmt<T>::pack(y + 4);
        }
        return;
    }
    float *pp = a.part + ((i * a.nh + h) * size_t(a.nchunks) + c) * (D + 2);
    *reinterpret_cast<float4 *>(pp + col) = make_float4(o[0], o[1], o[2], o[3]);
    *reinterpret_cast<float4 *>(pp + col + 4) = make_float4(o[4], o[5], o[6], o[7]);
    if (lane == 0) {
        pp[D] = m;
        pp[D + 1] = l;
    }
}

// Merge of the chunk partials of a split launch: one 64-thread block per (query, head).
template <typename T>
__global__ void __launch_bounds__(kWave)
    attnCombine(void *out, const float *part, int nh, int nchunks, int D) {
    const size_t ih = blockIdx.x; // i * nh + h
    const float *pp = part + ih * size_t(nchunks) * (D + 2);
    float M = -INFINITY;
    for (int c = 0; c < nchunks; ++c) M = fmaxf(M, pp[size_t(c) * (D + 2) + D]);
    float L = 0.0f;
    for (int c = 0; c < nchunks; ++c) {
        const float mc = pp[size_t(c) * (D + 2) + D];
        if (mc != -INFINITY) L += pp[size_t(c) * (D + 2) + D + 1] * __expf(mc - M);
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    for (int e = threadIdx.x; e < D; e += kWave) {
        float acc = 0.0f;
        for (int c = 0; c < nchunks; ++c) {
            const float mc = pp[size_t(c) * (D + 2) + D];
            if (mc != -INFINITY) acc += pp[size_t(c) * (D + 2) + e] * __expf(mc - M);
        }
        Fmt<T>::put(out, ih * D + e, acc * inv);
    }
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

template <typename T, bool kInt8>
void launch(AttnArgs a, int d, int dv, void *ws, size_t ws_bytes, hipStream_t s) {
    if (a.seq == 0 || a.nh == 0) return;
    const auto aligned = [](const void *p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; };
    const bool vec = d == dv && (d == 64 || d == 128) &&
                     aligned(a.q, 16) && aligned(a.out, 16) &&
                     (kInt8 ? aligned(a.k, 8) && aligned(a.v, 8) : aligned(a.k, 16) && aligned(a.v, 16));
    if (!vec) {
        a.nchunks = 1;
        attnScalar<T, kInt8><<<unsigned(a.seq * size_t(a.nh)), kWave, size_t(dv) * sizeof(float), s>>>(a, d, dv);
        return;
    }
    // Split the keys when few (query, head) pairs would leave the GPU idle: aim at ~8192
    // waves, chunks of at least kChunkKeys keys, partials within the workspace.
    const size_t pairs = a.seq * size_t(a.nh);
    size_t nchunks = 1;
    if (pairs < 4096 && a.total > size_t(kChunkKeys)) {
        nchunks = std::min((a.total + kChunkKeys - 1) / kChunkKeys, (8192 + pairs - 1) / pairs);
        const size_t per = size_t(d + 2) * sizeof(float);
        nchunks = std::max<size_t>(1, std::min(nchunks, ws_bytes / (pairs * per)));
    }
    a.nchunks = int(nchunks);
    a.chunk = int(std::min<size_t>(nchunks == 1 ? std::max<size_t>(a.total, 1)
                                                : (a.total + nchunks - 1) / nchunks,
                                   size_t(INT32_MAX)));
    a.part = static_cast<float *>(ws);
    a.head_blocks = (a.group + kMaxWavesPerBlock - 1) / kMaxWavesPerBlock;
    const int waves = std::min(a.group, kMaxWavesPerBlock);
    const size_t blocks = a.seq * size_t(a.nkvh) * size_t(a.head_blocks) * nchunks;
    switch (d) {
    case 64: attnWave<T, kInt8, 64><<<unsigned(blocks), waves * kWave, 0, s>>>(a); break;
    default: attnWave<T, kInt8, 128><<<unsigned(blocks), waves * kWave, 0, s>>>(a); break;
    }
    if (nchunks > 1)
        attnCombine<T><<<unsigned(pairs), kWave, 0, s>>>(a.out, a.part, a.nh, a.nchunks, d);
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

size_t selfAttentionWorkspaceBytes(size_t head_dim) {
    // a split launch has pairs < 4096 and at most ceil(8192 / pairs) chunks per pair, so
    // fewer than 8192 + 4096 partials of head_dim + 2 floats
    return size_t(8192 + 4096) * (head_dim + 2) * sizeof(float);
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
