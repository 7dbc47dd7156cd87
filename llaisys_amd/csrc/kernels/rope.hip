// Rotate-half RoPE for gfx950, for one tensor or for q and k in one launch.
//
// Semantics: reference src/ops/rope/cpu/rope_cpu.cpp:28-44.  For token i, head h and
// j < d/2: freq_j = 1 / pow((double)theta, (double)(2.0f * j / d)), angle = (double)p_i *
// freq_j, and the pair (x_j, x_{j+d/2}) is rotated in double precision; the result is
// rounded double -> float -> element type.  freq_j is computed on the host with the same
// libm pow the reference calls, so the angles are bit-identical; cos/sin come from the
// device's double-precision libm (within an ulp of glibc's, which the final float rounding
// absorbs).
//
// Design: HBM-bound.  A 256-thread block owns a run of tokens.  Each lane first issues the
// 16-byte loads of its (token, head, 8-pair) items (both halves of the head), then the
// block computes the (cos, sin) pairs of its tokens into LDS -- d/2 sincos per token,
// shared by every q and k head -- so the f64 trig overlaps the load latency; finally each
// lane rotates and stores its items.  Loads and stores are non-temporal (read once,
// written once).  q and k of the same tokens go through one launch.
#include "common.hpp"
#include "launch.hpp"
#include "rope_common.hpp"
#include "rowplan.hpp"

#include <algorithm>
#include <cmath>

namespace llaisys::kernels {

namespace {

using namespace rope_detail;

constexpr int kMaxItems = 4;    // 16-byte items per lane held in registers

// Two tensors sharing positions and head_dim; tensor 1 may be absent (n_heads1 == 0).
struct RopePair {
    void *out0;
    const void *in0;
    void *out1;
    const void *in1;
    int n_heads0;
    int n_heads1;
};

// Lane layout: item = one 16-byte vector of a head row, items of a row on consecutive
// lanes, so every load / store instruction of a wavefront covers one contiguous 1 KB
// (an earlier layout that gave each lane the vector pair (j, j + d/2) split every
// instruction into 8 half-rows 256 B apart and ran ~20 % slower).  The rotation partner of
// a vector sits VPH lanes away and is fetched with a cross-lane exchange.  VPH (16-byte
// vectors per half head) is a power of two <= 32, so a row never straddles a wavefront
// and item -> (row, vector) is a shift; item -> token uses `tok_magic`
// (floor(2^32 / items_per_token) + 1, exact while item * items_per_token < 2^32).
template <typename T, int IPT, int VPH>
__global__ void __launch_bounds__(256)
    ropeVec(RopePair tp, const int64_t *__restrict__ pos, size_t seq, int tok_per_block,
            uint32_t tok_magic, FreqTable ft) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    constexpr int kRowVec = 2 * VPH; // vectors per head row
    constexpr int kHalf = VPH * N;
    constexpr int kShift = __builtin_ctz(kRowVec);
    __shared__ double2 cs[kLdsPairs];

    const int per_tok = (tp.n_heads0 + tp.n_heads1) * kRowVec;
    const size_t t0 = size_t(blockIdx.x) * tok_per_block;
    const int ntok = int(min(size_t(tok_per_block), seq - t0));
    const int items = ntok * per_tok;

    // 1. issue this lane's loads (one contiguous 16-byte vector per item)
    v4u raw[IPT];
    size_t off[IPT];
    int tok[IPT];
    bool second[IPT];
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = threadIdx.x + k * 256;
        if (it < items) {
            const int tt = int(__umulhi(uint32_t(it), tok_magic));
            const int rem = it - tt * per_tok;
            int h = rem >> kShift;
            const int v = rem & (kRowVec - 1);
            second[k] = h >= tp.n_heads0;
            const int nh = second[k] ? tp.n_heads1 : tp.n_heads0;
            if (second[k]) h -= tp.n_heads0;
            tok[k] = tt;
            off[k] = ((t0 + tt) * size_t(nh) + h) * size_t(2 * kHalf) + size_t(v) * N;
            raw[k] = load16Stream<T>(second[k] ? tp.in1 : tp.in0, off[k]);
        } else {
            raw[k] = v4u{0, 0, 0, 0};
        }
    }

    // 2. (cos, sin) of this block's tokens
    for (int i = threadIdx.x; i < ntok * kHalf; i += 256) {
        const int tt = i / kHalf, j = i % kHalf;
        const double ang = double(pos[t0 + tt]) * ft.f[j];
        double sn, c;
        sincos(ang, &sn, &c);
        cs[i] = make_double2(c, sn);
    }
    __syncthreads();

    // 3. exchange with the partner vector, rotate, store.  First half of a row:
    //    y = x*c - partner*s; second half: y = x*c + partner*s -- the reference's
    //    a*c - b*s and b*c + a*s with the same operation order (rope_cpu.cpp:40-41).
    const int v_lane = threadIdx.x & (kRowVec - 1);
    const bool upper = v_lane >= VPH;
    const int jv = v_lane & (VPH - 1);
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        v4u other;
        other.x = partnerOf<VPH>(raw[k].x);
        other.y = partnerOf<VPH>(raw[k].y);
        other.z = partnerOf<VPH>(raw[k].z);
        other.w = partnerOf<VPH>(raw[k].w);
        const int it = threadIdx.x + k * 256;
        if (it < items) {
            float x[N], p[N], y[N];
            F::unpack(raw[k], x);
            F::unpack(other, p);
            const double2 *row = cs + tok[k] * kHalf + jv * N;
#pragma unroll
            for (int e = 0; e < N; ++e) {
                const double c = row[e].x, sn = row[e].y;
                const double own = x[e], partner = upper ? double(p[e]) : -double(p[e]);
                y[e] = float(own * c + partner * sn);
            }
            store16Stream<T>(second[k] ? tp.out1 : tp.out0, off[k], F::pack(y));
        }
    }
}

// Any head_dim / alignment: one thread per (token, head, j) pair of one tensor.
template <typename T>
__global__ void __launch_bounds__(256)
    ropeScalar(void *out, const void *in, const int64_t *pos, size_t seq, size_t n_heads,
               size_t d, float theta, FreqTable ft) {
    using F = Fmt<T>;
    const size_t half = d / 2;
    const size_t pairs = seq * n_heads * half;
    for (size_t k = size_t(blockIdx.x) * 256 + threadIdx.x; k < pairs;
         k += size_t(gridDim.x) * 256) {
        const size_t j = k % half;
        const size_t th = k / half; // token * n_heads + head
        const size_t tok = th / n_heads;
        const double ang = double(pos[tok]) * freqOf(ft, int(j), int(d), theta);
        double sn, c;
        sincos(ang, &sn, &c);
        const size_t base = th * d;
        const double A = F::get(in, base + j), B = F::get(in, base + j + half);
        F::put(out, base + j, float(A * c - B * sn));
        F::put(out, base + j + half, float(B * c + A * sn));
    }
}

template <typename T, int IPT>
void launchIpt(int vph, const RopePair &tp, const int64_t *pos, size_t seq, size_t tpb,
               uint32_t magic, const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor(seq, tpb);
    switch (vph) {
    case 2: ropeVec<T, IPT, 2><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic, ft); break;
    case 4: ropeVec<T, IPT, 4><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic, ft); break;
    case 8: ropeVec<T, IPT, 8><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic, ft); break;
    case 16: ropeVec<T, IPT, 16><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic, ft); break;
    case 32: ropeVec<T, IPT, 32><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic, ft); break;
    default: break;
    }
}

// Items per block: about 256 (one 16-byte item per lane).  Measured on MI355X for the
// Qwen2 shapes, 224-896 items per block are within 2 %, 128 is 15 % slower.  A persistent
// variant (blocks looping over token groups with the next group's loads in flight) was
// slower still: with one token per group the 64 f64 sincos ran on one wavefront while the
// other three waited at the per-group barrier.
constexpr size_t kItemsPerBlock = 256;

template <typename T>
bool launchVec(const RopePair &tp, const int64_t *pos, size_t seq, size_t d, const FreqTable &ft,
               hipStream_t s) {
    constexpr int N = Fmt<T>::kVec;
    const size_t half = d / 2;
    if (half % N != 0 || half > size_t(kMaxHalf)) return false;
    const size_t vph = half / N;
    if (vph & (vph - 1)) return false; // not a power of two
    for (const void *p : {static_cast<const void *>(tp.out0), tp.in0,
                          static_cast<const void *>(tp.out1), tp.in1})
        if (p && !aligned16(p)) return false;
    if (vph > 32) return false; // a head row must fit in one wavefront
    const size_t per_tok = size_t(tp.n_heads0 + tp.n_heads1) * 2 * vph;
    if (per_tok == 0 || per_tok > size_t(256 * kMaxItems)) return false;
    // Tokens per block: the fewest that keep >= 90 % of the lanes busy (q only: 4 tokens of
    // 192 items = 3 full items per lane), else one block's worth of ~256 items.
    size_t tpb = std::max<size_t>(1, kItemsPerBlock / per_tok);
    for (size_t t = 1; t * per_tok <= size_t(256 * kMaxItems); ++t) {
        const size_t slots = (t * per_tok + 255) / 256 * 256;
        if (t * per_tok * 10 >= slots * 9) {
            tpb = t;
            break;
        }
    }
    tpb = std::min(tpb, size_t(kLdsPairs) / half);
    const int ipt = int((tpb * per_tok + 255) / 256);
    const uint32_t magic = uint32_t((uint64_t(1) << 32) / per_tok + 1);
    switch (ipt) {
    case 1: launchIpt<T, 1>(int(vph), tp, pos, seq, tpb, magic, ft, s); break;
    case 2: launchIpt<T, 2>(int(vph), tp, pos, seq, tpb, magic, ft, s); break;
    case 3: launchIpt<T, 3>(int(vph), tp, pos, seq, tpb, magic, ft, s); break;
    default: launchIpt<T, 4>(int(vph), tp, pos, seq, tpb, magic, ft, s); break;
    }
    return true;
}

template <typename T>
void launchScalar(void *out, const void *in, const int64_t *pos, size_t seq, size_t nh,
                  size_t d, float theta, const FreqTable &ft, hipStream_t s) {
    const size_t pairs = seq * nh * (d / 2);
    if (pairs == 0) return;
    const unsigned grid = unsigned(std::min<size_t>(blocksFor(pairs, 256), 65536));
    ropeScalar<T><<<grid, 256, 0, s>>>(out, in, pos, seq, nh, d, theta, ft);
}

template <typename T>
void launch(const RopePair &tp, const int64_t *pos, size_t seq, size_t d, float theta,
            hipStream_t s) {
    if (seq == 0 || d == 0) return;
    const FreqTable ft = hostFreqs(d, theta);
    if (launchVec<T>(tp, pos, seq, d, ft, s)) return;
    launchScalar<T>(tp.out0, tp.in0, pos, seq, size_t(tp.n_heads0), d, theta, ft, s);
    if (tp.n_heads1) launchScalar<T>(tp.out1, tp.in1, pos, seq, size_t(tp.n_heads1), d, theta, ft, s);
}

template <typename T>
void launchAny(void *qo, const void *qi, size_t nhq, void *ko, const void *ki, size_t nhk,
               const int64_t *pos, size_t seq, size_t d, float theta, hipStream_t s) {
    if (nhq > size_t(INT32_MAX / 2) || nhk > size_t(INT32_MAX / 2)) {
        const FreqTable ft = hostFreqs(d, theta);
        launchScalar<T>(qo, qi, pos, seq, nhq, d, theta, ft, s);
        if (nhk) launchScalar<T>(ko, ki, pos, seq, nhk, d, theta, ft, s);
        return;
    }
    launch<T>(RopePair{qo, qi, ko, ki, int(nhq), int(nhk)}, pos, seq, d, theta, s);
}

} // namespace

void rope(void *out, const void *in, const int64_t *pos, size_t seq, size_t n_heads,
          size_t head_dim, float theta, llaisysDataType_t dt, hipStream_t s) {
    ropeQK(out, in, n_heads, nullptr, nullptr, 0, pos, seq, head_dim, theta, dt, s);
}

void ropeQK(void *q_out, const void *q_in, size_t nh_q, void *k_out, const void *k_in,
            size_t nh_k, const int64_t *pos, size_t seq, size_t head_dim, float theta,
            llaisysDataType_t dt, hipStream_t s) {
    if (nh_q == 0 && nh_k == 0) return;
    if (nh_q == 0) return ropeQK(k_out, k_in, nh_k, nullptr, nullptr, 0, pos, seq, head_dim, theta, dt, s);
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launchAny<F32>(q_out, q_in, nh_q, k_out, k_in, nh_k, pos, seq, head_dim, theta, s);
    case LLAISYS_DTYPE_BF16: return launchAny<BF16>(q_out, q_in, nh_q, k_out, k_in, nh_k, pos, seq, head_dim, theta, s);
    case LLAISYS_DTYPE_F16: return launchAny<F16>(q_out, q_in, nh_q, k_out, k_in, nh_k, pos, seq, head_dim, theta, s);
    default: return;
    }
}

} // namespace llaisys::kernels
