// Fused RoPE + INT8 KV-cache append (quantize-on-append) for gfx950.
//
// Semantics: exactly the composition the reference decoder performs per layer, with the
// cache made INT8 (src/models/qwen2/attention.hpp:54-59 and :108-123):
//   q_out = rope(q);  k_cache[pos..] = quantize(rope(k));  v_cache[pos..] = quantize(v)
// where rope is src/ops/rope/cpu/rope_cpu.cpp:28-44 (its result rounded to the element
// type, as llaisysROPE stores it) and quantize is the per-(token, head) rule of
// quantize.hpp.  The codes therefore equal llaisysROPE followed by llaisysKVAppendInt8 bit
// for bit; the rope'd k never goes to HBM in bf16.
//
// Design: one launch covers the q, k and v head rows of a run of tokens (Qwen2-1.5B: 12 +
// 2 + 2 rows of 16 vectors = 256 items per token, one per lane).  Lane layout and the f64
// (cos, sin) staging are those of rope.hip.  A k or v row sits on 2*VPH consecutive lanes;
// its absmax is reduced across them with xor shuffles, then each lane writes its 8 (bf16 /
// f16) or 4 (f32) codes, so the group stores the whole code row contiguously.
#include "common.hpp"
#include "launch.hpp"
#include "quantize.hpp"
#include "rope_common.hpp"
#include "rowplan.hpp"

#include <algorithm>

namespace llaisys::kernels {

namespace {

using namespace rope_detail;

constexpr int kMaxItemsKv = 4;

struct RopeKvArgs {
    void *q_out;
    const void *q_in;
    const void *k_in;
    const void *v_in;
    int8_t *k_codes; // cache row `pos` already applied
    float *k_scale;
    int8_t *v_codes;
    float *v_scale;
    int nq;
    int nk; // k and v heads
};

template <typename T, int IPT, int VPH>
__global__ void __launch_bounds__(256)
    ropeKvVec(RopeKvArgs a, const int64_t *__restrict__ pos, size_t seq, int tok_per_block,
              uint32_t tok_magic, FreqTable ft) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    constexpr int kRowVec = 2 * VPH;
    constexpr int kHalf = VPH * N;
    constexpr int kD = 2 * kHalf;
    constexpr int kShift = __builtin_ctz(kRowVec);
    __shared__ double2 cs[kLdsPairs];

    const int per_tok = (a.nq + 2 * a.nk) * kRowVec;
    const size_t t0 = size_t(blockIdx.x) * tok_per_block;
    const int ntok = int(min(size_t(tok_per_block), seq - t0));
    const int items = ntok * per_tok;
    const int v_lane = threadIdx.x & (kRowVec - 1);

    // 1. issue this lane's loads
    v4u raw[IPT];
    size_t row_of[IPT]; // (token, head) row within its tensor
    int tok[IPT], kind[IPT]; // kind: 0 = q, 1 = k, 2 = v
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = threadIdx.x + k * 256;
        raw[k] = v4u{0, 0, 0, 0};
        kind[k] = 0;
        if (it < items) {
            const int tt = int(__umulhi(uint32_t(it), tok_magic));
            const int h = (it - tt * per_tok) >> kShift;
            kind[k] = h < a.nq ? 0 : (h < a.nq + a.nk ? 1 : 2);
            const int hh = kind[k] == 0 ? h : (kind[k] == 1 ? h - a.nq : h - a.nq - a.nk);
            const int nh = kind[k] == 0 ? a.nq : a.nk;
            tok[k] = tt;
            row_of[k] = (t0 + tt) * size_t(nh) + hh;
            const void *src = kind[k] == 0 ? a.q_in : (kind[k] == 1 ? a.k_in : a.v_in);
            raw[k] = load16Stream<T>(src, row_of[k] * kD + size_t(v_lane) * N);
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

    // 3. rotate (q, k), quantize (k, v), store
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
        const bool active = it < items;
        v4u out = raw[k];
        if (active && kind[k] != 2) {
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
            out = F::pack(y); // the element-type value llaisysROPE would store
        }
        // quantizer input: the stored element values of the k / v row
        float val[N];
        F::unpack(out, val);
        float amax = 0.0f;
        if (active && kind[k] != 0) {
#pragma unroll
            for (int e = 0; e < N; ++e) amax = MaxOp::apply(amax, fabsf(val[e]));
        }
#pragma unroll
        for (int m = kRowVec / 2; m > 0; m >>= 1) amax = MaxOp::apply(amax, __shfl_xor(amax, m, kWave));
        if (!active) continue;
        if (kind[k] == 0) {
            store16Stream<T>(a.q_out, row_of[k] * kD + size_t(v_lane) * N, out);
        } else {
            const RowQuantizer qz(amax);
            uint32_t c[N];
            qz.codes<N>(val, c);
            int8_t *codes = kind[k] == 1 ? a.k_codes : a.v_codes;
            storeCodes<N>(codes, row_of[k] * kD + size_t(v_lane) * N, c);
            if (v_lane == 0) (kind[k] == 1 ? a.k_scale : a.v_scale)[row_of[k]] = qz.scale;
        }
    }
}

template <typename T, int IPT>
void launchKvIpt(int vph, const RopeKvArgs &a, const int64_t *pos, size_t seq, size_t tpb,
                 uint32_t magic, const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor(seq, tpb);
    switch (vph) {
    case 2: ropeKvVec<T, IPT, 2><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic, ft); break;
    case 4: ropeKvVec<T, IPT, 4><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic, ft); break;
    case 8: ropeKvVec<T, IPT, 8><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic, ft); break;
    case 16: ropeKvVec<T, IPT, 16><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic, ft); break;
    case 32: ropeKvVec<T, IPT, 32><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic, ft); break;
    default: break;
    }
}

template <typename T>
bool launchKv(const RopeKvArgs &a, const int64_t *pos, size_t seq, size_t d, float theta,
              hipStream_t s) {
    constexpr int N = Fmt<T>::kVec;
    const size_t half = d / 2;
    if (half % N != 0 || half > size_t(kMaxHalf)) return false;
    const size_t vph = half / N;
    if ((vph & (vph - 1)) || vph > 32) return false;
    for (const void *p : {static_cast<const void *>(a.q_out), a.q_in, a.k_in, a.v_in})
        if (!aligned16(p)) return false;
    if (reinterpret_cast<uintptr_t>(a.k_codes) % N || reinterpret_cast<uintptr_t>(a.v_codes) % N)
        return false;
    const size_t per_tok = (size_t(a.nq) + 2 * size_t(a.nk)) * 2 * vph;
    if (per_tok == 0 || per_tok > size_t(256 * kMaxItemsKv)) return false;
    // tokens per block: fewest that keep >= 90 % of the lanes busy, else ~256 items
    size_t tpb = std::max<size_t>(1, 256 / per_tok);
    for (size_t t = 1; t * per_tok <= size_t(256 * kMaxItemsKv); ++t) {
        const size_t slots = (t * per_tok + 255) / 256 * 256;
        if (t * per_tok * 10 >= slots * 9) {
            tpb = t;
            break;
        }
    }
    tpb = std::min(tpb, size_t(kLdsPairs) / half);
    const int ipt = int((tpb * per_tok + 255) / 256);
    const uint32_t magic = uint32_t((uint64_t(1) << 32) / per_tok + 1);
    const FreqTable ft = hostFreqs(d, theta);
    switch (ipt) {
    case 1: launchKvIpt<T, 1>(int(vph), a, pos, seq, tpb, magic, ft, s); break;
    case 2: launchKvIpt<T, 2>(int(vph), a, pos, seq, tpb, magic, ft, s); break;
    case 3: launchKvIpt<T, 3>(int(vph), a, pos, seq, tpb, magic, ft, s); break;
    default: launchKvIpt<T, 4>(int(vph), a, pos, seq, tpb, magic, ft, s); break;
    }
    return true;
}

} // namespace

size_t ropeKvAppendWorkspaceBytes(size_t seq, size_t nh_kv, size_t head_dim, llaisysDataType_t dt) {
    const size_t es = dt == LLAISYS_DTYPE_F32 ? 4 : 2;
    return (seq * nh_kv * head_dim * es + 255) / 256 * 256;
}

bool ropeKvAppendFused(void *q_out, const void *q_in, size_t nh_q, const void *k_in,
                       const void *v_in, size_t nh_kv, int8_t *k_codes, float *k_scale,
                       int8_t *v_codes, float *v_scale, const int64_t *pos, size_t seq,
                       size_t head_dim, float theta, llaisysDataType_t dt, hipStream_t s) {
    if (seq == 0) return true;
    if (nh_q > 65536 || nh_kv > 65536) return false;
    const RopeKvArgs a{q_out, q_in, k_in, v_in, k_codes, k_scale, v_codes, v_scale, int(nh_q), int(nh_kv)};
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launchKv<F32>(a, pos, seq, head_dim, theta, s);
    case LLAISYS_DTYPE_BF16: return launchKv<BF16>(a, pos, seq, head_dim, theta, s);
    case LLAISYS_DTYPE_F16: return launchKv<F16>(a, pos, seq, head_dim, theta, s);
    default: return false;
    }
}

} // namespace llaisys::kernels
