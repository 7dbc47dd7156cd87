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
#include <cmath>
#include <type_traits>

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

// Items of a block are tensor-major, as in rope.hip: the block's q vectors (one contiguous
// range of q), then its k vectors, then its v vectors; an item's addresses are per-block
// bases plus 32-bit lane offsets, and item -> token a multiply by the tensor's magic.
template <typename T, int IPT, int VPH>
__global__ void __launch_bounds__(256)
    ropeKvVec(RopeKvArgs a, const int64_t *__restrict__ pos, size_t seq, int tok_per_block,
              uint32_t magic_q, uint32_t magic_kv, FreqTable ft) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    constexpr int kRowVec = 2 * VPH;
    constexpr int kHalf = VPH * N;
    constexpr int kShift = __builtin_ctz(kRowVec);
    __shared__ double2 cs[kLdsPairs];

    const int nqv = a.nq * kRowVec, nkv = a.nk * kRowVec; // vectors per token
    const size_t t0 = size_t(blockIdx.x) * tok_per_block;
    const int ntok = int(min(size_t(tok_per_block), seq - t0));
    const int end_q = ntok * nqv, end_k = end_q + ntok * nkv, items = end_k + ntok * nkv;
    const int v_lane = threadIdx.x & (kRowVec - 1);
    const size_t vq0 = t0 * size_t(nqv), vkv0 = t0 * size_t(nkv); // first vector of the block
    const char *q_in = static_cast<const char *>(a.q_in) + vq0 * 16;
    const char *k_in = static_cast<const char *>(a.k_in) + vkv0 * 16;
    const char *v_in = static_cast<const char *>(a.v_in) + vkv0 * 16;
    char *q_out = static_cast<char *>(a.q_out) + vq0 * 16;
    int8_t *k_codes = a.k_codes + vkv0 * N, *v_codes = a.v_codes + vkv0 * N;
    float *k_scale = a.k_scale + vkv0 / kRowVec, *v_scale = a.v_scale + vkv0 / kRowVec;

    const AngleInputs ang0 = firstAngle(pos, t0, ntok, kHalf, ft); // before the item loads

    // 1. issue this lane's loads (unconditional: idle lanes read the block's first q vector,
    //    so the trig below can wait for its own inputs only)
    v4u raw[IPT];
    uint32_t rel[IPT]; // vector index within the block's range of its tensor
    int tok[IPT], kind[IPT]; // kind: 0 = q, 1 = k, 2 = v
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = threadIdx.x + k * 256;
        kind[k] = it < end_q ? 0 : (it < end_k ? 1 : 2);
        rel[k] = uint32_t(kind[k] == 0 ? it : (kind[k] == 1 ? it - end_q : it - end_k));
        tok[k] = int(__umulhi(rel[k], kind[k] == 0 ? magic_q : magic_kv));
        const char *src = it < items ? (kind[k] == 0 ? q_in : (kind[k] == 1 ? k_in : v_in)) + rel[k] * 16u : q_in;
        raw[k] = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(src));
    }

    // 2. (cos, sin) of this block's tokens, while the loads are in flight
    blockCosSin(cs, ang0, pos, t0, ntok, kHalf, ft);

    // 3. rotate (q, k), quantize (k, v), store
    const bool upper = v_lane >= VPH;
    const int jv = v_lane & (VPH - 1);
    const uint32_t flip = upper ? 0u : F::kSignBits; // first half: x*c + (-partner)*s
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        v4u other;
        other.x = partnerOf<VPH>(raw[k].x) ^ flip;
        other.y = partnerOf<VPH>(raw[k].y) ^ flip;
        other.z = partnerOf<VPH>(raw[k].z) ^ flip;
        other.w = partnerOf<VPH>(raw[k].w) ^ flip;
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
                y[e] = float(double(x[e]) * c + double(p[e]) * sn);
            }
            out = F::packQ(y); // the element-type value llaisysROPE would store
        }
        // quantizer input: the stored element values of the k / v row; amax as in
        // quant.hip (integer max of magnitude bits, float rule for a row with a NaN)
        using A = AbsBits<T>;
        uint32_t bits = active && kind[k] != 0 ? A::finish(A::fold(0u, out)) : 0u;
        bits = waveGroupReduce<kRowVec, MaxU32Op>(bits);
        float val[N];
        F::unpack(out, val);
        float amax = A::value(bits);
        if (__builtin_expect(bits > A::kInf, 0)) { // uniform over the row's lanes
            amax = 0.0f;
#pragma unroll
            for (int e = 0; e < N; ++e) amax = MaxOp::apply(amax, fabsf(val[e]));
#pragma unroll
            for (int m = kRowVec / 2; m > 0; m >>= 1) amax = MaxOp::apply(amax, __shfl_xor(amax, m, kWave));
        }
        if (!active) continue;
        if (kind[k] == 0) {
            __builtin_nontemporal_store(out, reinterpret_cast<v4u *>(q_out + rel[k] * 16u));
        } else {
            const RowQuantizer qz(amax);
            uint32_t c[N];
            qz.codes<N, std::is_same_v<T, F32>>(val, c);
            storeCodes<N>(kind[k] == 1 ? k_codes : v_codes, size_t(rel[k]) * N, c);
            if (v_lane == 0) (kind[k] == 1 ? k_scale : v_scale)[rel[k] >> kShift] = qz.scale;
        }
    }
}

template <typename T, int IPT>
void launchKvIpt(int vph, const RopeKvArgs &a, const int64_t *pos, size_t seq, size_t tpb,
                 uint32_t magic_q, uint32_t magic_kv, const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor(seq, tpb);
    switch (vph) {
    case 2: ropeKvVec<T, IPT, 2><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic_q, magic_kv, ft); break;
    case 4: ropeKvVec<T, IPT, 4><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic_q, magic_kv, ft); break;
    case 8: ropeKvVec<T, IPT, 8><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic_q, magic_kv, ft); break;
    case 16: ropeKvVec<T, IPT, 16><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic_q, magic_kv, ft); break;
    case 32: ropeKvVec<T, IPT, 32><<<grid, 256, 0, s>>>(a, pos, seq, int(tpb), magic_q, magic_kv, ft); break;
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
    const size_t tpb = tokensPerBlock(per_tok, half, 256 * kMaxItemsKv);
    const int ipt = int((tpb * per_tok + 255) / 256);
    const auto magicOf = [&](int heads) {
        return heads ? uint32_t((uint64_t(1) << 32) / (size_t(heads) * 2 * vph) + 1) : 0u;
    };
    const uint32_t magic_q = magicOf(a.nq), magic_kv = magicOf(a.nk);
    const FreqTable ft = hostFreqs(d, theta);
    switch (ipt) {
    case 1: launchKvIpt<T, 1>(int(vph), a, pos, seq, tpb, magic_q, magic_kv, ft, s); break;
    case 2: launchKvIpt<T, 2>(int(vph), a, pos, seq, tpb, magic_q, magic_kv, ft, s); break;
    case 3: launchKvIpt<T, 3>(int(vph), a, pos, seq, tpb, magic_q, magic_kv, ft, s); break;
    default: launchKvIpt<T, 4>(int(vph), a, pos, seq, tpb, magic_q, magic_kv, ft, s); break;
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
    if (nh_q > 65536 || nh_kv > 65536 || std::isnan(theta)) return false; // packQ needs a real theta
    const RopeKvArgs a{q_out, q_in, k_in, v_in, k_codes, k_scale, v_codes, v_scale, int(nh_q), int(nh_kv)};
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launchKv<F32>(a, pos, seq, head_dim, theta, s);
    case LLAISYS_DTYPE_BF16: return launchKv<BF16>(a, pos, seq, head_dim, theta, s);
    case LLAISYS_DTYPE_F16: return launchKv<F16>(a, pos, seq, head_dim, theta, s);
    default: return false;
    }
}

} // namespace llaisys::kernels
