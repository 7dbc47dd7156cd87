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
// Design: one launch covers the q, k and v head rows of the tokens in rope.hip's half-pair
// layout: each lane holds E whole rotation pairs (E elements of each half of a head row),
// so the rotation needs no cross-lane exchange and is the reference's two rounded f64
// products and their sum for q and k alike -- q equals llaisysROPE's output and k's codes
// are those of the reference's rope.  Each wave computes its token's f64 (cos, sin) pairs
// into its own LDS slice while the row loads are in flight; no block barrier.  A k or v
// row's absmax is reduced across its lanes with DPP / permlane butterflies, then each lane
// writes the E codes of each half it holds.
//
// Bound (MI355X, Qwen2 shapes, 2048 tokens, 15.8 MB): 4.58 us against 3.93 us for a copy
// kernel with the same traffic.  At 2048 tokens the launch has four waves per SIMD and
// every wave waits one HBM round trip before its VALU work (the f64 rotation, the f64
// sincos, the quantizer) and then its stores.
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

// Packed-magnitude maximum over one chunk (AbsBits's rule on 8 or 16 bytes).
template <typename T, typename V>
__device__ __forceinline__ uint32_t foldChunk(uint32_t m, const V &v) {
    constexpr int W = sizeof(V) / 4;
    if constexpr (std::is_same_v<T, F32>) {
#pragma unroll
        for (int w = 0; w < W; ++w) m = max(m, v[w] & 0x7FFFFFFFu);
    } else {
        v2u16 acc = __builtin_bit_cast(v2u16, m);
#pragma unroll
        for (int w = 0; w < W; ++w) acc = __builtin_elementwise_max(acc, __builtin_bit_cast(v2u16, v[w] & 0x7FFF7FFFu));
        m = __builtin_bit_cast(uint32_t, acc);
    }
    return m;
}

// Half-pair layout (rope.hip's ropeHalves): lane l of a group of RL = d / (2E) lanes holds
// elements E*l .. E*l + E-1 of both halves of a head row, i.e. E whole rotation pairs.  A
// wavefront takes one token's rows -- q rows, then k rows, then v rows, 64 / RL per row
// instruction -- in passes of IPT instructions, computes the token's (cos, sin) pairs (one
// per lane) into its own LDS slice while the loads are in flight, and keeps its lanes' E
// pairs in registers.  k and v rows: the row's absmax is a max over the RL lanes' packed
// magnitudes (DPP / permlane butterflies), then each lane writes the E codes of each half
// it holds.  An instruction whose rows are all q rows (wave-uniform) rotates and stores
// only.  Waves past the last token redo the last token and store nothing.
template <typename T, int IPT, int RL, bool kOnePass, int E>
__global__ void __launch_bounds__(256)
    ropeKvHalves(RopeKvArgs a, const int64_t *__restrict__ pos, size_t seq, int passes, int split_log2,
                 FreqTable ft) {
    using C = Chunk4<T, E>;
    using Vc = typename C::V;
    constexpr int kRows = kWave / RL;          // rows per wave instruction
    constexpr int kHalf = RL * E;              // elements per half row
    constexpr int kHalfBytes = kHalf * Fmt<T>::kBytes;
    constexpr int kRowBytes = 2 * kHalfBytes;
    constexpr int kRowCodes = 2 * kHalf;       // head_dim
    // (cos, sin) of angle j = E l + e sits in slot e * RL + l: lane l's read of its element e
    // and the lanes' writes (slot = lane) both touch consecutive 16-byte slots, free of LDS
    // bank conflicts (slots E * 16 bytes apart conflicted E-fold)
    __shared__ double2 cs[256 / kWave][kHalf];
    const auto angleOf = [](int slot) { return (slot % RL) * E + slot / RL; };

    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const uint32_t gw = blockIdx.x * (256 / kWave) + uint32_t(wave);
    const size_t t0 = gw >> split_log2;
    const int first_instr = int(gw & ((1u << split_log2) - 1)) * passes * IPT;
    const bool live = t0 < seq;
    const size_t t = live ? t0 : seq - 1;
    const int nq = a.nq, nk = a.nk, rows = nq + 2 * nk;
    const int rlane = lane / RL, l = lane % RL;
    const char *q_in = static_cast<const char *>(a.q_in) + t * size_t(nq) * kRowBytes + l * C::kBytes;
    const char *k_in = static_cast<const char *>(a.k_in) + t * size_t(nk) * kRowBytes + l * C::kBytes;
    const char *v_in = static_cast<const char *>(a.v_in) + t * size_t(nk) * kRowBytes + l * C::kBytes;
    char *q_out = static_cast<char *>(a.q_out) + t * size_t(nq) * kRowBytes + l * C::kBytes;
    int8_t *k_codes = a.k_codes + t * size_t(nk) * kRowCodes + l * E;
    int8_t *v_codes = a.v_codes + t * size_t(nk) * kRowCodes + l * E;
    float *k_scale = a.k_scale + t * size_t(nk), *v_scale = a.v_scale + t * size_t(nk);

    // the lane's first frequency before the row loads (vector loads complete in issue order)
    const double f_first = ft.f[angleOf(lane < kHalf ? lane : 0)];
    __builtin_amdgcn_sched_barrier(0);
    double c[E], sn[E];
    const int npass = kOnePass ? 1 : passes;
    for (int pass = 0; pass < npass; ++pass) {
        Vc xa[IPT], xb[IPT];
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int ins = first_instr + pass * IPT + k; // wave-uniform
            const int r = ins * kRows + rlane;
            const char *src;
            if ((ins + 1) * kRows <= nq) {
                src = q_in + size_t(r) * kRowBytes;
            } else {
                // rows past the token's last one read its first q row and store nothing
                src = r < nq ? q_in + size_t(r) * kRowBytes
                      : r < nq + nk ? k_in + size_t(r - nq) * kRowBytes
                      : r < rows ? v_in + size_t(r - nq - nk) * kRowBytes
                                 : q_in;
            }
            xa[k] = C::load(src);
            xb[k] = C::load(src + kHalfBytes);
        }
        if (pass == 0) {
            const int64_t p = pos[t];
            bool far = false;
            for (int sl = lane; sl < kHalf; sl += kWave) {
                const double ang = double(p) * (sl == lane ? f_first : ft.f[angleOf(sl)]);
                double s0 = 0.0, c0 = 0.0;
                if (fabs(ang) <= kSincosFastLimit)
                    sincosReduced(ang, &s0, &c0);
                else
                    far = true; // also NaN
                cs[wave][sl] = make_double2(c0, s0);
            }
            if (__builtin_expect(__any(far), 0)) {
                for (int sl = lane; sl < kHalf; sl += kWave) {
                    const double ang = double(p) * ft.f[angleOf(sl)];
                    if (!(fabs(ang) <= kSincosFastLimit)) {
                        double s0, c0;
                        librarySinCos(ang, &s0, &c0);
                        cs[wave][sl] = make_double2(c0, s0);
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int e = 0; e < E; ++e) {
                const double2 v = cs[wave][e * RL + l];
                c[e] = v.x;
                sn[e] = v.y;
            }
        }
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int ins = first_instr + pass * IPT + k; // wave-uniform
            const int r = ins * kRows + rlane;
            if ((ins + 1) * kRows <= nq) {
                // every row of this instruction is a q row: rotate and store
                if (!live) continue;
                float x0[E], x1[E], y0[E], y1[E];
                C::unpack(xa[k], x0);
                C::unpack(xb[k], x1);
#pragma unroll
                for (int e = 0; e < E; ++e) rotatePair(x0[e], x1[e], c[e], sn[e], y0[e], y1[e]);
                char *dst = q_out + size_t(r) * kRowBytes;
                C::store(dst, C::packQ(y0));
                C::store(dst + kHalfBytes, C::packQ(y1));
                continue;
            }
            const int kind = r < nq ? 0 : (r < nq + nk ? 1 : (r < rows ? 2 : 3)); // 3: none
            Vc o0 = xa[k], o1 = xb[k];
            if (kind <= 1) {
                float x0[E], x1[E], y0[E], y1[E];
                C::unpack(xa[k], x0);
                C::unpack(xb[k], x1);
#pragma unroll
                for (int e = 0; e < E; ++e) rotatePair(x0[e], x1[e], c[e], sn[e], y0[e], y1[e]);
                o0 = C::packQ(y0); // the element-type values llaisysROPE would store
                o1 = C::packQ(y1);
            }
            // k / v rows: the quantizer's input is the row's stored element values; amax as
            // in quant.hip (integer max of magnitude bits, the float rule for a row with a NaN)
            using A = AbsBits<T>;
            uint32_t bits = kind == 1 || kind == 2 ? A::finish(foldChunk<T>(foldChunk<T>(0u, o0), o1)) : 0u;
            bits = waveGroupReduce<RL, MaxU32Op>(bits);
            float v0[E], v1[E];
            C::unpack(o0, v0);
            C::unpack(o1, v1);
            float amax = A::value(bits);
            if (__builtin_expect(bits > A::kInf, 0)) { // uniform over the row's lanes
                amax = 0.0f;
#pragma unroll
                for (int e = 0; e < E; ++e) amax = MaxOp::apply(MaxOp::apply(amax, fabsf(v0[e])), fabsf(v1[e]));
                amax = waveGroupReduce<RL, MaxOp>(amax);
            }
            if (!live || kind == 3) continue;
            if (kind == 0) {
                char *dst = q_out + size_t(r) * kRowBytes;
                C::store(dst, o0);
                C::store(dst + kHalfBytes, o1);
            } else {
                const int hr = kind == 1 ? r - nq : r - nq - nk; // head row within k / v
                const RowQuantizer qz(amax);
                uint32_t cd0[E], cd1[E];
                qz.codes<E, std::is_same_v<T, F32>>(v0, cd0);
                qz.codes<E, std::is_same_v<T, F32>>(v1, cd1);
                int8_t *dst = (kind == 1 ? k_codes : v_codes) + size_t(hr) * kRowCodes;
                storeCodes<E>(dst, 0, cd0);
                storeCodes<E>(dst, kHalf, cd1);
                if (l == 0) (kind == 1 ? k_scale : v_scale)[hr] = qz.scale;
            }
        }
    }
}

template <typename T, int IPT, bool kOnePass, int E>
void launchKvHalvesRl(int rl, int passes, int split_log2, const RopeKvArgs &a, const int64_t *pos, size_t seq,
                      const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor(seq << split_log2, 256 / kWave);
    switch (rl) {
    case 1: ropeKvHalves<T, IPT, 1, kOnePass, E><<<grid, 256, 0, s>>>(a, pos, seq, passes, split_log2, ft); break;
    case 2: ropeKvHalves<T, IPT, 2, kOnePass, E><<<grid, 256, 0, s>>>(a, pos, seq, passes, split_log2, ft); break;
    case 4: ropeKvHalves<T, IPT, 4, kOnePass, E><<<grid, 256, 0, s>>>(a, pos, seq, passes, split_log2, ft); break;
    case 8: ropeKvHalves<T, IPT, 8, kOnePass, E><<<grid, 256, 0, s>>>(a, pos, seq, passes, split_log2, ft); break;
    case 16: ropeKvHalves<T, IPT, 16, kOnePass, E><<<grid, 256, 0, s>>>(a, pos, seq, passes, split_log2, ft); break;
    case 32: ropeKvHalves<T, IPT, 32, kOnePass, E><<<grid, 256, 0, s>>>(a, pos, seq, passes, split_log2, ft); break;
    default: break;
    }
}

template <typename T, int E>
void launchKvHalvesE(int rl, int instr, int split_log2, const RopeKvArgs &a, const int64_t *pos, size_t seq,
                     const FreqTable &ft, hipStream_t s) {
    const int per_wave = (instr + (1 << split_log2) - 1) >> split_log2;
    const int passes = (per_wave + 3) / 4, ipt = (per_wave + passes - 1) / passes;
    const auto go = [&](auto ipt_c) {
        constexpr int I = decltype(ipt_c)::value;
        if (passes == 1)
            launchKvHalvesRl<T, I, true, E>(rl, passes, split_log2, a, pos, seq, ft, s);
        else
            launchKvHalvesRl<T, I, false, E>(rl, passes, split_log2, a, pos, seq, ft, s);
    };
    switch (ipt) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    default: go(std::integral_constant<int, 4>{}); break;
    }
}

// The half-pair kernel when the shape fits it (head_dim / 2 <= 128, a power-of-two lane
// group of at most 32, chunk-aligned pointers); E = 8 for 16-bit types once the rows fill
// a row instruction, else E = 4; two waves per token from two row instructions on, each
// with half of them.  Measured on MI355X (bf16, graph-replayed medians over >= 1 GiB of
// rotating sets): the config-4 layer, 2048 tokens of Qwen2 q / k / v (2 instructions at
// E = 8), 4.58 us with 2 waves per token against 4.79 with 1, 4.68 at E = 4 with 1 and
// 4.83 for the previous layout (16-byte vectors, partner by DPP); a variant whose first
// wave per token computes the pairs for both, behind an LDS barrier, 5.09 us.  Llama-8B
// heads at 2048 tokens 10.65 us against 11.42 with 1 and 12.27 before; one decode token
// 2.34 against 2.80 and 2.89.
template <typename T>
bool launchKvHalves(const RopeKvArgs &a, const int64_t *pos, size_t seq, size_t half,
                    const FreqTable &ft, hipStream_t s) {
    constexpr bool k16 = Fmt<T>::kBytes == 2;
    const size_t rows = size_t(a.nq) + 2 * size_t(a.nk);
    if (half % 4 != 0 || half > size_t(kMaxHalf) || rows == 0 || seq >= (size_t(1) << 31)) return false;
    const auto fits = [&](size_t e) {
        const size_t rl = half / e;
        if (rl == 0 || rl > 32 || (rl & (rl - 1)) != 0) return false;
        const uintptr_t chunk = e * size_t(Fmt<T>::kBytes);
        for (const void *p : {static_cast<const void *>(a.q_out), a.q_in, a.k_in, a.v_in})
            if (reinterpret_cast<uintptr_t>(p) % chunk != 0) return false;
        return reinterpret_cast<uintptr_t>(a.k_codes) % e == 0 && reinterpret_cast<uintptr_t>(a.v_codes) % e == 0;
    };
    int e = 4;
    if (k16 && half % 8 == 0 && fits(8) && rows >= size_t(kWave) / (half / 8)) e = 8;
    if (e == 4 && !fits(4)) return false;
    const int rl = int(half / size_t(e)), rpi = kWave / rl;
    const int instr = int((rows + size_t(rpi) - 1) / size_t(rpi));
    const int split_log2 = instr >= 2 && seq < (size_t(1) << 30) ? 1 : 0;
    if (e == 8) {
        if constexpr (k16) launchKvHalvesE<T, 8>(rl, instr, split_log2, a, pos, seq, ft, s);
    } else {
        launchKvHalvesE<T, 4>(rl, instr, split_log2, a, pos, seq, ft, s);
    }
    return true;
}

template <typename T>
bool launchKv(const RopeKvArgs &a, const int64_t *pos, size_t seq, size_t d, float theta,
              hipStream_t s) {
    return launchKvHalves<T>(a, pos, seq, d / 2, hostFreqs(d, theta), s);
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
