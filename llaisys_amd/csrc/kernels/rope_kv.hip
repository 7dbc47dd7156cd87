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
// Design: one launch covers the q, k and v head rows of the tokens; one wavefront per token
// (rope.hip's ropeWave layout: a head row on 2*VPH consecutive lanes, 16 bytes each, so
// every wave instruction moves 1 KB of contiguous rows).  The wave computes its token's
// f64 (cos, sin) pairs into its own LDS slice while the row loads are in flight; no block
// barrier.  A k or v row's absmax is reduced across its lanes with DPP, then each lane
// writes its 8 (bf16 / f16) or 4 (f32) codes, so the group stores the whole code row
// contiguously.
//
// Bound (MI355X, Qwen2 shapes, 2048 tokens, 15.8 MB): 5.06 us against 3.92 us for a copy
// kernel with the same traffic.  At 2048 tokens the launch has two waves per SIMD, and
// the VALU issue of the exact f64 rotation (two f32 -> f64 conversions, two products, a
// sum and the conversion back per element, which the bit-exact k codes need), the f64
// sincos and the quantizer is only partly hidden behind the loads: rocprofv3 counted 600
// VALU instructions per token-wave before the pure-q fast path and the one-pass layout
// (5.43 -> 5.06 us).  Tried and slower: 2 or 4 waves per token (5.73 / 6.30 us; each
// wave repeats the token's sincos), a block-per-2-tokens layout with block-wide
// (cos, sin) staging (5.3-5.45 us).
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

// One wavefront per token (the layout of rope.hip's ropeWave): the token's head rows --
// q rows, then k rows, then v rows, kRowVec lanes each -- are taken in passes of IPT wave
// instructions.  Each lane computes one (cos, sin) pair of the token into the wave's own
// LDS slice (no block barrier) while the row loads are in flight, then keeps its column's
// pairs in registers.  Waves past the last token redo the last token and store nothing.
// An instruction whose rows are all q rows (wave-uniform) takes a rotate-and-store path
// with no quantizer work; kOnePass (all rows in one pass, e.g. Qwen2's 16 rows) lets the
// compiler lay the whole token out as straight-line code.
template <typename T, int IPT, int VPH, bool kOnePass>
__global__ void __launch_bounds__(256)
    ropeKvWave(RopeKvArgs a, const int64_t *__restrict__ pos, size_t seq, int passes, FreqTable ft) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    constexpr int kRowVec = 2 * VPH;       // lanes per head row
    constexpr int kRows = kWave / kRowVec; // rows per wave instruction
    constexpr int kHalf = VPH * N;
    constexpr int kRowBytes = kRowVec * 16;
    constexpr int kRowCodes = kRowVec * N; // head_dim
    __shared__ double2 cs[256 / kWave][kHalf];
    const auto angleOf = [](int slot) { return (slot % VPH) * N + slot / VPH; };

    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const size_t t0 = size_t(blockIdx.x) * (256 / kWave) + size_t(wave);
    const bool live = t0 < seq;
    const size_t t = live ? t0 : seq - 1;
    const int nq = a.nq, nk = a.nk, rows = nq + 2 * nk;
    const int rlane = lane / kRowVec, v_lane = lane % kRowVec;
    const int jv = v_lane & (VPH - 1);
    const bool lower = v_lane < VPH;
    const char *q_in = static_cast<const char *>(a.q_in) + t * size_t(nq) * kRowBytes + v_lane * 16;
    const char *k_in = static_cast<const char *>(a.k_in) + t * size_t(nk) * kRowBytes + v_lane * 16;
    const char *v_in = static_cast<const char *>(a.v_in) + t * size_t(nk) * kRowBytes + v_lane * 16;
    char *q_out = static_cast<char *>(a.q_out) + t * size_t(nq) * kRowBytes + v_lane * 16;
    int8_t *k_codes = a.k_codes + t * size_t(nk) * kRowCodes + v_lane * N;
    int8_t *v_codes = a.v_codes + t * size_t(nk) * kRowCodes + v_lane * N;
    float *k_scale = a.k_scale + t * size_t(nk), *v_scale = a.v_scale + t * size_t(nk);

    // the first frequency before the row loads (vector loads complete in issue order)
    const double f_first = ft.f[angleOf(lane < kHalf ? lane : 0)];
    __builtin_amdgcn_sched_barrier(0);
    double c[N], sn[N];
    const int npass = kOnePass ? 1 : passes;
    for (int pass = 0; pass < npass; ++pass) {
        v4u raw[IPT];
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int ins = pass * IPT + k; // wave-uniform
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
            raw[k] = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(src));
        }
        if (pass == 0) {
            const int64_t p = pos[t];
            bool far = false;
            for (int sl = lane; sl < kHalf; sl += kWave) {
                const int j = angleOf(sl);
                const double ang = double(p) * (sl == lane ? f_first : ft.f[j]);
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
            for (int e = 0; e < N; ++e) {
                const double2 v = cs[wave][e * VPH + jv];
                c[e] = v.x;
                sn[e] = lower ? -v.y : v.y; // first half: x*c - partner*s
            }
        }
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            v4u other;
            other.x = partnerOf<VPH>(raw[k].x);
            other.y = partnerOf<VPH>(raw[k].y);
            other.z = partnerOf<VPH>(raw[k].z);
            other.w = partnerOf<VPH>(raw[k].w);
            const int ins = pass * IPT + k; // wave-uniform
            const int r = ins * kRows + rlane;
            if ((ins + 1) * kRows <= nq) {
                // every row of this instruction is a q row: rotation and store only, in
                // ropeWave's form (rope.hip), so q equals llaisysROPE's
                if (!live) continue;
                float x[N], q[N], y[N];
                F::unpack(raw[k], x);
                F::unpack(other, q);
#pragma unroll
                for (int e = 0; e < N; ++e) y[e] = float(fma(double(q[e]), sn[e], double(x[e]) * c[e]));
                __builtin_nontemporal_store(F::packQ(y), reinterpret_cast<v4u *>(q_out + size_t(r) * kRowBytes));
                continue;
            }
            const int kind = r < nq ? 0 : (r < nq + nk ? 1 : (r < rows ? 2 : 3)); // 3: none
            v4u out = raw[k];
            if (kind <= 1) {
                float x[N], q[N], y[N];
                F::unpack(raw[k], x);
                F::unpack(other, q);
#pragma unroll
                // the reference's two rounded f64 products and their rounded sum
                // (rope_cpu.cpp:40-41), so k's codes are those of the reference's rope
                for (int e = 0; e < N; ++e) y[e] = float(double(x[e]) * c[e] + double(q[e]) * sn[e]);
                out = F::packQ(y); // the element-type value llaisysROPE would store
            }
            // k / v rows: quantizer input is the stored element values of the row; amax as
            // in quant.hip (integer max of magnitude bits, float rule for a row with a NaN)
            using A = AbsBits<T>;
            uint32_t bits = kind == 1 || kind == 2 ? A::finish(A::fold(0u, out)) : 0u;
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
            if (!live || kind == 3) continue;
            if (kind == 0) {
                __builtin_nontemporal_store(out, reinterpret_cast<v4u *>(q_out + size_t(r) * kRowBytes));
            } else {
                const int hr = kind == 1 ? r - nq : r - nq - nk; // head row within k / v
                const RowQuantizer qz(amax);
                uint32_t cd[N];
                qz.codes<N, std::is_same_v<T, F32>>(val, cd);
                storeCodes<N>(kind == 1 ? k_codes : v_codes, size_t(hr) * kRowCodes, cd);
                if (v_lane == 0) (kind == 1 ? k_scale : v_scale)[hr] = qz.scale;
            }
        }
    }
}

template <typename T, int IPT, bool kOnePass>
void launchKvWaveIpt(int vph, int passes, const RopeKvArgs &a, const int64_t *pos, size_t seq,
                     const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor(seq, 256 / kWave);
    switch (vph) {
    case 2: ropeKvWave<T, IPT, 2, kOnePass><<<grid, 256, 0, s>>>(a, pos, seq, passes, ft); break;
    case 4: ropeKvWave<T, IPT, 4, kOnePass><<<grid, 256, 0, s>>>(a, pos, seq, passes, ft); break;
    case 8: ropeKvWave<T, IPT, 8, kOnePass><<<grid, 256, 0, s>>>(a, pos, seq, passes, ft); break;
    case 16: ropeKvWave<T, IPT, 16, kOnePass><<<grid, 256, 0, s>>>(a, pos, seq, passes, ft); break;
    case 32: ropeKvWave<T, IPT, 32, kOnePass><<<grid, 256, 0, s>>>(a, pos, seq, passes, ft); break;
    default: break;
    }
}

template <typename T>
void launchKvWave(int vph, const RopeKvArgs &a, const int64_t *pos, size_t seq, const FreqTable &ft,
                  hipStream_t s) {
    const int rows_per_instr = kWave / (2 * vph);
    const int instr = (a.nq + 2 * a.nk + rows_per_instr - 1) / rows_per_instr;
    const int passes = (instr + 3) / 4, ipt = (instr + passes - 1) / passes;
    if (passes == 1) {
        switch (ipt) {
        case 1: launchKvWaveIpt<T, 1, true>(vph, passes, a, pos, seq, ft, s); break;
        case 2: launchKvWaveIpt<T, 2, true>(vph, passes, a, pos, seq, ft, s); break;
        case 3: launchKvWaveIpt<T, 3, true>(vph, passes, a, pos, seq, ft, s); break;
        default: launchKvWaveIpt<T, 4, true>(vph, passes, a, pos, seq, ft, s); break;
        }
        return;
    }
    switch (ipt) {
    case 1: launchKvWaveIpt<T, 1, false>(vph, passes, a, pos, seq, ft, s); break;
    case 2: launchKvWaveIpt<T, 2, false>(vph, passes, a, pos, seq, ft, s); break;
    case 3: launchKvWaveIpt<T, 3, false>(vph, passes, a, pos, seq, ft, s); break;
    default: launchKvWaveIpt<T, 4, false>(vph, passes, a, pos, seq, ft, s); break;
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
    if (a.nq + 2 * a.nk == 0) return false;
    launchKvWave<T>(int(vph), a, pos, seq, hostFreqs(d, theta), s);
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
