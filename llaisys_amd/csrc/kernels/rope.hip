// Rotate-half RoPE for gfx950, for one tensor or for q and k in one launch.
//
// Semantics: reference src/ops/rope/cpu/rope_cpu.cpp:28-44.  For token i, head h and
// j < d/2: freq_j = 1 / pow((double)theta, (double)(2.0f * j / d)), angle = (double)p_i *
// freq_j, and the pair (x_j, x_{j+d/2}) is rotated in double precision; the result is
// rounded double -> float -> element type.  freq_j is computed on the host with the same
// libm pow the reference calls, so the angles are bit-identical; cos/sin come from
// sincos.hpp (within an ulp of glibc's, which the final float rounding absorbs).  The
// wave kernel of several instructions per token forms x*c +- p*s as one f64 product and
// one f64 fma (the reference rounds both products); the double results differ by at most
// an ulp, which the rounding to float absorbs except within 2^-29 of a float tie.  The
// one-instruction wave kernel (kExact) and ropeVec round both products as the reference.
//
// Design: HBM-bound, no MFMA (no contraction).  Two kernels:
//  * ropeWave (most shapes): 2^split_log2 wavefronts per token (each a contiguous share
//    of the token's head-row instructions), no block barrier.  A wave issues the 16-byte
//    loads of its rows, computes the token's d/2 (cos, sin) pairs (one per lane) into its
//    own LDS slice while they are in flight, and each lane then keeps the pairs of its
//    column in registers for every head row it rotates.
//  * ropeVec (at most 1/8 of a wave's lanes per token, e.g. one 64-wide head): a 256-thread block owns a run of tokens,
//    computes their pairs into LDS behind a block barrier and rotates items that read
//    their pairs from LDS; it packs several tokens into a block, so lanes stay busy.
// The trig is the ~40-instruction routine of sincos.hpp, the device library only on an
// out-of-line rare path.  Loads and stores are non-temporal (read once, written once).
// q and k of the same tokens go through one launch.
//
// Measured on MI355X (median of batched launches over >= 1 GiB of rotating sets): q+k of
// Qwen2 at 8192 tokens 12.1 us with 2 waves per token (13.2 with one, 13.5 with ropeVec);
// q alone 10.3 us; Llama-8B q+k at 16384 tokens 54.0 us with 4 waves per token (57.0
// with one).  A copy kernel moving the same bytes takes 10.4 us (q+k); the rest is the
// f64 rotation (two f32 -> f64 conversions, a multiply, an fma and the conversion back
// per element) issuing behind the loads.  Tried and slower: a persistent double-buffered
// block loop (18.7-25.8 us), 8 waves/SIMD by register cap (spills, 40 us).
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
// instruction into 8 half-rows 256 B apart and ran ~20 % slower).  A block's items are
// tensor-major: first the ntok * nv0 vectors of tensor 0 for its tokens (one contiguous
// range of that tensor), then tensor 1's; so an item's address is a per-block base
// (scalar registers) plus a 32-bit lane offset.  The rotation partner of a vector sits
// VPH lanes away and is fetched with a cross-lane exchange.  VPH (16-byte vectors per
// half head) is a power of two <= 32, so a row never straddles a wavefront; item ->
// token is a multiply by magic_t = floor(2^32 / nv_t) + 1, exact for item * nv_t < 2^32.
template <typename T, int IPT, int VPH>
__global__ void __launch_bounds__(256)
    ropeVec(RopePair tp, const int64_t *__restrict__ pos, size_t seq, int tok_per_block,
            uint32_t magic0, uint32_t magic1, FreqTable ft) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    constexpr int kRowVec = 2 * VPH; // vectors per head row
    constexpr int kHalf = VPH * N;
    __shared__ double2 cs[kLdsPairs];

    const int nv0 = tp.n_heads0 * kRowVec, nv1 = tp.n_heads1 * kRowVec;
    const size_t t0 = size_t(blockIdx.x) * tok_per_block;
    const int ntok = int(min(size_t(tok_per_block), seq - t0));
    const int items0 = ntok * nv0;
    const int items = items0 + ntok * nv1;
    const size_t blk0 = t0 * size_t(nv0) * 16, blk1 = t0 * size_t(nv1) * 16; // bytes
    const char *in0 = static_cast<const char *>(tp.in0) + blk0;
    const char *in1 = static_cast<const char *>(tp.in1) + blk1;
    char *out0 = static_cast<char *>(tp.out0) + blk0;
    char *out1 = static_cast<char *>(tp.out1) + blk1;

    const AngleInputs ang0 = firstAngle(pos, t0, ntok, kHalf, ft); // before the item loads

    // 1. issue this lane's loads (one contiguous 16-byte vector per item)
    v4u raw[IPT];
    uint32_t off[IPT];
    int tok[IPT];
    bool second[IPT];
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        const int it = threadIdx.x + k * 256;
        second[k] = it >= items0;
        const uint32_t rel = uint32_t(second[k] ? it - items0 : it);
        tok[k] = int(__umulhi(rel, second[k] ? magic1 : magic0));
        off[k] = rel * 16u;
        // unconditional load (idle lanes read the block's first vector), so the compiler can
        // count these loads as outstanding when the trig waits for its own inputs
        const char *src = it < items ? (second[k] ? in1 : in0) + off[k] : in0;
        raw[k] = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(src));
    }

    // 2. (cos, sin) of this block's tokens, while the loads are in flight
    blockCosSin(cs, ang0, pos, t0, ntok, kHalf, ft);

    // 3. exchange with the partner vector, rotate, store.  First half of a row:
    //    y = x*c + (-partner)*s; second half: y = x*c + partner*s -- the reference's
    //    a*c - b*s and b*c + a*s with the same roundings (rope_cpu.cpp:40-41); the
    //    partner's sign is flipped on its packed words, one XOR per 32 bits.
    const int v_lane = threadIdx.x & (kRowVec - 1);
    const bool upper = v_lane >= VPH;
    const int jv = v_lane & (VPH - 1);
    const uint32_t flip = upper ? 0u : F::kSignBits;
#pragma unroll
    for (int k = 0; k < IPT; ++k) {
        v4u other;
        other.x = partnerOf<VPH>(raw[k].x) ^ flip;
        other.y = partnerOf<VPH>(raw[k].y) ^ flip;
        other.z = partnerOf<VPH>(raw[k].z) ^ flip;
        other.w = partnerOf<VPH>(raw[k].w) ^ flip;
        const int it = threadIdx.x + k * 256;
        if (it < items) {
            float x[N], p[N], y[N];
            F::unpack(raw[k], x);
            F::unpack(other, p);
            const double2 *row = cs + tok[k] * kHalf + jv * N;
#pragma unroll
            for (int e = 0; e < N; ++e) {
                const double c = row[e].x, sn = row[e].y;
                y[e] = float(double(x[e]) * c + double(p[e]) * sn);
            }
            // packQ: the values are arithmetic on the inputs and the host frequencies,
            // which carry no foreign NaN payload (a NaN theta takes the scalar kernel)
            __builtin_nontemporal_store(F::packQ(y), reinterpret_cast<v4u *>((second[k] ? out1 : out0) + off[k]));
        }
    }
}

// One wavefront per token, no block barrier.  Each lane computes one (cos, sin) pair (two
// or more when d/2 > 64) of its token into the wave's own LDS slice, then reads
// back the N (cos, sin) pairs of its vector column into registers and uses them for every
// head row of the token: a row is kRowVec consecutive lanes, so a wave instruction covers
// 64 / kRowVec rows (q rows first, then k rows) and the lane's column is the same in all
// of them.  Rows are taken in passes of IPT wave instructions (kOnePass: one pass, laid
// out as straight-line code).  Waves past the last token
// redo the last token and store nothing, so no wave leaves before the loads (a branch
// there would serialise the kernel-argument loads ahead of the first global load).
template <typename T, int IPT, int VPH, bool kOnePass, bool kExact>
__global__ void __launch_bounds__(256)
    ropeWave(RopePair tp, const int64_t *__restrict__ pos, size_t seq, int passes, int split_log2,
             FreqTable ft) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    constexpr int kRowVec = 2 * VPH;          // lanes per head row
    constexpr int kRows = kWave / kRowVec;    // rows per wave instruction
    constexpr int kHalf = VPH * N;
    constexpr int kRowBytes = kRowVec * 16;
    // (cos, sin) of angle j = jv * N + e sits in slot e * VPH + jv, and lane l computes the
    // angle of slot l: both the write and every read instruction (same e, consecutive jv)
    // touch consecutive 16-byte slots, with no LDS bank conflicts (slots N * 16 bytes apart
    // had shown 4 % of the kernel's time in bank conflicts)
    __shared__ double2 cs[256 / kWave][kHalf];
    const auto angleOf = [](int slot) { return (slot % VPH) * N + slot / VPH; };

    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const uint32_t gw = blockIdx.x * (256 / kWave) + uint32_t(wave);
    const uint32_t t0 = gw >> split_log2;
    const int first_instr = int(gw & ((1u << split_log2) - 1)) * passes * IPT;
    const bool live = t0 < seq;                // waves past the end redo the last token
    const size_t t = live ? t0 : seq - 1;      // and store nothing
    const int nh0 = tp.n_heads0, rows = nh0 + tp.n_heads1;
    const int rlane = lane / kRowVec, v_lane = lane % kRowVec;
    const int jv = v_lane & (VPH - 1);
    const bool lower = v_lane < VPH;
    const char *in0 = static_cast<const char *>(tp.in0) + t * size_t(nh0) * kRowBytes + v_lane * 16;
    const char *in1 = static_cast<const char *>(tp.in1) + t * size_t(tp.n_heads1) * kRowBytes + v_lane * 16 -
                      size_t(nh0) * kRowBytes;
    char *out0 = static_cast<char *>(tp.out0) + t * size_t(nh0) * kRowBytes + v_lane * 16;
    char *out1 = static_cast<char *>(tp.out1) + t * size_t(tp.n_heads1) * kRowBytes + v_lane * 16 -
                 size_t(nh0) * kRowBytes;

    // the lane's first frequency before the row loads: the vector memory counter drains in
    // issue order, so a frequency read issued after them would hold the angle work until all
    // the rows had landed
    const double f_first = ft.f[angleOf(lane < kHalf ? lane : 0)];
    __builtin_amdgcn_sched_barrier(0);
    double c[N], sn[N];
    const int npass = kOnePass ? 1 : passes;
    for (int pass = 0; pass < npass; ++pass) {
        v4u raw[IPT];
#pragma unroll
        for (int k = 0; k < IPT; ++k) {
            const int r = (first_instr + pass * IPT + k) * kRows + rlane;
            const char *src = (r < nh0 ? in0 : (r < rows ? in1 : in0 - size_t(r) * kRowBytes)) + size_t(r) * kRowBytes;
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
            const int r = (first_instr + pass * IPT + k) * kRows + rlane;
            if (live && r < rows) {
                float x[N], q[N], y[N];
                F::unpack(raw[k], x);
                F::unpack(other, q);
                if constexpr (kExact) { // the reference's two rounded products and their sum
#pragma unroll
                    for (int e = 0; e < N; ++e) y[e] = float(double(x[e]) * c[e] + double(q[e]) * sn[e]);
                } else {
#pragma unroll
                    for (int e = 0; e < N; ++e) y[e] = float(fma(double(q[e]), sn[e], double(x[e]) * c[e]));
                }
                __builtin_nontemporal_store(F::packQ(y), reinterpret_cast<v4u *>((r < nh0 ? out0 : out1) + size_t(r) * kRowBytes));
            }
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
        angleSinCos(ang, &sn, &c);
        const size_t base = th * d;
        const double A = F::get(in, base + j), B = F::get(in, base + j + half);
        F::put(out, base + j, float(A * c - B * sn));
        F::put(out, base + j + half, float(B * c + A * sn));
    }
}

template <typename T, int IPT, bool kOnePass, bool kExact>
void launchWaveVph(int vph, int passes, int split_log2, const RopePair &tp, const int64_t *pos,
                   size_t seq, const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor(seq << split_log2, 256 / kWave);
    switch (vph) {
    case 2: ropeWave<T, IPT, 2, kOnePass, kExact><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    case 4: ropeWave<T, IPT, 4, kOnePass, kExact><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    case 8: ropeWave<T, IPT, 8, kOnePass, kExact><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    case 16: ropeWave<T, IPT, 16, kOnePass, kExact><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    case 32: ropeWave<T, IPT, 32, kOnePass, kExact><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    default: break;
    }
}

template <typename T, int IPT>
void launchWaveIpt(int vph, int passes, int split_log2, const RopePair &tp, const int64_t *pos,
                   size_t seq, const FreqTable &ft, hipStream_t s) {
    if (passes == 1)
        launchWaveVph<T, IPT, true, false>(vph, passes, split_log2, tp, pos, seq, ft, s);
    else
        launchWaveVph<T, IPT, false, false>(vph, passes, split_log2, tp, pos, seq, ft, s);
}

// `instr` wave instructions per token, taken in passes of at most 4 (registers).
template <typename T>
void launchWave(int vph, int instr, const RopePair &tp, const int64_t *pos, size_t seq,
                const FreqTable &ft, hipStream_t s) {
    // Waves per token: the fewest (a power of two, at least 2 from 3 instructions on) that
    // leave each wave <= 3 row instructions.  Measured on MI355X, 16-byte items: q+k of
    // Qwen2 at 8192 tokens (4 instructions) 12.1 us with 2 waves vs 13.2 with 1 and 13.3
    // with 4; q alone (3) 10.3 vs 11.1 with 1; Llama-8B q+k at 16384 tokens (10) 54.0 with
    // 4 vs 55.5 with 2 and 57.0 with 1.  More waves overlap one token's loads with
    // another's rotation; each repeats the token's (cos, sin) work.
    int split_log2 = instr >= 3 ? 1 : 0;
    while ((instr + (1 << split_log2) - 1) >> split_log2 > 3) ++split_log2;
    while (split_log2 > 0 && (seq << split_log2) >= (size_t(1) << 31)) --split_log2;
    const int split = 1 << split_log2;
    const int per_wave = (instr + split - 1) / split;
    const int passes = (per_wave + 3) / 4, ipt = (per_wave + passes - 1) / passes;
    switch (ipt) {
    case 1: launchWaveIpt<T, 1>(vph, passes, split_log2, tp, pos, seq, ft, s); break;
    case 2: launchWaveIpt<T, 2>(vph, passes, split_log2, tp, pos, seq, ft, s); break;
    case 3: launchWaveIpt<T, 3>(vph, passes, split_log2, tp, pos, seq, ft, s); break;
    default: launchWaveIpt<T, 4>(vph, passes, split_log2, tp, pos, seq, ft, s); break;
    }
}

template <typename T, int IPT>
void launchIpt(int vph, const RopePair &tp, const int64_t *pos, size_t seq, size_t tpb,
               uint32_t magic0, uint32_t magic1, const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor(seq, tpb);
    switch (vph) {
    case 2: ropeVec<T, IPT, 2><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic0, magic1, ft); break;
    case 4: ropeVec<T, IPT, 4><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic0, magic1, ft); break;
    case 8: ropeVec<T, IPT, 8><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic0, magic1, ft); break;
    case 16: ropeVec<T, IPT, 16><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic0, magic1, ft); break;
    case 32: ropeVec<T, IPT, 32><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic0, magic1, ft); break;
    default: break;
    }
}

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
    const size_t tpb = tokensPerBlock(per_tok, half, 256 * kMaxItems);
    const int ipt = int((tpb * per_tok + 255) / 256);
    const auto magicOf = [&](int heads) {
        return heads ? uint32_t((uint64_t(1) << 32) / (size_t(heads) * 2 * vph) + 1) : 0u;
    };
    const uint32_t magic0 = magicOf(tp.n_heads0), magic1 = magicOf(tp.n_heads1);
    // One wave per token when its instructions keep >= 3/4 of the lanes busy (q+k of Qwen2:
    // 14 of 16 rows, q alone and Llama-8B q+k: all).  One token of one instruction with at
    // least 1/4 of the lanes busy (k alone) also takes one wave, with the reference's two
    // rounded products (the exact form of ropeVec); measured on MI355X, bf16, 8192 tokens:
    // k [2 heads, 128] 6.02 -> 4.56 us, [1, 128] 4.68 -> 4.39 us, [2, 64] 5.20 -> 4.89 us,
    // [4, 64] 4.96 -> 4.91 us; at 1/8 ([1, 64]) ropeVec's packed tokens win, 3.96 against
    // 5.06 us.  Fewer rows per token pack several tokens per block with ropeVec.
    const int rpi = int(kWave / (2 * vph));
    const size_t rows = size_t(tp.n_heads0 + tp.n_heads1);
    const int instr = int((rows + rpi - 1) / rpi);
    if (rows * 4 >= size_t(instr) * rpi * 3) {
        launchWave<T>(int(vph), instr, tp, pos, seq, ft, s);
        return true;
    }
    if (instr == 1 && rows * 4 >= size_t(rpi)) {
        launchWaveVph<T, 1, true, true>(int(vph), 1, 0, tp, pos, seq, ft, s);
        return true;
    }
    switch (ipt) {
    case 1: launchIpt<T, 1>(int(vph), tp, pos, seq, tpb, magic0, magic1, ft, s); break;
    case 2: launchIpt<T, 2>(int(vph), tp, pos, seq, tpb, magic0, magic1, ft, s); break;
    case 3: launchIpt<T, 3>(int(vph), tp, pos, seq, tpb, magic0, magic1, ft, s); break;
    default: launchIpt<T, 4>(int(vph), tp, pos, seq, tpb, magic0, magic1, ft, s); break;
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
    // A NaN theta gives NaN frequencies carrying its payload, which the vector kernel's
    // packQ would not round like the reference; the scalar kernel rounds exactly.
    if (!std::isnan(theta) && launchVec<T>(tp, pos, seq, d, ft, s)) return;
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
