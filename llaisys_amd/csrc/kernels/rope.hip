// Rotate-half RoPE for gfx950, for one tensor or for q and k in one launch.
//
// Semantics: reference src/ops/rope/cpu/rope_cpu.cpp:28-44.  For token i, head h and
// j < d/2: freq_j = 1 / pow((double)theta, (double)(2.0f * j / d)), angle = (double)p_i *
// freq_j, and the pair (a, b) = (x_j, x_{j+d/2}) becomes (a*c - b*s, b*c + a*s) with both
// products rounded in f64, then their sum, then the rounding double -> float -> element
// type, in every kernel below.  freq_j is computed on the host with the same libm pow the
// reference calls, so the angles are bit-identical; cos/sin come from sincos.hpp (within
// an ulp of glibc's, which the final float rounding absorbs).
//
// Design: HBM-bound, no MFMA (no contraction).  The kernels:
//  * ropeHalves (most shapes): each lane holds E consecutive elements of the first half
//    of a head row and the same E of the second half -- whole rotation pairs, so no lane
//    needs another lane's values.  A wave takes a contiguous share of one token's head
//    rows (or four tokens' rows), computes the tokens' d/2 (cos, sin) pairs (one per lane)
//    into its own LDS slice while its loads are in flight, and keeps its lanes' E pairs in
//    registers; every load lands before the first store.
//  * ropeFlat (one tensor of 9-15 heads, e.g. Qwen2 q alone): the same, with four tokens'
//    rows taken as one flat run so that no row slot of an instruction idles.
//  * ropeHalvesPacked (one tensor filling 1/2 or 1/4 of a row instruction, e.g. k alone):
//    several tokens per row instruction.
//  * ropeVec (under a quarter of a wave's lanes per token, e.g. one 64-wide head): a
//    256-thread block packs a run of tokens, computes their pairs into LDS behind a block
//    barrier and rotates 16-byte items that fetch their partner with a cross-lane move.
//  * ropeScalar: any other head_dim or alignment.
// The trig is the ~40-instruction routine of sincos.hpp, the device library only on an
// out-of-line rare path.  Loads and stores are non-temporal (read once, written once).
//
// Measured on MI355X (bf16, medians of graph-replayed launches over >= 1 GiB of rotating
// sets, one box) when the half-pair layout replaced the DPP one, before the four-token
// waves, the two-phase order and ropeFlat: Qwen2 q+k at 8192 tokens 11.38 us, against 11.36-11.47 us for a copy
// kernel with the same access pattern and no arithmetic, and 11.77 us for the previous
// layout (16-byte vectors, partner fetched by DPP: every element widened twice, 560 VALU
// instructions per token against 370 here); q alone 10.26 us (copy 9.69-9.90); k alone
// 4.17 us (copy 3.06; the token's sincos dominates a one-instruction token); Llama-8B q+k
// at 16384 tokens 53.39 us.  f64 fma / mul / add and the f32 <-> f64 conversions issue at
// the f32 fma rate on gfx950 (4.6-5.2 cycles per wave64 instruction, measured), so an
// f32 rotation with an error-bound test would issue more, not fewer, instructions.
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

// Half-pair layout.  Lane l of a group of RL = d / (2E) consecutive lanes holds elements
// E*l .. E*l + E-1 of the first half of a head row and the same E of the second half
// (chunks of E * element size bytes: 8 or 16 for bf16 / f16, 16 for f32).  Each of a row
// instruction's two loads covers 64 / RL half-rows, RL * E elements contiguous per group
// (128 B for bf16 at head_dim 128, the cache line).  One wavefront takes a token's rows
// (tensor 0's, then tensor 1's) in 2^split_log2 contiguous shares, passes of IPT row
// instructions each.  Waves past the last token redo the last token and store nothing, so
// no wave leaves before the loads (a branch there would serialise the kernel-argument
// loads ahead of the first global load).
template <typename T, int IPT, int RL, bool kOnePass, int E, int TPW>
__global__ void __launch_bounds__(256)
    ropeHalves(RopePair tp, const int64_t *__restrict__ pos, size_t seq, int passes, int split_log2,
               FreqTable ft) {
    static_assert(TPW == 1 || kOnePass, "several tokens per wave take their rows in one pass");
    using C = Chunk4<T, E>;
    using V = typename C::V;
    constexpr int kRows = kWave / RL;          // rows per wave instruction
    constexpr int kHalf = RL * E;              // elements per half row
    constexpr int kHalfBytes = kHalf * Fmt<T>::kBytes;
    constexpr int kRowBytes = 2 * kHalfBytes;
    // (cos, sin) of angle j = E l + e sits in slot e * RL + l: lane l's read of its element e
    // and the lanes' writes (slot = lane) both touch consecutive 16-byte slots, free of LDS
    // bank conflicts (slots E * 16 bytes apart conflicted E-fold)
    __shared__ double2 cs[256 / kWave][TPW][kHalf];
    const auto angleOf = [](int slot) { return (slot % RL) * E + slot / RL; };

    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const uint32_t gw = blockIdx.x * (256 / kWave) + uint32_t(wave);
    const size_t tbase = size_t(gw >> split_log2) * TPW; // the wave's first token
    const int first_instr = int(gw & ((1u << split_log2) - 1)) * passes * IPT;
    const int nh0 = tp.n_heads0, rows = nh0 + tp.n_heads1;
    const int rlane = lane / RL, l = lane % RL;
    const size_t tok0 = size_t(nh0) * kRowBytes, tok1 = size_t(tp.n_heads1) * kRowBytes; // token strides
    const char *in0 = static_cast<const char *>(tp.in0) + l * C::kBytes;
    const char *in1 = static_cast<const char *>(tp.in1) + l * C::kBytes - size_t(nh0) * kRowBytes;
    char *out0 = static_cast<char *>(tp.out0) + l * C::kBytes;
    char *out1 = static_cast<char *>(tp.out1) + l * C::kBytes - size_t(nh0) * kRowBytes;
    // tokens past the last redo the last token and store nothing
    const auto tokenOf = [&](int tk) { return min(tbase + size_t(tk), seq - 1); };

    // the lane's first frequency before the row loads (vector loads complete in issue order);
    // the wave's tokens share the frequencies
    const double f_first = ft.f[angleOf(lane < kHalf ? lane : 0)];
    __builtin_amdgcn_sched_barrier(0);
    double c[E], sn[E];
    const int npass = kOnePass ? 1 : passes;
    for (int pass = 0; pass < npass; ++pass) {
        V xa[TPW][IPT], xb[TPW][IPT];
#pragma unroll
        for (int tk = 0; tk < TPW; ++tk) {
            const size_t t = tokenOf(tk);
#pragma unroll
            for (int k = 0; k < IPT; ++k) {
                const int r = (first_instr + pass * IPT + k) * kRows + rlane;
                // rows past the token's last read its first q row (and store nothing)
                const char *src = (r < nh0 ? in0 + t * tok0 : (r < rows ? in1 + t * tok1 : in0 + t * tok0 - size_t(r) * kRowBytes)) +
                                  size_t(r) * kRowBytes;
                xa[tk][k] = C::load(src);
                xb[tk][k] = C::load(src + kHalfBytes);
            }
        }
        if (pass == 0) {
            bool far = false;
#pragma unroll
            for (int tk = 0; tk < TPW; ++tk) {
                const int64_t p = pos[tokenOf(tk)];
                for (int sl = lane; sl < kHalf; sl += kWave) {
                    const double ang = double(p) * (sl == lane ? f_first : ft.f[angleOf(sl)]);
                    double s0 = 0.0, c0 = 0.0;
                    if (fabs(ang) <= kSincosFastLimit)
                        sincosReduced(ang, &s0, &c0);
                    else
                        far = true; // also NaN
                    cs[wave][tk][sl] = make_double2(c0, s0);
                }
            }
            if (__builtin_expect(__any(far), 0)) {
                for (int tk = 0; tk < TPW; ++tk) {
                    const int64_t p = pos[tokenOf(tk)];
                    for (int sl = lane; sl < kHalf; sl += kWave) {
                        const double ang = double(p) * ft.f[angleOf(sl)];
                        if (!(fabs(ang) <= kSincosFastLimit)) {
                            double s0, c0;
                            librarySinCos(ang, &s0, &c0);
                            cs[wave][tk][sl] = make_double2(c0, s0);
                        }
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        // All of the pass's row loads land before the first rotation and store: the wave's
        // reads and writes then reach HBM as two phases.  Rotating token 0 as soon as its
        // rows arrive, its stores interleaved with the later tokens' loads, was slower:
        // q + k at 8192 tokens 10.78-10.85 -> 10.46-10.52 us (same-box A/B, 4 runs each; on
        // another box 10.71-10.76 -> 10.12-10.19 us).
        __builtin_amdgcn_sched_barrier(0);
        waitVmcnt<0>();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int tk = 0; tk < TPW; ++tk) {
            if (TPW > 1 || pass == 0) {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const double2 v = cs[wave][tk][e * RL + l];
                    c[e] = v.x;
                    sn[e] = v.y;
                }
            }
            const size_t t = tokenOf(tk);
            const bool live = tbase + size_t(tk) < seq;
#pragma unroll
            for (int k = 0; k < IPT; ++k) {
                const int r = (first_instr + pass * IPT + k) * kRows + rlane;
                if (live && r < rows) {
                    char *dst = (r < nh0 ? out0 + t * tok0 : out1 + t * tok1) + size_t(r) * kRowBytes;
                    float a[E], b[E], ya[E], yb[E];
                    C::unpack(xa[tk][k], a);
                    C::unpack(xb[tk][k], b);
#pragma unroll
                    for (int e = 0; e < E; ++e) rotatePair(a[e], b[e], c[e], sn[e], ya[e], yb[e]);
                    // packQ: arithmetic on the inputs and the host frequencies, no foreign NaN
                    // payload (a NaN theta takes the scalar kernel)
                    C::store(dst, C::packQ(ya));
                    C::store(dst + kHalfBytes, C::packQ(yb));
                }
            }
        }
    }
}

// TPW tokens per wave with each tensor's rows of those tokens taken as one flat run: a
// token's nh rows of one tensor sit next to the next token's in memory, so row instruction
// k of the wave covers flat rows k * kRows .. + kRows - 1 of the run, whichever tokens they
// belong to, and no lane of an instruction idles when a token's rows do not fill whole
// instructions (Qwen2 q: 12 rows of 8 per instruction, 6 instructions per 4 tokens instead
// of 8).  Instructions 0 .. i0 - 1 take tensor 0's run, the rest tensor 1's (the launcher
// uses one tensor).  Each lane reads the (cos, sin) pairs of its own row's token.  Otherwise as
// ropeHalves: the same rotation, the tokens' pairs computed while the loads are in flight,
// every load landed before the first rotation and store.
template <typename T, int RL, int E, int TPW, int I>
__global__ void __launch_bounds__(256)
    ropeFlat(RopePair tp, const int64_t *__restrict__ pos, size_t seq, int i0, FreqTable ft) {
    using C = Chunk4<T, E>;
    using V = typename C::V;
    constexpr int kRows = kWave / RL;          // rows per wave instruction
    constexpr int kHalf = RL * E;              // elements per half row
    constexpr int kHalfBytes = kHalf * Fmt<T>::kBytes;
    constexpr int kRowBytes = 2 * kHalfBytes;
    __shared__ double2 cs[256 / kWave][TPW][kHalf]; // slot e * RL + l holds angle E l + e
    const auto angleOf = [](int slot) { return (slot % RL) * E + slot / RL; };

    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const size_t tbase = (size_t(blockIdx.x) * (256 / kWave) + size_t(wave)) * TPW;
    const int rlane = lane / RL, l = lane % RL;
    const auto tokenOf = [&](int tk) { return min(tbase + size_t(tk), seq - 1); };

    // instruction k: the lane's token within the wave and its row in the tensor; a slot past
    // the run or past the last token reads row 0 and stores nothing
    int tkOf[I];
    size_t rowOf[I];
    bool ok[I];
#pragma unroll
    for (int k = 0; k < I; ++k) {
        const bool t1 = k >= i0; // wave-uniform
        const int nh = t1 ? tp.n_heads1 : tp.n_heads0;
        const int fr = (t1 ? k - i0 : k) * kRows + rlane; // flat row within the wave's run
        int tk = 0;
#pragma unroll
        for (int q = 1; q < TPW; ++q) tk += fr >= q * nh ? 1 : 0;
        const int rr = fr - tk * nh;
        ok[k] = rr < nh && tbase + size_t(tk) < seq;
        tkOf[k] = tk;
        rowOf[k] = ok[k] ? (tbase + size_t(tk)) * size_t(nh) + size_t(rr) : 0;
    }
    const double f_first = ft.f[angleOf(lane < kHalf ? lane : 0)];
    __builtin_amdgcn_sched_barrier(0);
    V xa[I], xb[I];
#pragma unroll
    for (int k = 0; k < I; ++k) {
        const char *src = static_cast<const char *>(k >= i0 ? tp.in1 : tp.in0) + rowOf[k] * kRowBytes + l * C::kBytes;
        xa[k] = C::load(src);
        xb[k] = C::load(src + kHalfBytes);
    }
    bool far = false;
#pragma unroll
    for (int tk = 0; tk < TPW; ++tk) {
        const int64_t p = pos[tokenOf(tk)];
        for (int sl = lane; sl < kHalf; sl += kWave) {
            const double ang = double(p) * (sl == lane ? f_first : ft.f[angleOf(sl)]);
            double s0 = 0.0, c0 = 0.0;
            if (fabs(ang) <= kSincosFastLimit)
                sincosReduced(ang, &s0, &c0);
            else
                far = true; // also NaN
            cs[wave][tk][sl] = make_double2(c0, s0);
        }
    }
    if (__builtin_expect(__any(far), 0)) {
        for (int tk = 0; tk < TPW; ++tk) {
            const int64_t p = pos[tokenOf(tk)];
            for (int sl = lane; sl < kHalf; sl += kWave) {
                const double ang = double(p) * ft.f[angleOf(sl)];
                if (!(fabs(ang) <= kSincosFastLimit)) {
                    double s0, c0;
                    librarySinCos(ang, &s0, &c0);
                    cs[wave][tk][sl] = make_double2(c0, s0);
                }
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // every row load lands before the first rotation and store (as in ropeHalves)
    __builtin_amdgcn_sched_barrier(0);
    waitVmcnt<0>();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < I; ++k) {
        if (!ok[k]) continue;
        double c[E], sn[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const double2 v = cs[wave][tkOf[k]][e * RL + l];
            c[e] = v.x;
            sn[e] = v.y;
        }
        char *dst = static_cast<char *>(k >= i0 ? tp.out1 : tp.out0) + rowOf[k] * kRowBytes + l * C::kBytes;
        float a[E], b[E], ya[E], yb[E];
        C::unpack(xa[k], a);
        C::unpack(xb[k], b);
#pragma unroll
        for (int e = 0; e < E; ++e) rotatePair(a[e], b[e], c[e], sn[e], ya[e], yb[e]);
        C::store(dst, C::packQ(ya));
        C::store(dst + kHalfBytes, C::packQ(yb));
    }
}

// One tensor whose head rows fill 1/TPI of a row instruction (k alone: 2 heads of 128 at
// E = 4 fill half): one wave instruction covers TPI consecutive tokens, the half-pair
// layout otherwise.  The wave computes the TPI tokens' (cos, sin) pairs, one per lane and
// token, and each lane reads its own token's.  Every lane carries data, so a token costs
// 1/TPI of a rotation instruction stream instead of a whole one.
template <typename T, int RL, int E, int TPI>
__global__ void __launch_bounds__(256)
    ropeHalvesPacked(RopePair tp, const int64_t *__restrict__ pos, size_t seq, FreqTable ft) {
    using C = Chunk4<T, E>;
    using V = typename C::V;
    constexpr int kRows = kWave / RL;          // rows per wave instruction
    constexpr int R = kRows / TPI;             // rows per token
    constexpr int kHalf = RL * E;
    constexpr int kHalfBytes = kHalf * Fmt<T>::kBytes;
    constexpr int kRowBytes = 2 * kHalfBytes;
    __shared__ double2 cs[256 / kWave][TPI][kHalf]; // slot e * RL + l holds angle E l + e
    const auto angleOf = [](int slot) { return (slot % RL) * E + slot / RL; };

    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const size_t tbase = (size_t(blockIdx.x) * (256 / kWave) + size_t(wave)) * TPI;
    const int rlane = lane / RL, l = lane % RL;
    const int tk = rlane / R, r = rlane % R;
    const bool live = tbase + size_t(tk) < seq;
    const size_t t = live ? tbase + size_t(tk) : seq - 1; // past the end: redo the last token
    const size_t row = t * R + size_t(r);
    const char *src = static_cast<const char *>(tp.in0) + row * kRowBytes + l * C::kBytes;

    const double f_first = ft.f[angleOf(lane < kHalf ? lane : 0)];
    __builtin_amdgcn_sched_barrier(0);
    const V xa = C::load(src), xb = C::load(src + kHalfBytes);
    bool far = false;
#pragma unroll
    for (int k = 0; k < TPI; ++k) {
        const int64_t p = pos[min(tbase + size_t(k), seq - 1)];
        for (int sl = lane; sl < kHalf; sl += kWave) {
            const double ang = double(p) * (sl == lane ? f_first : ft.f[angleOf(sl)]);
            double s0 = 0.0, c0 = 0.0;
            if (fabs(ang) <= kSincosFastLimit)
                sincosReduced(ang, &s0, &c0);
            else
                far = true; // also NaN
            cs[wave][k][sl] = make_double2(c0, s0);
        }
    }
    if (__builtin_expect(__any(far), 0)) {
        for (int k = 0; k < TPI; ++k) {
            const int64_t p = pos[min(tbase + size_t(k), seq - 1)];
            for (int sl = lane; sl < kHalf; sl += kWave) {
                const double ang = double(p) * ft.f[angleOf(sl)];
                if (!(fabs(ang) <= kSincosFastLimit)) {
                    double s0, c0;
                    librarySinCos(ang, &s0, &c0);
                    cs[wave][k][sl] = make_double2(c0, s0);
                }
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    double c[E], sn[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const double2 v = cs[wave][tk][e * RL + l];
        c[e] = v.x;
        sn[e] = v.y;
    }
    if (!live) return;
    float a[E], b[E], ya[E], yb[E];
    C::unpack(xa, a);
    C::unpack(xb, b);
#pragma unroll
    for (int e = 0; e < E; ++e) rotatePair(a[e], b[e], c[e], sn[e], ya[e], yb[e]);
    char *dst = static_cast<char *>(tp.out0) + row * kRowBytes + l * C::kBytes;
    C::store(dst, C::packQ(ya));
    C::store(dst + kHalfBytes, C::packQ(yb));
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

template <typename T, int IPT, bool kOnePass, int E, int TPW>
void launchHalvesRl(int rl, int passes, int split_log2, const RopePair &tp, const int64_t *pos,
                    size_t seq, const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor(((seq + TPW - 1) / TPW) << split_log2, 256 / kWave);
    switch (rl) {
    case 1: ropeHalves<T, IPT, 1, kOnePass, E, TPW><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    case 2: ropeHalves<T, IPT, 2, kOnePass, E, TPW><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    case 4: ropeHalves<T, IPT, 4, kOnePass, E, TPW><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    case 8: ropeHalves<T, IPT, 8, kOnePass, E, TPW><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    case 16: ropeHalves<T, IPT, 16, kOnePass, E, TPW><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    case 32: ropeHalves<T, IPT, 32, kOnePass, E, TPW><<<grid, 256, 0, s>>>(tp, pos, seq, passes, split_log2, ft); break;
    default: break;
    }
}

template <typename T, int E, int TPI>
void launchPackedRl(int rl, const RopePair &tp, const int64_t *pos, size_t seq, const FreqTable &ft,
                    hipStream_t s) {
    const unsigned grid = blocksFor((seq + TPI - 1) / TPI, 256 / kWave);
    switch (rl) {
    case 4: if constexpr (kWave / 4 >= TPI) ropeHalvesPacked<T, 4, E, TPI><<<grid, 256, 0, s>>>(tp, pos, seq, ft); break;
    case 8: if constexpr (kWave / 8 >= TPI) ropeHalvesPacked<T, 8, E, TPI><<<grid, 256, 0, s>>>(tp, pos, seq, ft); break;
    case 16: if constexpr (kWave / 16 >= TPI) ropeHalvesPacked<T, 16, E, TPI><<<grid, 256, 0, s>>>(tp, pos, seq, ft); break;
    case 32: if constexpr (kWave / 32 >= TPI) ropeHalvesPacked<T, 32, E, TPI><<<grid, 256, 0, s>>>(tp, pos, seq, ft); break;
    default: break;
    }
}

template <typename T, int TPW, int I>
void launchFlat(int i0, const RopePair &tp, const int64_t *pos, size_t seq, const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor((seq + TPW - 1) / TPW, 256 / kWave);
    ropeFlat<T, 8, 8, TPW, I><<<grid, 256, 0, s>>>(tp, pos, seq, i0, ft);
}

template <typename T, int E>
void launchHalvesE(int rl, int instr, int split_log2, int tpw, const RopePair &tp, const int64_t *pos,
                   size_t seq, const FreqTable &ft, hipStream_t s) {
    const int split = 1 << split_log2;
    const int per_wave = (instr + split - 1) / split;
    const int passes = (per_wave + 3) / 4, ipt = (per_wave + passes - 1) / passes;
    const auto go = [&](auto ipt_c) {
        constexpr int I = decltype(ipt_c)::value;
        if (passes == 1) {
            if (tpw == 4)
                launchHalvesRl<T, I, true, E, 4>(rl, passes, split_log2, tp, pos, seq, ft, s);
            else
                launchHalvesRl<T, I, true, E, 1>(rl, passes, split_log2, tp, pos, seq, ft, s);
        } else {
            launchHalvesRl<T, I, false, E, 1>(rl, passes, split_log2, tp, pos, seq, ft, s);
        }
    };
    switch (ipt) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    default: go(std::integral_constant<int, 4>{}); break;
    }
}

// The half-pair kernel when the shape fits it: head_dim / 2 <= 128 and a power-of-two
// lane group of at most 32, chunk-aligned pointers, and at least a quarter of a wave's
// lanes busy per token (fewer: ropeVec packs several tokens per block).  E = 8 (16-byte
// chunks) for 16-bit types once the rows fill a row instruction, else E = 4.  Tokens of 2
// row instructions with >= 8192 tokens: 4 tokens per wave, one wave each; otherwise waves
// per token: one for a single row instruction, else the fewest (at least two) that leave
// each wave <= 2 instructions.  Measured on MI355X, bf16, graph-replayed medians over >= 1
// GiB of rotating sets: q+k of Qwen2 at 8192 tokens (2 instructions at E = 8) 10.77 us
// with 4 tokens per wave, against 11.38 with 2 waves per token, 12.05 with 1, 11.30 with
// 8 tokens per wave and 11.47-11.57 for copy kernels of the same access pattern with 1-2
// tokens per wave (10.50 with 4, 10.70 for the best plain copy); q alone 9.51-9.78 with 4
// tokens per wave against 9.97-10.02; k alone (1 instruction at E = 4) 3.99 with one wave
// per token against 4.54 with 4 tokens per wave and 5.66 with 2 waves per token; Llama-8B
// q+k at 16384 tokens (5 instructions) 53.3-53.7 with 4 waves per token against 54.17 with
// 2, 56.65 with 1 and 56.7 with 4 tokens per wave; the chain's 2048-token q+k 3.86 with 2
// waves per token against 5.90 with 4 tokens per wave.
template <typename T>
bool launchHalves(const RopePair &tp, const int64_t *pos, size_t seq, size_t half,
                  const FreqTable &ft, hipStream_t s) {
    constexpr bool k16 = Fmt<T>::kBytes == 2;
    const size_t rows = size_t(tp.n_heads0) + size_t(tp.n_heads1);
    if (half % 4 != 0 || half > size_t(kMaxHalf) || rows == 0) return false;
    const auto fits = [&](size_t e) {
        const size_t rl = half / e;
        if (rl == 0 || rl > 32 || (rl & (rl - 1)) != 0) return false;
        const uintptr_t chunk = e * size_t(Fmt<T>::kBytes);
        for (const void *p : {static_cast<const void *>(tp.out0), tp.in0, static_cast<const void *>(tp.out1), tp.in1})
            if (p && (reinterpret_cast<uintptr_t>(p) % chunk) != 0) return false;
        return true;
    };
    int e = 4;
    if (k16 && half % 8 == 0 && fits(8) && rows >= size_t(kWave) / (half / 8)) e = 8;
    if (e == 4 && !fits(4)) return false;
    const int rl = int(half / size_t(e)), rpi = kWave / rl;
    if (rows * size_t(rl) * 4 < size_t(kWave)) return false;
    const size_t instr = (rows + size_t(rpi) - 1) / size_t(rpi);
    if (instr > size_t(INT32_MAX / 2)) return false;
    if (seq >= (size_t(1) << 31)) return false; // wave index is 32-bit
    // one tensor filling 1/2 or 1/4 of a row instruction: tokens packed per instruction.
    // Measured on MI355X (bf16, graph-replayed medians over >= 1 GiB of rotating sets): k
    // [8192, 2, 128] 3.43 us against 3.99 us with one token per wave; [8191, 1, 128] 3.26
    // against 3.88 us.
    if (tp.n_heads1 == 0 && e == 4 && rl >= 4 && (rows * 2 == size_t(rpi) || rows * 4 == size_t(rpi))) {
        if (rows * 2 == size_t(rpi))
            launchPackedRl<T, 4, 2>(rl, tp, pos, seq, ft, s);
        else
            launchPackedRl<T, 4, 4>(rl, tp, pos, seq, ft, s);
        return true;
    }
    // Four tokens per wave (16 loads of 16 bytes in flight per lane) when a token takes 2
    // row instructions and that still leaves >= 2048 waves; else one token per wave in
    // 2^split_log2 shares.
    // One tensor of 9-15 rows per token in 8-row instructions of 16-byte chunks (Qwen2 q
    // alone, as the reference's separate rope calls issue it): 4 tokens per wave as flat row
    // runs, every row slot busy (ropeFlat).  Measured on MI355X (graph-replayed medians over
    // >= 1 GiB of rotating sets, same-box A/B, 3 runs each): q [8192, 12, 128] 9.29-9.33 ->
    // 9.17-9.18 us (9.35 -> 9.09-9.12 on another box); 2 tokens per wave 10.35-10.39 us, 8
    // tokens 11.32-11.35 us.  With k in the same launch (7 instructions instead of 8) it
    // measured slower, 10.21-10.28 -> 11.06-11.08 us, so q + k keeps ropeHalves.
    if constexpr (k16) {
        if (tp.n_heads1 == 0 && instr == 2 && (seq + 3) / 4 >= 2048 && e == 8 && rl == 8) {
            const int i0 = (4 * tp.n_heads0 + 7) / 8;
            switch (i0) {
            case 5: launchFlat<T, 4, 5>(i0, tp, pos, seq, ft, s); return true;
            case 6: launchFlat<T, 4, 6>(i0, tp, pos, seq, ft, s); return true;
            case 7: launchFlat<T, 4, 7>(i0, tp, pos, seq, ft, s); return true;
            default: break; // 8: every slot already busy
            }
        }
    }
    int tpw = 1, split_log2 = 0;
    if (instr == 2 && (seq + 3) / 4 >= 2048) {
        tpw = 4;
    } else {
        split_log2 = instr >= 2 ? 1 : 0;
        while ((instr + (size_t(1) << split_log2) - 1) >> split_log2 > 2) ++split_log2;
        while (split_log2 > 0 && (seq << split_log2) >= (size_t(1) << 31)) --split_log2;
    }
    if (e == 8) {
        if constexpr (k16) launchHalvesE<T, 8>(rl, int(instr), split_log2, tpw, tp, pos, seq, ft, s);
    } else {
        launchHalvesE<T, 4>(rl, int(instr), split_log2, tpw, tp, pos, seq, ft, s);
    }
    return true;
}

template <typename T, int IPT>
void launchIpt(int vph, const RopePair &tp, const int64_t *pos, size_t seq, size_t tpb,
               uint32_t magic0, uint32_t magic1, const FreqTable &ft, hipStream_t s) {
    const unsigned grid = blocksFor(seq, tpb);
    switch (vph) {
    case 1: ropeVec<T, IPT, 1><<<grid, 256, 0, s>>>(tp, pos, seq, int(tpb), magic0, magic1, ft); break;
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
    if (!std::isnan(theta) && (launchHalves<T>(tp, pos, seq, d / 2, ft, s) || launchVec<T>(tp, pos, seq, d, ft, s)))
        return;
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
