// Linear layers for gfx950: the reference's dense linear and W8A16 over INT8 weights.
//
// Semantics: reference src/ops/linear/cpu/linear_cpu.cpp:11-41 -- out[m][n] =
// T(sum_k x[m][k] * w[n][k] + bias[n]) with an f32 sum, x [rows, K], w [N, K].  W8A16 (no
// reference kernel): w is INT8 codes [N, K] with one f32 scale per output channel n, and
// out[m][n] = T(scale[n] * sum_k x[m][k] * code[n][k] + bias[n]).  The MFMA path sums the
// exact products of bf16 / f16 operands (INT8 codes are exact in both) in f32; the order of
// the sum differs from the reference's left-to-right loop, which the tests bound by the f32
// accumulation error.
//
// Design, by row count M (the launcher at the end picks the kernel):
//  - M = 1 (decode), linearGemvRow: HBM-bound on the weights, one wave per output channel
//    (4 for the INT8 lm_head) with its whole weight row requested up front in 1 KB load
//    instructions, x in LDS or L1 / L2, f32 FMAs, a butterfly.  linearGemv (the same sum,
//    no LDS) takes rows too long for that and M = 2 (INT8 weights with N >= 4096 and M = 2
//    go to linearSkinny instead).
//  - M <= 16, linearSkinny: HBM-bound; a block owns 16 channels, its waves split K, load
//    weight rows row-contiguously and transpose them through a per-wave LDS tile into
//    v_mfma_f32_16x16x32 operands; partials summed in LDS in wave order.
//  - more rows (prefill): MFMA-bound, v_mfma_f32_32x32x16 on 128 x 128 output tiles of 8
//    waves computing out^T = w x^T (each lane ends with 4 consecutive channels of one row).
//    linearDirect (16-bit weights, K % 64 == 0) moves the operands HBM -> LDS with
//    global_load_lds_dwordx4 through 3 stages and XOR-swizzled rows; linearTiled (INT8
//    weights or other K) stages them through registers and a padded LDS tile, converting
//    INT8 codes to exact bf16 / f16 on the way.  Blocks map to the 8 XCDs so that a weight
//    tile stays in one L2 while the row tiles pass over it.
//  - anything else (f32, unaligned rows, K not a multiple of 8 / 16): linearScalar, one
//    thread per output with the reference's sequential sum.
// INT8 codes enter every MFMA as exact bf16 / f16 values and the per-channel scale multiplies
// the f32 sum once.
#include "common.hpp"
#include "launch.hpp"
#include "linear_common.hpp"
#include "rowplan.hpp"

#include <algorithm>
#include <type_traits>

namespace llaisys::kernels {

namespace {

using namespace lin;
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct LinearArgs {
    void *out;
    const void *x;
    const void *w;       // elements of T, or INT8 codes
    const float *scale;  // INT8 only
    const void *bias;    // T, or null
    int M, N, K;
};

// 32 x 32 x 16: A[m = l % 32][k = 8 (l / 32) + j], B[k = 8 (l / 32) + j][n = l % 32],
// D[m = 8 (i / 4) + 4 (l / 32) + i % 4][n = l % 32]; twice the sustained rate of 16 x 16 x 32
template <typename T>
__device__ __forceinline__ f32x16 mfma32(const v4u &a, const v4u &b, const f32x16 &c) {
    if constexpr (std::is_same_v<T, BF16>)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Many rows (prefill): MFMA-bound.  A block of NWW x NWX waves owns BW output channels x BX rows;
// per stage of 64 k it stages both tiles in LDS (row-contiguous global loads, 144-byte row
// pitch: the MFMA-operand reads and the tile writes are bank-conflict-free), double-buffered
// with the next stage's global loads in flight during the MFMAs.  The MFMA computes
// out^T = w x^T: weight rows are the A operand and activation rows the B operand, so each
// lane ends with 4 consecutive output channels of one row (one 8-byte store).  INT8 codes
// are converted to exact bf16 / f16 values on their way into LDS.
constexpr int kTK = 64;               // k per stage
constexpr int kXcds = 8;              // accelerator complex dies of an MI355X

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS accesses, not for its
// global loads (__syncthreads' fence would also drain the prefetches in flight).  The
// memory clobber keeps the compiler from moving accesses across it.
constexpr int kTPitch = 2 * kTK + 16; // LDS row pitch (bytes)

// Epilogue of the tiled kernels: D[8 q + 4 h + e][r32] of 32 x 32 tile (i, j) (q, e < 4) is
// out[row xr + 32 j + r32][channel wr + 32 i + 8 q + 4 h + e], 4 consecutive channels per
// (q, lane): scale (INT8), bias, one 8-byte store (or element stores at the edge).
template <typename T, bool kInt8, int TW, int TX>
__device__ __forceinline__ void storeTiles(const LinearArgs &a, const f32x16 (&acc)[TW][TX], int wr, int xr, int lane) {
    const int r32 = lane % 32, h2 = lane / 32;
    const bool vec = a.N % 4 == 0;
    using C = std::conditional_t<std::is_same_v<T, BF16>, Bf16Cvt, F16Cvt>;
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = wr + 32 * i + 8 * q + 4 * h2;
            float sc[4], bv[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int ne = min(n + e, a.N - 1);
                sc[e] = kInt8 ? a.scale[ne] : 1.0f;
                bv[e] = a.bias ? Fmt<T>::get(a.bias, ne) : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < TX; ++j) {
                const int m = xr + 32 * j + r32;
                if (m >= a.M) continue;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float sum = kInt8 ? sc[e] * acc[i][j][4 * q + e] : acc[i][j][4 * q + e];
                    v[e] = a.bias ? sum + bv[e] : sum;
                }
                if (vec && n + 3 < a.N) {
                    const uint32_t lo = C::narrow(v[0]) | (C::narrow(v[1]) << 16);
                    const uint32_t hi = C::narrow(v[2]) | (C::narrow(v[3]) << 16);
                    *reinterpret_cast<v2u *>(static_cast<char *>(a.out) + (size_t(m) * a.N + n) * 2) = v2u{lo, hi};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < a.N) Fmt<T>::put(a.out, size_t(m) * a.N + n + e, v[e]);
                }
            }
        }
}

template <typename T, bool kInt8, int BW, int BX, int NWW, int NWX, int P>
__global__ void __launch_bounds__(NWW * NWX * 64)
    linearTiled(LinearArgs a) {
    constexpr int NT = NWW * NWX * kWave;         // threads
    constexpr int WW = BW / NWW, WX = BX / NWX;   // wave tile (NWW x NWX waves)
    constexpr int TW = WW / 32, TX = WX / 32;     // 32 x 32 MFMA tiles per wave
    constexpr int kXRows = NT / 8;                // 16-bit rows: 8 lanes x 16 B
    constexpr int kXLoads = BX / kXRows;
    constexpr int kWRows = kInt8 ? NT / 4 : NT / 8; // INT8 rows: 4 lanes x 16 codes
    constexpr int kWLoads = BW / kWRows;
    static_assert(kXLoads >= 1 && kWLoads >= 1 && TW >= 1 && TX >= 1, "tile too small for the block");
    static_assert(BX % kXRows == 0 && BW % kWRows == 0, "the load passes must cover the tile rows");
    __shared__ __align__(16) char lds[2][(BW + BX) * kTPitch];
    const int tid = int(threadIdx.x);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    // Blocks are dispatched to the 8 XCDs round-robin, each XCD with its own L2: give each
    // XCD a contiguous range of weight tiles and walk the activation tiles fastest inside it,
    // so that a weight tile stays in that L2 while every row tile passes over it.
    const int nbx = (a.M + BX - 1) / BX;
    const int nb = int(gridDim.x), b = int(blockIdx.x);
    const int v = nb % kXcds == 0 ? (b % kXcds) * (nb / kXcds) + b / kXcds : b;
    const int bx = v % nbx, bw = v / nbx;
    const int w0 = bw * BW, x0 = bx * BX;
    const int ww0 = (wave % NWW) * WW, wx0 = (wave / NWW) * WX;
    const char *xb = static_cast<const char *>(a.x);
    const char *wb = static_cast<const char *>(a.w);
    const int nk = (a.K + kTK - 1) / kTK;

    // global loads of stage kt: activation rows (t / 8 + 32 i, chunk t % 8) and weight rows
    const int xr = tid / 8, xc = tid % 8;
    const int wr = tid / (NT / kWRows), wc = tid % (NT / kWRows);
    // global loads of stage kt into ring slot r; past the last stage: the last stage again
    // (loads stay unconditional, so that the compiler keeps them where they are issued)
    v4u gx[P][kXLoads], gw[P][kWLoads];
    const auto loadGlobal = [&](int kt, v4u(&rx)[kXLoads], v4u(&rw)[kWLoads]) {
        kt = min(kt, nk - 1);
        const int kx = kt * kTK + 8 * xc;
        const bool xin = kx < a.K; // K % 8 == 0
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int row = min(x0 + xr + kXRows * i, a.M - 1);
            rx[i] = *reinterpret_cast<const v4u *>(xb + (size_t(row) * a.K + (xin ? kx : 0)) * 2);
            if (!xin) rx[i] = v4u{0u, 0u, 0u, 0u};
        }
        const int kw = kt * kTK + (kInt8 ? 16 : 8) * wc;
        const bool win = kw < a.K; // K % 8 == 0 (16-bit) / K % 16 == 0 (INT8)
#pragma unroll
        for (int i = 0; i < kWLoads; ++i) {
            const int row = min(w0 + wr + kWRows * i, a.N - 1);
            rw[i] = *reinterpret_cast<const v4u *>(wb + (size_t(row) * a.K + (win ? kw : 0)) * (kInt8 ? 1 : 2));
            if (!win) rw[i] = v4u{0u, 0u, 0u, 0u};
        }
    };
    const auto storeLds = [&](int buf, const v4u(&rx)[kXLoads], const v4u(&rw)[kWLoads]) {
        char *base = lds[buf];
#pragma unroll
        for (int i = 0; i < kXLoads; ++i)
            *reinterpret_cast<v4u *>(base + (BW + xr + kXRows * i) * kTPitch + 16 * xc) = rx[i];
#pragma unroll
        for (int i = 0; i < kWLoads; ++i) {
            char *dst = base + (wr + kWRows * i) * kTPitch;
            if constexpr (kInt8) {
                *reinterpret_cast<v4u *>(dst + 32 * wc) = codesToT<T>(v2u{rw[i].x, rw[i].y});
                *reinterpret_cast<v4u *>(dst + 32 * wc + 16) = codesToT<T>(v2u{rw[i].z, rw[i].w});
            } else {
                *reinterpret_cast<v4u *>(dst + 16 * wc) = rw[i];
            }
        }
    };

    f32x16 acc[TW][TX];
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int j = 0; j < TX; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    const int r32 = lane % 32, h2 = lane / 32;

    // stage 0 to LDS, stages 1..P in flight
    loadGlobal(0, gx[0], gw[0]);
    storeLds(0, gx[0], gw[0]);
#pragma unroll
    for (int r = 0; r < P; ++r) loadGlobal(1 + r, gx[r], gw[r]);
    ldsBarrier();
    for (int base = 0; base < nk; base += P) {
#pragma unroll
        for (int r = 0; r < P; ++r) {
            const int kt = base + r; // stage in LDS; ring slot r holds stage kt + 1
            if (kt >= nk) break;
            const char *tile = lds[kt & 1];
#pragma unroll
            for (int st = 0; st < kTK / 16; ++st) {
                v4u fa[TW], fb[TX];
#pragma unroll
                for (int i = 0; i < TW; ++i)
                    fa[i] = *reinterpret_cast<const v4u *>(tile + (ww0 + 32 * i + r32) * kTPitch + 32 * st + 16 * h2);
#pragma unroll
                for (int j = 0; j < TX; ++j)
                    fb[j] = *reinterpret_cast<const v4u *>(tile + (BW + wx0 + 32 * j + r32) * kTPitch + 32 * st + 16 * h2);
#pragma unroll
                for (int i = 0; i < TW; ++i)
#pragma unroll
                    for (int j = 0; j < TX; ++j) acc[i][j] = mfma32<T>(fa[i], fb[j], acc[i][j]);
            }
            // stage kt + 1 (past the end: harmless, nothing reads it) into the other buffer,
            // whose last readers finished before the previous barrier; then refill the slot
            storeLds((kt + 1) & 1, gx[r], gw[r]);
            loadGlobal(kt + 1 + P, gx[r], gw[r]);
            ldsBarrier();
        }
    }

    storeTiles<T, kInt8, TW, TX>(a, acc, w0 + ww0, x0 + wx0, lane);
}

// Many rows, 16-bit weights, K a multiple of 64: the tiled kernel's MFMA work with the
// operands moved HBM -> LDS by global_load_lds_dwordx4 (no register staging, no LDS write
// instructions) through S stages (S - 1 in flight while the MFMAs run on one).  A load
// instruction fills 1 KB of LDS contiguously (8 rows x 128 B, one 64-k stage of a row),
// so rows cannot be padded; instead the lane that fills slot c of row r fetches k-chunk
// c ^ ((r >> 1) & 7), and the MFMA-operand reads apply the same XOR (bank-conflict-free,
// measured).  Waits count this wave's loads (vmcnt) and one LDS-only barrier per stage
// makes every wave's loads visible and frees the stage read two steps ago.
template <typename T, int BW, int BX, int NWW, int NWX, int S>
__global__ void __launch_bounds__(NWW * NWX * 64)
    linearDirect(LinearArgs a) {
    constexpr int NWV = NWW * NWX;
    constexpr int WW = BW / NWW, WX = BX / NWX, TW = WW / 32, TX = WX / 32;
    constexpr int kRowB = 2 * kTK;                 // bytes of a row per stage
    constexpr int kStageB = (BW + BX) * kRowB;
    constexpr int kLoads = (BW + BX) / 8 / NWV;    // loads (8 rows each) per wave per stage
    static_assert((BW + BX) % (8 * NWV) == 0 && kLoads * (S - 2) < 64, "load split");
    __shared__ __align__(16) char lds[S * kStageB];
    const int tid = int(threadIdx.x), lane = tid % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int nbx = (a.M + BX - 1) / BX;
    const int nb = int(gridDim.x), b = int(blockIdx.x);
    const int v = nb % kXcds == 0 ? (b % kXcds) * (nb / kXcds) + b / kXcds : b;
    const int bx = v % nbx, bw = v / nbx;
    const int w0 = bw * BW, x0 = bx * BX;
    const int ww0 = (wave % NWW) * WW, wx0 = (wave / NWW) * WX;
    const char *xb = static_cast<const char *>(a.x), *wb = static_cast<const char *>(a.w);
    const int nk = a.K / kTK;
    // tile rows [0, BW) are weight rows, [BW, BW + BX) activation rows (clamped at the edges)
    const char *src[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const int tr = 8 * (wave * kLoads + i) + lane / 8;
        const int kc = (lane % 8) ^ ((tr >> 1) & 7);
        src[i] = tr < BW ? wb + (size_t(min(w0 + tr, a.N - 1)) * a.K + 8 * kc) * 2
                         : xb + (size_t(min(x0 + tr - BW, a.M - 1)) * a.K + 8 * kc) * 2;
    }
    const auto issue = [&](int kt) { // past the last stage: the last stage again, never read
        const int ktc = min(kt, nk - 1);
        char *dst = lds + (kt % S) * kStageB;
#pragma unroll
        for (int i = 0; i < kLoads; ++i)
            __builtin_amdgcn_global_load_lds(
                (const void __attribute__((address_space(1))) *)(src[i] + size_t(ktc) * kRowB),
                (void __attribute__((address_space(3))) *)(dst + 8 * (wave * kLoads + i) * kRowB), 16, 0, 0);
    };
    f32x16 acc[TW][TX];
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int j = 0; j < TX; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    const int r32 = lane % 32, h2 = lane / 32;
#pragma unroll
    for (int st = 0; st < S - 1; ++st) issue(st);
    for (int kt = 0; kt < nk; ++kt) {
        waitVmcnt<kLoads * (S - 2)>(); // this wave's loads of stage kt have landed
        ldsBarrier();                  // every wave's have; stage kt - 1 is no longer read
        issue(kt + S - 1);
        const char *tile = lds + (kt % S) * kStageB;
#pragma unroll
        for (int st = 0; st < kTK / 16; ++st) {
            v4u fa[TW], fb[TX];
#pragma unroll
            for (int i = 0; i < TW; ++i) {
                const int row = ww0 + 32 * i + r32;
                fa[i] = *reinterpret_cast<const v4u *>(tile + row * kRowB + 16 * ((2 * st + h2) ^ ((row >> 1) & 7)));
            }
#pragma unroll
            for (int j = 0; j < TX; ++j) {
                const int row = BW + wx0 + 32 * j + r32;
                fb[j] = *reinterpret_cast<const v4u *>(tile + row * kRowB + 16 * ((2 * st + h2) ^ ((row >> 1) & 7)));
            }
#pragma unroll
            for (int i = 0; i < TW; ++i)
#pragma unroll
                for (int j = 0; j < TX; ++j) acc[i][j] = mfma32<T>(fa[i], fb[j], acc[i][j]);
        }
    }
    waitVmcnt<0>(); // no LDS write may still be landing when the wave ends
    storeTiles<T, false, TW, TX>(a, acc, w0 + ww0, x0 + wx0, lane);
}

// Few rows (M <= 16, decode): HBM-bound on the weights; the skinny MFMA loop of
// linear_common.hpp over one set of 16 channels, x rows >= M entering as zeros.  The waves'
// 16 x 16 partials are summed in LDS in wave order.
template <typename T, bool kInt8>
__global__ void __launch_bounds__(1024)
    linearSkinny(LinearArgs a) {
    // dynamic LDS, sized by the launch: nw transpose tiles, then nw partial tiles
    extern __shared__ __align__(16) char smem[];
    const int nw = int(blockDim.x) / kWave;
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int lane = int(threadIdx.x) % kWave;
    const int r16 = lane % 16, g4 = lane / 16;
    const int n0 = int(blockIdx.x) * 16;
    char *tile = smem + size_t(wave) * 16 * skinnyPitch(kInt8);
    float(*red)[256] = reinterpret_cast<float(*)[256]>(smem + nw * 16 * skinnyPitch(kInt8));
    const char *xrow = static_cast<const char *>(a.x) + size_t(min(r16, a.M - 1)) * a.K * 2;
    const bool xlane = r16 < a.M;
    const v4u z4 = {0u, 0u, 0u, 0u};
    const auto xop = [&](int k) {
        const v4u v = *reinterpret_cast<const v4u *>(xrow + size_t(k < a.K ? k : 0) * 2);
        return xlane && k < a.K ? v : z4;
    };
    f32x4 acc[1] = {{0.0f, 0.0f, 0.0f, 0.0f}};
    const int rows0[1] = {n0};
    skinnyGroups<T, kInt8, 1>(acc, static_cast<const char *>(a.w), rows0, a.N, a.K, tile, wave, nw, lane, xop);
    // D[m = 4 g + e][n = r16]
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][(4 * g4 + e) * 16 + r16] = acc[0][e];
    __syncthreads();
    for (int t = int(threadIdx.x); t < 16 * a.M; t += int(blockDim.x)) {
        const int m = t / 16, n = n0 + t % 16;
        if (n < a.N) {
            float s = 0.0f;
            for (int w = 0; w < nw; ++w) s += red[w][t];
            if constexpr (kInt8) s = a.scale[n] * s;
            if (a.bias) s = s + Fmt<T>::get(a.bias, n);
            Fmt<T>::put(a.out, size_t(m) * a.N + n, s);
        }
    }
}

// One or two rows (decode): each wave owns one output channel and streams its weight row,
// 16 bytes per lane per load (1 KB contiguous per instruction, the pattern that streams HBM
// fastest), with FMAs in f32 against the matching x chunks (cache hits) and a DPP /
// permlane butterfly over the lane partials at the end.  No LDS and no cross-block
// synchronisation, so N output channels give N waves however small N is.
template <typename T, bool kInt8, int M>
__global__ void __launch_bounds__(256)
    linearGemv(LinearArgs a) {
    constexpr int E = kInt8 ? 16 : 8;  // weight elements per 16-byte chunk
    constexpr int U = 4;               // chunks in flight per lane
    const int lane = int(threadIdx.x) % kWave;
    const int n = int(blockIdx.x) * 4 + int(threadIdx.x) / kWave; // wave-uniform
    if (n >= a.N) return;
    const int nc = a.K / E; // K % E == 0
    const char *wrow = static_cast<const char *>(a.w) + size_t(n) * a.K * (kInt8 ? 1 : 2);
    const char *xb = static_cast<const char *>(a.x);
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    for (int c0 = lane; c0 < nc; c0 += kWave * U) {
        // all loads first (a chunk past the row end reads chunk 0 and is masked below)
        v4u wv[U], xv[U][M][E / 8];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int c = c0 + kWave * u < nc ? c0 + kWave * u : 0;
            wv[u] = *reinterpret_cast<const v4u *>(wrow + size_t(c) * 16);
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int h = 0; h < E / 8; ++h)
                    xv[u][m][h] = *reinterpret_cast<const v4u *>(xb + (size_t(m) * a.K + size_t(c) * E + 8 * h) * 2);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + kWave * u >= nc) continue;
            float wf[E];
            if constexpr (kInt8) {
                const uint32_t ww[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
                for (int e = 0; e < E; ++e) wf[e] = float(int8_t(ww[e / 4] >> (8 * (e % 4))));
            } else {
                Fmt<T>::unpack(wv[u], wf);
            }
#pragma unroll
            for (int m = 0; m < M; ++m)
#pragma unroll
                for (int h = 0; h < E / 8; ++h) {
                    float xf[8];
                    Fmt<T>::unpack(xv[u][m][h], xf);
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[m] = __builtin_fmaf(xf[e], wf[8 * h + e], acc[m]);
                }
        }
    }
    const float sc = kInt8 ? a.scale[n] : 1.0f;
    const float bv = a.bias ? Fmt<T>::get(a.bias, n) : 0.0f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float s = waveGroupReduce<kWave, SumOp>(acc[m]);
        if (lane == 0) {
            if constexpr (kInt8) s = sc * s;
            if (a.bias) s = s + bv;
            Fmt<T>::put(a.out, size_t(m) * a.N + n, s);
        }
    }
}

// One row (decode): linearGemv's sum -- per output channel one wave, lane chunks lane,
// lane + 64, ... in one FMA chain, then the same butterfly -- with every weight chunk of the
// wave's C channels requested before anything else (C x J per lane) and x staged once per
// block in LDS (kLds) or read through L1 / L2, so the loads are all in flight behind one x
// round trip.  Same bits as linearGemv (and
// as the fused rms_norm -> projection, which sums the same way).  Measured on MI355X (M = 1,
// >= 1 GiB of rotating weight sets): W8A16 [8960, 1536] 5.47 us against 6.79 us for
// linearSkinny and 7.55 us for linearGemv; bf16 [8960, 1536] 6.17 against 7.39 us; W8A16
// [1536, 8960] 6.41 against 7.00 us; bf16 [1536, 8960] 8.28 against 9.38 us.
template <typename T, bool kInt8, int J, int C, bool kLds, int NW>
__global__ void __launch_bounds__(NW * kWave)
    linearGemvRow(LinearArgs a) {
    using F = Fmt<T>;
    constexpr int E = kInt8 ? 16 : 8; // weight elements per 16-byte chunk
    extern __shared__ __align__(16) char xs_raw[];
    const uint16_t *xs = kLds ? reinterpret_cast<const uint16_t *>(xs_raw) : static_cast<const uint16_t *>(a.x);
    const int lane = int(threadIdx.x) % kWave;
    const int n0 = (int(blockIdx.x) * NW + int(threadIdx.x) / kWave) * C; // wave-uniform
    const int nc = a.K / E;
    // a channel past the last loads a valid row and stores nothing (its wave still joins the
    // block barrier); a chunk past the row end reads chunk 0 and is skipped
    v4u wv[C][J];
#pragma unroll
    for (int ci = 0; ci < C; ++ci) {
        const int n = n0 + ci;
        const char *wrow = static_cast<const char *>(a.w) + size_t(n < a.N ? n : a.N - 1) * a.K * (kInt8 ? 1 : 2);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = lane + kWave * j;
            wv[ci][j] = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(wrow + size_t(c < nc ? c : 0) * 16));
        }
    }
    if constexpr (kLds) {
        for (int i = int(threadIdx.x); i < a.K / 8; i += NW * kWave)
            reinterpret_cast<v4u *>(xs_raw)[i] = reinterpret_cast<const v4u *>(a.x)[i];
        __syncthreads();
    }
    // chunk-major: the lane's x chunk is unpacked once for the wave's C channels; each
    // channel still sums its chunks and elements in the same order (one FMA chain)
    float acc[C];
#pragma unroll
    for (int ci = 0; ci < C; ++ci) acc[ci] = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int c = lane + kWave * j;
        if (c >= nc) continue; // (the lane's remaining chunks are past the end too)
        float xf[E];
#pragma unroll
        for (int h = 0; h < E / 8; ++h) F::unpack(*reinterpret_cast<const v4u *>(xs + c * E + 8 * h), xf + 8 * h);
#pragma unroll
        for (int ci = 0; ci < C; ++ci) {
            float wf[E];
            if constexpr (kInt8) {
                const uint32_t ww[4] = {wv[ci][j].x, wv[ci][j].y, wv[ci][j].z, wv[ci][j].w};
#pragma unroll
                for (int e = 0; e < E; ++e) wf[e] = float(int8_t(ww[e / 4] >> (8 * (e % 4))));
            } else {
                F::unpack(wv[ci][j], wf);
            }
#pragma unroll
            for (int e = 0; e < E; ++e) acc[ci] = __builtin_fmaf(xf[e], wf[e], acc[ci]);
        }
    }
#pragma unroll
    for (int ci = 0; ci < C; ++ci) {
        float t = waveGroupReduce<kWave, SumOp>(acc[ci]);
        const int n = n0 + ci;
        if (lane == 0 && n < a.N) {
            if constexpr (kInt8) t = a.scale[n] * t;
            if (a.bias) t = t + F::get(a.bias, n);
            F::put(a.out, n, t);
        }
    }
}

// Any shape and type: one thread per output, the sum in the reference's order.
template <typename T, bool kInt8>
__global__ void __launch_bounds__(256)
    linearScalar(LinearArgs a) {
    const size_t idx = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= size_t(a.M) * a.N) return;
    const size_t m = idx / a.N, n = idx % a.N;
    float sum = 0.0f;
    for (int k = 0; k < a.K; ++k) {
        const float wv = kInt8 ? float(static_cast<const int8_t *>(a.w)[n * a.K + k]) : Fmt<T>::get(a.w, n * a.K + k);
        sum = sum + Fmt<T>::get(a.x, m * a.K + k) * wv;
    }
    if constexpr (kInt8) sum = a.scale[n] * sum;
    if (a.bias) sum = sum + Fmt<T>::get(a.bias, n);
    Fmt<T>::put(a.out, idx, sum);
}

// One row: linearGemvRow with J = ceil(chunks / 64) <= 24; false (linearGemv, the same sum)
// otherwise.  Variants (event timings of 5-16 rotating weight sets, all bit-identical):
//  - x staged in LDS by the block, except INT8 weights over at most 4096 channels, where the
//    block's staging is not hidden behind its 4 rows of codes and x is read from L1 / L2:
//    [3584, 3584] 5.54 -> 5.23 us, [1536, 8960] 6.26 -> 5.86 us, [3584, 18944] 18.7 -> 17.5 us
//    (larger N loses: [18944, 3584] 14.4 -> 15.3 us; bf16 [1536, 8960] 8.1 -> 8.7 us);
//  - 4 channels per wave for INT8 rows of at most 2 chunks per lane over 65536+ channels (the
//    lm_head), which spreads the block's x staging over 16 rows: [151936, 1536] 46.0 -> 40.0 us
//    (at [8960, 1536] it loses, 5.45 -> 6.57 us: too few blocks); 2 channels per wave in
//    4-wave blocks for such rows over 4097..65535 channels: [8960, 1536] 5.28-5.31 ->
//    4.99-5.03 us, [17920, 1536] 7.73-7.82 -> 7.66-7.68 us (same-box A/B, 3 runs each);
//  - waves per block: 8 where x is staged (the staging shared by more rows: bf16 [1536, 8960]
//    8.19 -> 7.70 us, [1536, 1536] 3.10 -> 2.95 us, [8960, 1536] 6.17 -> 6.09 us; 16 waves
//    10.5 us), 2 where it is read from L1 / L2 (INT8 [1536, 8960] 5.88 -> 5.68 us), 4 for
//    the 4-channel lm_head waves (8: 40.7 -> 42.6 us).
template <typename T, bool kInt8, int C, bool kLds, int NW, int J>
bool launchRowJ(const LinearArgs &a, int j, hipStream_t s) {
    if constexpr (J > 0) {
        if (j == J) {
            const unsigned blocks = unsigned((a.N + NW * C - 1) / (NW * C));
            linearGemvRow<T, kInt8, J, C, kLds, NW><<<blocks, NW * kWave, kLds ? size_t(a.K) * 2 : 0, s>>>(a);
            return true;
        }
        return launchRowJ<T, kInt8, C, kLds, NW, J - 1>(a, j, s);
    }
    return false;
}

template <typename T, bool kInt8>
bool launchGemv1(const LinearArgs &a, hipStream_t s) {
    constexpr int E = kInt8 ? 16 : 8;
    if (a.K % E != 0 || size_t(a.K) * 2 > 64 * 1024) return false;
    const int j = (a.K / E + kWave - 1) / kWave;
    if (j < 1 || j > 24) return false;
    if constexpr (kInt8) {
        if (a.N <= 4096) return launchRowJ<T, true, 1, false, 2, 24>(a, j, s);
        if (a.N >= 65536 && j <= 2) return launchRowJ<T, true, 4, true, 4, 2>(a, j, s);
        if (j <= 2) return launchRowJ<T, true, 2, true, 4, 2>(a, j, s);
    }
    return launchRowJ<T, kInt8, 1, true, 8, 24>(a, j, s);
}

template <typename T, bool kInt8>
void launch(const LinearArgs &a, hipStream_t s) {
    if (a.M == 0 || a.N == 0) return;
    const auto al = [](const void *p, size_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; };
    constexpr bool kMfmaType = std::is_same_v<T, BF16> || std::is_same_v<T, F16>;
    // MFMA paths: 16-bit activations, 16-byte aligned rows (K % 8 == 0; INT8 codes K % 16 == 0)
    if (kMfmaType && a.K > 0 && a.K % (kInt8 ? 16 : 8) == 0 && al(a.x, 16) && al(a.w, 16)) {
        if constexpr (kMfmaType) {
            // one or two rows: the VALU GEMV (one wave per channel) while its f32 work stays
            // under the HBM time -- always for 16-bit weights; for INT8 weights (16 codes per
            // 16 bytes to convert) only when there are too few 16-channel tiles for the MFMA
            // kernel to occupy the chip
            // one row: the VALU sum of linearGemv (linearGemvRow when the row fits its
            // registers) -- also for INT8 weights, whatever N, so that the fused rms_norm ->
            // projection, which sums the same way, matches it bit for bit
            if (a.M == 1 && launchGemv1<T, kInt8>(a, s)) return;
            if (a.M == 1 || (a.M == 2 && (!kInt8 || (a.N + 15) / 16 < 256))) {
                const unsigned blocks = unsigned((a.N + 3) / 4);
                if (a.M == 1)
                    linearGemv<T, kInt8, 1><<<blocks, 256, 0, s>>>(a);
                else
                    linearGemv<T, kInt8, 2><<<blocks, 256, 0, s>>>(a);
                return;
            }
            if (a.M <= 16) {
                // waves per block: enough blocks x waves to fill the chip, at most one wave
                // per group of 128 k
                const int tiles = (a.N + 15) / 16, nw = skinnyWaves(a.N, a.K);
                const size_t lds = size_t(nw) * (16 * skinnyPitch(kInt8) + 256 * sizeof(float));
                linearSkinny<T, kInt8><<<unsigned(tiles), unsigned(nw * kWave), lds, s>>>(a);
                return;
            }
            // tile shape: 128 x 128 (8 waves, 2 stages of loads in flight) while that still
            // gives most CUs a block, else 64 x 64
            const auto blocks = [&](int bw, int bx) {
                return unsigned((a.N + bw - 1) / bw) * unsigned((a.M + bx - 1) / bx);
            };
            if (blocks(128, 128) >= 192) {
                // 16-bit weights: 96 x 128 tiles (4 waves of 96 x 32, 4 stages) when 128 x 128
                // tiles leave CUs idle in a single round and the narrower tiles still fit one:
                // prefill 2048 x 8960 -> 1536 (192 vs 256 tiles) 73.9 -> 69.9 us, the same bits
                // Grids of 512+ tiles: 4 waves of 64 x 64 and 2 stages (64 KB of LDS, two blocks
                // per CU): prefill 2048 x 1536 -> 8960 85.2 -> 73.7 us, 4096 rows 166 -> 143 us
                // (with one or two blocks per CU the 3-stage 8-wave form stays ahead)
                if (!kInt8 && a.K % kTK == 0 && blocks(128, 128) < 256 && blocks(96, 128) <= 256)
                    linearDirect<T, 96, 128, 1, 4, 4><<<blocks(96, 128), 256, 0, s>>>(a);
                else if (!kInt8 && a.K % kTK == 0 && blocks(128, 128) >= 512)
                    linearDirect<T, 128, 128, 2, 2, 2><<<blocks(128, 128), 256, 0, s>>>(a);
                else if (!kInt8 && a.K % kTK == 0)
                    linearDirect<T, 128, 128, 4, 2, 3><<<blocks(128, 128), 512, 0, s>>>(a);
                else
                    linearTiled<T, kInt8, 128, 128, 4, 2, 2><<<blocks(128, 128), 512, 0, s>>>(a);
            } else {
                linearTiled<T, kInt8, 64, 64, 2, 2, 2><<<blocks(64, 64), 256, 0, s>>>(a);
            }
        }
        return;
    }
    const size_t n = size_t(a.M) * a.N;
    linearScalar<T, kInt8><<<unsigned((n + 255) / 256), 256, 0, s>>>(a);
}

template <bool kInt8>
void dispatch(const LinearArgs &a, llaisysDataType_t dt, hipStream_t s) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launch<F32, kInt8>(a, s);
    case LLAISYS_DTYPE_BF16: return launch<BF16, kInt8>(a, s);
    case LLAISYS_DTYPE_F16: return launch<F16, kInt8>(a, s);
    default: return;
    }
}

} // namespace

void linear(void *out, const void *x, const void *w, const float *w_scale, const void *bias,
            size_t rows, size_t in_features, size_t out_features, llaisysDataType_t dt,
            hipStream_t s) {
    const LinearArgs a{out, x, w, w_scale, bias, int(rows), int(out_features), int(in_features)};
    if (w_scale)
        dispatch<true>(a, dt, s);
    else
        dispatch<false>(a, dt, s);
}

} // namespace llaisys::kernels
