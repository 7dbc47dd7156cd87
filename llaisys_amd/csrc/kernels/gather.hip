// Embedding row gather for gfx950.
//
// Semantics: reference src/ops/embedding/cpu/embedding_cpu.cpp:16-22 -- out[i, :] =
// weight[index[i], :] byte for byte, I32 or I64 ids.  The reference throws on an id outside
// [0, vocab) (embedding_cpu.cpp:18); a kernel cannot, so the row is left untouched and 1 is
// ORed into the device error word, which the runtime's synchronize calls turn into the
// same "Embedding index out of bound" error.
//
// Design: pure copy, HBM-bound.  Rows of 16-byte units up to 8 KB (every config shape):
// one wavefront gathers R rows.  Lanes 0..R-1 load the R ids in one vector load, the ids are
// broadcast with v_readlane, and the wave issues the loads of all R rows (PL units per lane
// per row) before any store; for 3 KB rows (8 per wave) the stores start once all of them
// have landed, so a wave's reads and writes reach HBM as two phases rather than interleaved
// (same-box A/B, 4 runs each: 9.24-9.29 -> 9.14-9.17 us, against holding each row's stores
// only for that row's loads), and when every id is in range (the normal case) they are one
// straight run.  R rows per wave keep
// R * 3 KB in flight per wave behind a single id round trip: measured on MI355X (8192
// random ids into [151936, 1536] bf16, >= 1 GiB of rotating sets) 9.14 us with R = 8 (1024
// waves, one per SIMD), against 9.87 / 10.15 / 9.96 / 9.33 / 9.18 us with R = 4 / 6 / 10
// / 12 / 16 and 9.7 us with one row per wave and a scalar id load; a copy kernel of the
// same bytes takes 9.07 us.  Other rows: one wavefront
// per id, UNROLL units in flight per lane.  Table rows use ordinary loads (non-temporal
// gathers measured 6-7 % slower), output rows non-temporal stores.
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

namespace llaisys::kernels {

namespace {

constexpr int kRowsPerBlock = 4; // one wavefront per row, 256 threads
constexpr int kUnroll = 4;
constexpr int kMultiUnits = 24;  // R * PL: 16-byte units per lane held by the multi-row kernel

template <typename Unit, bool kI64>
__global__ void __launch_bounds__(256)
    gatherRows(void *__restrict__ out, const void *__restrict__ index, size_t n_index,
               const void *__restrict__ weight, size_t vocab, size_t units_per_row, int *err) {
    const size_t row = size_t(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (row >= n_index) return;
    const int64_t id = kI64 ? static_cast<const int64_t *>(index)[row]
                            : int64_t(static_cast<const int32_t *>(index)[row]);
    if (id < 0 || uint64_t(id) >= vocab) {
        if (lane == 0) atomicOr(err, 1);
        return;
    }
    const Unit *src = static_cast<const Unit *>(weight) + size_t(id) * units_per_row;
    Unit *dst = static_cast<Unit *>(out) + row * units_per_row;
    for (size_t u = lane; u < units_per_row; u += kUnroll * kWave) {
        Unit r[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; ++k)
            if (u + k * kWave < units_per_row) r[k] = src[u + k * kWave];
#pragma unroll
        for (int k = 0; k < kUnroll; ++k)
            if (u + k * kWave < units_per_row) __builtin_nontemporal_store(r[k], dst + u + k * kWave);
    }
}

// R rows per wavefront, PL 16-byte units per lane per row (units_per_row <= 64 * PL;
// kFull: units_per_row == 64 * PL, so no lane needs a bounds test).
template <bool kI64, int R, int PL, bool kFull>
__global__ void __launch_bounds__(kWave)
    gatherMulti(v4u *__restrict__ out, const void *__restrict__ index, size_t n_index,
                const v4u *__restrict__ weight, size_t vocab, int units_per_row, int *err) {
    const size_t row0 = size_t(blockIdx.x) * R;
    const int lane = threadIdx.x;
    const bool mine = lane < R && row0 + lane < n_index;
    const int64_t myid = !mine ? 0
                         : kI64 ? static_cast<const int64_t *>(index)[row0 + lane]
                                : int64_t(static_cast<const int32_t *>(index)[row0 + lane]);
    const uint64_t bad = __builtin_amdgcn_ballot_w64(mine && (myid < 0 || uint64_t(myid) >= vocab));
    v4u r[R][PL];
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint64_t(myid)), j));
        const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint64_t(myid) >> 32), j));
        const uint64_t id = (uint64_t(hi) << 32) | lo;
        const v4u *src = weight + (id < vocab ? id : 0) * size_t(units_per_row); // bad ids read row 0
#pragma unroll
        for (int k = 0; k < PL; ++k)
            if (kFull || lane + k * kWave < units_per_row) r[j][k] = src[lane + k * kWave];
    }
    if constexpr (PL == 3) {
        // 3 KB rows, 8 per wave: every row's loads land before the first store (the read and
        // write phases of the wave apart); the scheduling barriers keep the compiler from
        // moving loads below the wait.  Other plans measured slower with it: 8 KB rows, one
        // per wave, 42.4 -> 43.6 us ([128256, 4096] x 16384); 128 f32 rows of 6 KB, 4 per
        // wave, 2.87 -> 3.02 us.
        __builtin_amdgcn_sched_barrier(0);
        waitVmcnt<0>();
        __builtin_amdgcn_sched_barrier(0);
    }
    if (bad == 0 && row0 + R <= n_index) {
#pragma unroll
        for (int j = 0; j < R; ++j) {
            v4u *dst = out + (row0 + j) * size_t(units_per_row);
#pragma unroll
            for (int k = 0; k < PL; ++k)
                if (kFull || lane + k * kWave < units_per_row) __builtin_nontemporal_store(r[j][k], dst + lane + k * kWave);
        }
        return;
    }
    if (bad != 0 && lane == 0) atomicOr(err, 1);
#pragma unroll
    for (int j = 0; j < R; ++j) {
        if (row0 + j >= n_index || ((bad >> j) & 1)) continue; // out-of-range ids leave their row
        v4u *dst = out + (row0 + j) * size_t(units_per_row);
#pragma unroll
        for (int k = 0; k < PL; ++k)
            if (kFull || lane + k * kWave < units_per_row) __builtin_nontemporal_store(r[j][k], dst + lane + k * kWave);
    }
}

template <int PL, bool kFull>
void launchMultiAs(void *out, const void *index, bool i64, size_t n, const void *w, size_t vocab,
                   size_t units, int *err, hipStream_t s) {
    // 8 KB rows (Llama-8B): one row per wave, 42.2 us against 44.8 us with 3 rows per
    // wave (16384 random ids into [128256, 4096] bf16, >= 1 GiB of rotating sets)
    constexpr int R = PL >= 8 ? 1 : kMultiUnits / PL;
    const unsigned grid = blocksFor(n, R);
    if (i64)
        gatherMulti<true, R, PL, kFull><<<grid, kWave, 0, s>>>(static_cast<v4u *>(out), index, n,
                                                               static_cast<const v4u *>(w), vocab, int(units), err);
    else
        gatherMulti<false, R, PL, kFull><<<grid, kWave, 0, s>>>(static_cast<v4u *>(out), index, n,
                                                                static_cast<const v4u *>(w), vocab, int(units), err);
}

template <int PL>
void launchMulti(void *out, const void *index, bool i64, size_t n, const void *w, size_t vocab,
                 size_t units, int *err, hipStream_t s) {
    if (units == size_t(PL) * kWave)
        launchMultiAs<PL, true>(out, index, i64, n, w, vocab, units, err, s);
    else
        launchMultiAs<PL, false>(out, index, i64, n, w, vocab, units, err, s);
}

template <typename Unit>
void launchUnit(void *out, const void *index, bool i64, size_t n, const void *w, size_t vocab,
                size_t row_bytes, int *err, hipStream_t s) {
    const size_t units = row_bytes / sizeof(Unit);
    const unsigned grid = blocksFor(n, kRowsPerBlock);
    if (i64)
        gatherRows<Unit, true><<<grid, 256, 0, s>>>(out, index, n, w, vocab, units, err);
    else
        gatherRows<Unit, false><<<grid, 256, 0, s>>>(out, index, n, w, vocab, units, err);
}

} // namespace

void embedding(void *out, const void *index, bool i64, size_t n, const void *w, size_t vocab,
               size_t row_bytes, int *err, hipStream_t s) {
    if (n == 0) return;
    const uintptr_t mis = reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(w) |
                          uintptr_t(row_bytes);
    typedef uint32_t v2u __attribute__((ext_vector_type(2)));
    if ((mis & 15u) == 0) {
        const size_t units = row_bytes / 16;
        switch ((units + kWave - 1) / kWave) {
        case 1: return launchMulti<1>(out, index, i64, n, w, vocab, units, err, s);
        case 2: return launchMulti<2>(out, index, i64, n, w, vocab, units, err, s);
        case 3: return launchMulti<3>(out, index, i64, n, w, vocab, units, err, s);
        case 4: return launchMulti<4>(out, index, i64, n, w, vocab, units, err, s);
        case 6: return launchMulti<6>(out, index, i64, n, w, vocab, units, err, s);
        case 8: return launchMulti<8>(out, index, i64, n, w, vocab, units, err, s);
        default: return launchUnit<v4u>(out, index, i64, n, w, vocab, row_bytes, err, s);
        }
    }
    if ((mis & 7u) == 0) return launchUnit<v2u>(out, index, i64, n, w, vocab, row_bytes, err, s);
    if ((mis & 3u) == 0) return launchUnit<uint32_t>(out, index, i64, n, w, vocab, row_bytes, err, s);
    if ((mis & 1u) == 0) return launchUnit<uint16_t>(out, index, i64, n, w, vocab, row_bytes, err, s);
    launchUnit<uint8_t>(out, index, i64, n, w, vocab, row_bytes, err, s);
}

} // namespace llaisys::kernels
