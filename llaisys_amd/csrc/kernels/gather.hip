// Embedding row gather for gfx950.
//
// Semantics: reference src/ops/embedding/cpu/embedding_cpu.cpp:16-22 -- out[i, :] =
// weight[index[i], :] byte for byte, I32 or I64 ids.  The reference throws on an id outside
// [0, vocab) (embedding_cpu.cpp:18); a kernel cannot, so the row is left untouched and 1 is
// ORed into the device error word, which the runtime's synchronize calls turn into the
// same "Embedding index out of bound" error.
//
// Design: pure copy, HBM-bound.  One wavefront per id; lanes copy the row in the widest
// unit the row size and addresses allow (16 B normally), UNROLL units in flight per lane.
// Output rows are written with non-temporal stores; table rows use ordinary loads (a
// repeated id hits the cache, and non-temporal gathers measured ~20 % slower).
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

namespace llaisys::kernels {

namespace {

constexpr int kRowsPerBlock = 4; // one wavefront per row, 256 threads
constexpr int kUnroll = 4;

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
    size_t u = lane;
    for (; u + (kUnroll - 1) * kWave < units_per_row; u += kUnroll * kWave) {
        Unit r[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) r[k] = src[u + k * kWave];
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) __builtin_nontemporal_store(r[k], dst + u + k * kWave);
    }
    for (; u < units_per_row; u += kWave) __builtin_nontemporal_store(src[u], dst + u);
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
    if ((mis & 15u) == 0) return launchUnit<v4u>(out, index, i64, n, w, vocab, row_bytes, err, s);
    if ((mis & 7u) == 0) return launchUnit<v2u>(out, index, i64, n, w, vocab, row_bytes, err, s);
    if ((mis & 3u) == 0) return launchUnit<uint32_t>(out, index, i64, n, w, vocab, row_bytes, err, s);
    if ((mis & 1u) == 0) return launchUnit<uint16_t>(out, index, i64, n, w, vocab, row_bytes, err, s);
    launchUnit<uint8_t>(out, index, i64, n, w, vocab, row_bytes, err, s);
}

} // namespace llaisys::kernels
