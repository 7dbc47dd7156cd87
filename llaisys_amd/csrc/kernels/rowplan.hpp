// Host-side choice of the lane group and registers per lane for row kernels.
//
// A row of `nvec` 16-byte vectors is owned by a group of G consecutive lanes; each lane
// holds up to VMAX of the row's vectors in registers (vector k of a lane is lane + k*G, so
// every load instruction of a group covers G*16 contiguous bytes).  The row is read from
// HBM once and written once.  G <= 64 reduces inside one wavefront with butterflies;
// G = 256 / 1024 joins the wave partials through LDS.
//
// Measured on MI355X (interleaved medians, bf16 rows of 1536 / 4096 at 2-16K rows): up to
// 4 vectors per lane with a wider group beats fewer, fatter lanes (rms_norm 8192x1536:
// 8.9 us with 64 lanes x 3 vectors vs 10.0 us with 16 lanes x 12; 16384x4096: 44.8 us with
// 256 lanes x 2 vs 46.3 us with 64 x 8), so the plan takes the smallest group that keeps
// each lane at <= 4 vectors -- up to 256 lanes.  A 1024-lane group (one row per block,
// 16 waves joined through LDS) comes last: INT8 quantize of 1536x8960 ran 8.8 us with
// 256 lanes x 5 vectors against 11.1 us with 1024 x 2.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <type_traits>

namespace llaisys::kernels {

struct RowPlan {
    int group = 0; // 0: no register-resident plan, use the scalar kernel
    int vmax = 0;
};

constexpr int kRowGroups[] = {4, 16, 32, 64, 256, 1024};
constexpr int kRowVmax[] = {4, 8};

inline RowPlan planRow(size_t nvec) {
    // Short rows (a 128-wide KV head) still get 16 lanes, so one load instruction of a
    // group covers 256 contiguous bytes instead of 64.
    const size_t min_g = nvec < 16 ? nvec : 16;
    const auto fits = [&](int g, int v) {
        return size_t(g) >= min_g && (nvec + size_t(g) - 1) / size_t(g) <= size_t(v);
    };
    for (int v : kRowVmax)
        for (int g : kRowGroups)
            if (g <= 256 && fits(g, v)) return {g, v};
    for (int v : kRowVmax)
        if (fits(1024, v)) return {1024, v};
    return {};
}

template <int G>
constexpr int blockFor() {
    // wider groups: one row per block; rows of <= 64 lanes four to a block (one-wavefront
    // blocks measured slower: config-1 rms_norm 8.62 -> 8.69 us, add + rms_norm 17.05 ->
    // 17.22 us)
    return G <= 64 ? 256 : G;
}

// Calls f(integral_constant<G>, integral_constant<VMAX>) for the plan.
template <int G, typename F>
void withVmax(int v, F &&f) {
    using std::integral_constant;
    switch (v) {
    case 4: f(integral_constant<int, G>{}, integral_constant<int, 4>{}); break;
    case 8: f(integral_constant<int, G>{}, integral_constant<int, 8>{}); break;
    default: break;
    }
}

template <typename F>
void withPlan(const RowPlan &p, F &&f) {
    switch (p.group) {
    case 4: withVmax<4>(p.vmax, f); break;
    case 16: withVmax<16>(p.vmax, f); break;
    case 32: withVmax<32>(p.vmax, f); break;
    case 64: withVmax<64>(p.vmax, f); break;
    case 256: withVmax<256>(p.vmax, f); break;
    case 1024: withVmax<1024>(p.vmax, f); break;
    default: break;
    }
}

// Unsigned division by a launch constant d >= 1 without a divide sequence: with
// m = ceil(2^64 / d) = (2^64 + e) / d, 0 <= e < d, floor(i * m / 2^64) = floor(i / d)
// whenever i * e < 2^64, which holds for every i < 2^64 / d (any index into a buffer).
struct DivU64 {
    uint64_t m = 0; // 0 encodes d == 1
    DivU64() = default;
    explicit DivU64(uint64_t d) : m(d <= 1 ? 0 : ~uint64_t(0) / d + 1) {}
    __device__ uint64_t div(uint64_t i) const { return m == 0 ? i : __umul64hi(i, m); }
};

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned blocksFor(size_t work, size_t per_block) {
    return unsigned((work + per_block - 1) / per_block);
}

} // namespace llaisys::kernels
