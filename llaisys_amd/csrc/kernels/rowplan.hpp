// Host-side choice of the lane group and registers per lane for row kernels.
//
// A row of `nvec` 16-byte vectors is owned by a group of G consecutive lanes, each lane
// holding V vectors in registers (vector k of a lane is lane + k*G, so a group's loads
// are contiguous).  The row is read from HBM once and written once.  G <= 64 reduces in
// one wavefront with butterflies; G = 256 / 1024 combines wave partials through LDS.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <type_traits>

namespace llaisys::kernels {

struct RowPlan {
    int group = 0; // 0: no register-resident plan, use the scalar kernel
    int vpl = 0;
};

inline RowPlan planRow(size_t nvec) {
    static constexpr int kGroups[] = {16, 64, 256, 1024};
    static constexpr int kMaxV[] = {2, 8, 8, 8};
    for (int k = 0; k < 4; ++k) {
        const size_t g = size_t(kGroups[k]);
        if (nvec <= g * size_t(kMaxV[k])) {
            int v = int((nvec + g - 1) / g);
            if (v == 5) v = 6;
            if (v == 7) v = 8;
            return {kGroups[k], v < 1 ? 1 : v};
        }
    }
    return {};
}

template <int G>
constexpr int blockFor() {
    return G < 256 ? 256 : G;
}

template <int G, typename F>
void withV(int v, F &&f) {
    using std::integral_constant;
    switch (v) {
    case 1: f(integral_constant<int, G>{}, integral_constant<int, 1>{}); break;
    case 2: f(integral_constant<int, G>{}, integral_constant<int, 2>{}); break;
    case 3:
        if constexpr (G > 16) f(integral_constant<int, G>{}, integral_constant<int, 3>{});
        break;
    case 4:
        if constexpr (G > 16) f(integral_constant<int, G>{}, integral_constant<int, 4>{});
        break;
    case 6:
        if constexpr (G > 16) f(integral_constant<int, G>{}, integral_constant<int, 6>{});
        break;
    case 8:
        if constexpr (G > 16) f(integral_constant<int, G>{}, integral_constant<int, 8>{});
        break;
    default: break;
    }
}

// Calls f(integral_constant<G>, integral_constant<V>) for the plan's (G, V).
template <typename F>
void withPlan(const RowPlan &p, F &&f) {
    switch (p.group) {
    case 16: withV<16>(p.vpl, f); break;
    case 64: withV<64>(p.vpl, f); break;
    case 256: withV<256>(p.vpl, f); break;
    case 1024: withV<1024>(p.vpl, f); break;
    default: break;
    }
}

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned blocksFor(size_t work, size_t per_block) {
    return unsigned((work + per_block - 1) / per_block);
}

} // namespace llaisys::kernels
