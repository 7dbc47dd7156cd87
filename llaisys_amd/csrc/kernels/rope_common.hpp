// Pieces shared by the RoPE kernels (rope.hip, rope_kv.hip): the host-side frequency table
// and the cross-lane partner exchange.
#pragma once

#include "common.hpp"

#include <cmath>
#include <cstddef>

namespace llaisys::kernels::rope_detail {

constexpr int kMaxHalf = 128;   // head_dim <= 256 uses the host frequency table
constexpr int kLdsPairs = 1024; // (cos, sin) doubles staged per block: 16 KB

struct FreqTable {
    double f[kMaxHalf];
};

__device__ __forceinline__ double freqOf(const FreqTable &ft, int j, int d, float theta) {
    if (j < kMaxHalf) return ft.f[j];
    return 1.0 / pow(double(theta), double(2.0f * float(j) / float(d)));
}

// Partner exchange: the vector VPH lanes away.  For VPH = 8 (bf16 / f16 with head_dim 128)
// the partner is in the same 16-lane DPP row, rotated by 8 (= lane ^ 8): a DPP move,
// no LDS traffic.  Other widths use a cross-lane shuffle.
template <int VPH>
__device__ __forceinline__ uint32_t partnerOf(uint32_t v) {
    if constexpr (VPH == 8)
        return uint32_t(__builtin_amdgcn_mov_dpp(int(v), 0x128 /* row_ror:8 */, 0xF, 0xF, false));
    else
        return uint32_t(__shfl_xor(int(v), VPH, kWave));
}

inline FreqTable hostFreqs(size_t d, float theta) {
    FreqTable ft{};
    for (size_t j = 0; j < d / 2 && j < size_t(kMaxHalf); ++j) {
        // Same expression and libm call as rope_cpu.cpp:31.
        const float ex = 2.0f * float(j) / float(d);
        ft.f[j] = 1.0 / std::pow(double(theta), double(ex));
    }
    return ft;
}

} // namespace llaisys::kernels::rope_detail
