#include "types.hpp"

namespace llaisys::utils {

// Exact binary16 -> binary32 widening (subnormals become normal f32 values).
float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1F;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | (uint32_t(exp + 112) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        int e = 113; // biased f32 exponent of 2^-14
        while ((man & 0x400u) == 0) {
            man <<= 1;
            --e;
        }
        bits = sign | (uint32_t(e) << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

} // namespace llaisys::utils
