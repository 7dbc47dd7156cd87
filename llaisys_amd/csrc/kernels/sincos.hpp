// Double-precision sin and cos of one angle for the RoPE kernels.
//
// Method (Cody & Waite argument reduction, Taylor polynomials):
//  * n = rint(a * 2/pi), r = a - n * pi/2 with pi/2 = P1 + P2 + P3 (three doubles, each the
//    nearest double to what remains of pi/2).  The first step fma(-n, P1, a) is exact for
//    |a| >= 1 (a and n*P1 are both multiples of 2^-52 and the difference is below 2 in
//    magnitude), the next two round once each relative to r, so r carries about 1 ulp.
//  * on |r| <= pi/4 (slightly more when n rounds the other way):
//      sin r = r + r z (-1/3! + z (1/5! - ... + z / 17!)),      z = r^2,
//      cos r = (1 - z/2) + [low part of 1 - z/2] + z^2 (1/4! - z/6! + ... + z^6/16!),
//    the Taylor series truncated where the first dropped term is below 2^-62 of the result
//    (r^19/19! < 1.3e-19 and r^18/18! < 2.1e-18 at r = pi/4 + 2^-20); the 1 - z/2 split
//    keeps the cos rounding error near half an ulp.
//  * the quadrant n mod 4 swaps and negates (sin r, cos r).
// Measured against glibc's sin/cos over every RoPE angle p * freq_j of 128 K positions,
// three thetas and 64 frequencies (25 M angles): at most 1 ulp apart.  Outside
// |a| <= 2^30 callers use the device library's sincos.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

#if defined(__HIPCC__)
#define LLAISYS_HD __host__ __device__
#else
#define LLAISYS_HD
#endif

namespace llaisys::kernels {

constexpr double kSincosFastLimit = 1073741824.0; // 2^30

LLAISYS_HD inline double flipSign(double v, bool neg) {
#if defined(__HIP_DEVICE_COMPILE__)
    // one XOR on the high word (the generic form below compiled to byte-wise masking)
    return __hiloint2double(__double2hiint(v) ^ int(uint32_t(neg) << 31), __double2loint(v));
#else
    uint32_t w[2]; // little-endian: w[1] holds the sign
    std::memcpy(w, &v, 8);
    w[1] ^= uint32_t(neg) << 31;
    std::memcpy(&v, w, 8);
    return v;
#endif
}

// fma(a, b, k) for a constant k.  On the device the constant is an SGPR operand of
// v_fma_f64: left to itself the compiler emits v_fmac_f64 and first copies each
// coefficient into the accumulator VGPR pair (two v_mov_b32 per Horner step, about a
// third of the routine's VALU instructions).  Same correctly rounded fma either way.
LLAISYS_HD inline double fmaK(double a, double b, double k) {
#if defined(__HIP_DEVICE_COMPILE__)
    double r;
    asm("v_fma_f64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(k));
    return r;
#else
    return fma(a, b, k);
#endif
}

// Valid for |a| <= kSincosFastLimit.
LLAISYS_HD inline void sincosReduced(double a, double *s_out, double *c_out) {
    constexpr double kTwoOverPi = 0x1.45f306dc9c883p-1;
    constexpr double kP1 = 0x1.921fb54442d18p+0;
    constexpr double kP2 = 0x1.1a62633145c07p-54;
    constexpr double kP3 = -0x1.f1976b7ed8fbcp-110;
    const double n = rint(a * kTwoOverPi);
    double r = fma(-n, kP1, a);
    r = fma(-n, kP2, r);
    r = fma(-n, kP3, r);
    const double z = r * r;

    // sin: 1/k! for odd k = 3 .. 17, alternating signs
    double ps = 0x1.952c77030ad4ap-49; // 1/17!
    ps = fmaK(ps, z, -0x1.ae7f3e733b81fp-41); // -1/15!
    ps = fmaK(ps, z, 0x1.6124613a86d09p-33);  // 1/13!
    ps = fmaK(ps, z, -0x1.ae64567f544e4p-26); // -1/11!
    ps = fmaK(ps, z, 0x1.71de3a556c734p-19);  // 1/9!
    ps = fmaK(ps, z, -0x1.a01a01a01a01ap-13); // -1/7!
    ps = fmaK(ps, z, 0x1.1111111111111p-7);   // 1/5!
    ps = fmaK(ps, z, -0x1.5555555555555p-3);  // -1/3!
    const double s = fma(r * z, ps, r);

    // cos: 1/k! for even k = 4 .. 16
    double pc = 0x1.ae7f3e733b81fp-45;       // 1/16!
    pc = fmaK(pc, z, -0x1.93974a8c07c9dp-37); // -1/14!
    pc = fmaK(pc, z, 0x1.1eed8eff8d898p-29);  // 1/12!
    pc = fmaK(pc, z, -0x1.27e4fb7789f5cp-22); // -1/10!
    pc = fmaK(pc, z, 0x1.a01a01a01a01ap-16);  // 1/8!
    pc = fmaK(pc, z, -0x1.6c16c16c16c17p-10); // -1/6!
    pc = fmaK(pc, z, 0x1.5555555555555p-5);   // 1/4!
    const double hz = 0.5 * z;
    const double w = 1.0 - hz;
    const double c = w + (((1.0 - w) - hz) + (z * z) * pc);

    const int32_t q = int32_t(n); // |n| <= 2^30 * 2/pi: a 32-bit conversion is exact
    const bool swap = (q & 1) != 0;
    *s_out = flipSign(swap ? c : s, (q & 2) != 0);
    *c_out = flipSign(swap ? s : c, ((q + 1) & 2) != 0);
}

} // namespace llaisys::kernels
