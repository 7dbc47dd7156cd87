// Checks the RoPE kernels' double-precision sincos (llaisys_amd/csrc/kernels/sincos.hpp,
// compiled here for the host) against glibc's sin/cos, which the reference's rope calls
// (src/ops/rope/cpu/rope_cpu.cpp:33-34).  Prints "angles ulp_differ max_ulp f32_differ".
#include "sincos.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

using llaisys::kernels::sincosReduced;

static long long ulpDist(double x, double y) {
    long long a, b;
    std::memcpy(&a, &x, 8);
    std::memcpy(&b, &y, 8);
    if (a < 0) a = (long long)(0x8000000000000000ULL - (unsigned long long)a);
    if (b < 0) b = (long long)(0x8000000000000000ULL - (unsigned long long)b);
    return a > b ? a - b : b - a;
}

int main(int argc, char **argv) {
    const int positions = argc > 1 ? std::atoi(argv[1]) : 32768;
    const float thetas[] = {10000.0f, 500000.0f, 1000000.0f};
    long long angles = 0, differ = 0, max_ulp = 0, f32_differ = 0;
    unsigned seed = 12345;
    auto next = [&] { return seed = seed * 1664525u + 1013904223u; };
    auto track = [&](double a) {
        double s, c;
        sincosReduced(a, &s, &c);
        const double gs = std::sin(a), gc = std::cos(a);
        const long long u = std::max(ulpDist(s, gs), ulpDist(c, gc));
        max_ulp = std::max(max_ulp, u);
        differ += u != 0;
        ++angles;
        // the reference's use: rotate a pair, round to float
        const float A = float(int(next() >> 8) % 2001 - 1000) / 317.0f;
        const float B = float(int(next() >> 8) % 2001 - 1000) / 291.0f;
        f32_differ += float(double(A) * c - double(B) * s) != float(double(A) * gc - double(B) * gs);
        f32_differ += float(double(B) * c + double(A) * s) != float(double(B) * gc + double(A) * gs);
    };
    for (float th : thetas)
        for (int j = 0; j < 64; ++j) {
            const double freq = 1.0 / std::pow(double(th), double(2.0f * float(j) / 128.0f));
            for (int p = 0; p < positions; ++p) track(double(p) * freq);
        }
    // random magnitudes up to the fast-path limit 2^30, both signs
    for (int i = 0; i < 200000; ++i) {
        const double a = std::ldexp(double(next()) / 4294967296.0, i % 31);
        track(i & 1 ? -a : a);
    }
    std::printf("%lld %lld %lld %lld\n", angles, differ, max_ulp, f32_differ);
    return 0;
}
