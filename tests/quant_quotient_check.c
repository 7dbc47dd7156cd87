/* Checks the arithmetic identity the INT8 kernels rely on (llaisys_amd/csrc/kernels/
 * quantize.hpp, RowQuantizer::fastCodes): for s = RN(amax / 127) >= 2^-96, r = RN(1 / s),
 * q0 = RN(x r), e = fma(-q0, s, x), q1 = fma(e, r, q0) and k = the low byte of
 * RN(q1 + 1.5 * 2^23), k equals the code clamp(rint(RN(x / s)), -127, 127) of the INT8
 * rule for every |x| <= amax.  Exhaustive over bf16 and f16 data (every amax, every x);
 * random and near-tie f32 pairs.  Prints "pairs mismatches". */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float bits_f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static uint32_t f_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float half_f(uint32_t h) {
    uint32_t s = (h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1F) return bits_f(s | 0x7F800000u | (m << 13));
    if (e) return bits_f(s | ((e + 112u) << 23) | (m << 13));
    float v = (float)m * 5.9604644775390625e-8f;
    return s ? -v : v;
}
static int ieee_code(float x, float s) {
    float t = x / s;
    if (t != t) return 0;
    t = rintf(t);
    if (t > 127.0f) t = 127.0f;
    if (t < -127.0f) t = -127.0f;
    return (int)t;
}
static int fast_code(float x, float s, float r) {
    float q0 = x * r, e = fmaf(-q0, s, x), q1 = fmaf(e, r, q0);
    if (q1 != q1) return 0;
    return (int)(int8_t)(f_bits(q1 + 12582912.0f) & 0xFFu);
}

int main(int argc, char **argv) {
    long long f32_samples = argc > 1 ? atoll(argv[1]) : 20000000;
    long long pairs = 0, bad = 0;
    for (int kind = 0; kind < 2; ++kind) {
        const int top = kind == 0 ? 0x7F80 : 0x7C00; /* first non-finite magnitude */
#pragma omp parallel for reduction(+ : pairs, bad) schedule(dynamic, 64)
        for (int ab = 1; ab < top; ++ab) {
            const float amax = kind == 0 ? bits_f((uint32_t)ab << 16) : half_f((uint32_t)ab);
            const float s = amax / 127.0f;
            if (!(s >= 0x1p-96f)) continue;
            const float r = 1.0f / s;
            for (int xb = 0; xb <= ab; ++xb)
                for (int sg = 0; sg < 2; ++sg) {
                    const float x = kind == 0 ? bits_f(((uint32_t)xb << 16) | (sg ? 0x80000000u : 0))
                                              : half_f((uint32_t)xb | (sg ? 0x8000u : 0));
                    ++pairs;
                    bad += ieee_code(x, s) != fast_code(x, s, r);
                }
        }
    }
    uint64_t st = 0x9E3779B97F4A7C15ull;
    for (long long i = 0; i < f32_samples; ++i) {
        st ^= st << 13; st ^= st >> 7; st ^= st << 17;
        float amax = bits_f((uint32_t)st & 0x7F7FFFFFu);
        st ^= st << 13; st ^= st >> 7; st ^= st << 17;
        if (i % 8 == 2) amax = ldexpf(1.0f + (float)(st >> 41) / 8388608.0f, -80 - (int)(st % 17));
        const float s = amax / 127.0f;
        if (!(s >= 0x1p-96f)) continue;
        const float r = 1.0f / s;
        float x = amax * ((float)(uint32_t)(st >> 40) / 16777216.0f) * ((st & 1) ? -1.0f : 1.0f);
        if (i % 4 == 0) x = (rintf(x / s) + 0.5f) * s;                         /* ties */
        if (i % 4 == 1) x = nextafterf((rintf(x / s) + 0.5f) * s, 0.0f);       /* near ties */
        if (!(fabsf(x) <= amax)) continue;
        ++pairs;
        bad += ieee_code(x, s) != fast_code(x, s, r);
    }
    printf("%lld %lld\n", pairs, bad);
    return 0;
}
