// Rotate-half RoPE for gfx950.
//
// Semantics: reference src/ops/rope/cpu/rope_cpu.cpp:28-44.  For token i, head h and
// j < d/2: freq_j = 1 / pow((double)theta, (double)(2.0f * j / d)), angle = (double)p_i *
// freq_j, and the pair (x_j, x_{j+d/2}) is rotated in double precision; the result is
// rounded double -> float -> element type.  freq_j is computed on the host with the same
// libm pow the reference calls, so the angles are bit-identical; cos/sin come from the
// device's double-precision libm.
//
// Design: HBM-bound (about 13 VALU ops per element in f64, well under the 8 TB/s
// budget).  A block owns a run of tokens; the (cos, sin) pairs of those tokens are
// computed once into LDS and reused by every head, so the f64 trig costs d/2 sincos per
// token instead of n_heads * d/2.  Each lane rotates 8 (bf16) or 4 (f32) pairs with two
// 16-byte loads and two 16-byte stores.
#include "common.hpp"
#include "launch.hpp"
#include "rowplan.hpp"

#include <algorithm>
#include <cmath>

namespace llaisys::kernels {

namespace {

constexpr int kMaxHalf = 128;     // head_dim <= 256 uses the host frequency table
constexpr int kLdsPairs = 1024;   // (cos, sin) doubles staged per block: 16 KB

struct FreqTable {
    double f[kMaxHalf];
};

__device__ __forceinline__ double freqOf(const FreqTable &ft, int j, int d, float theta) {
    if (j < kMaxHalf) return ft.f[j];
    return 1.0 / pow(double(theta), double(2.0f * float(j) / float(d)));
}

template <typename T>
__global__ void __launch_bounds__(256)
    ropeVec(void *__restrict__ out, const void *__restrict__ in, const int64_t *__restrict__ pos,
            size_t seq, int n_heads, int d, int tok_per_block, FreqTable ft) {
    using F = Fmt<T>;
    constexpr int N = F::kVec;
    __shared__ double2 cs[kLdsPairs];

    const int half = d / 2;
    const size_t t0 = size_t(blockIdx.x) * tok_per_block;
    const int ntok = int(min(size_t(tok_per_block), seq - t0));

    for (int i = threadIdx.x; i < ntok * half; i += 256) {
        const int tt = i / half, j = i - tt * half;
        const double ang = double(pos[t0 + tt]) * ft.f[j];
        double sn, c;
        sincos(ang, &sn, &c);
        cs[i] = make_double2(c, sn);
    }
    __syncthreads();

    const int vph = half / N; // vectors per half head
    const int items = ntok * n_heads * vph;
    for (int it = threadIdx.x; it < items; it += 256) {
        const int jv = it % vph;
        const int rest = it / vph;
        const int h = rest % n_heads;
        const int tt = rest / n_heads;
        const size_t base = ((t0 + tt) * size_t(n_heads) + h) * size_t(d) + size_t(jv) * N;
        float a[N], b[N], ya[N], yb[N];
        F::unpack(load16<T>(in, base), a);
        F::unpack(load16<T>(in, base + half), b);
        const double2 *row = cs + tt * half + jv * N;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const double c = row[e].x, sn = row[e].y;
            const double A = a[e], B = b[e];
            ya[e] = float(A * c - B * sn);
            yb[e] = float(B * c + A * sn);
        }
        store16<T>(out, base, F::pack(ya));
        store16<T>(out, base + half, F::pack(yb));
    }
}

// Any head_dim / alignment: one thread per (token, head, j) pair.
template <typename T>
__global__ void __launch_bounds__(256)
    ropeScalar(void *out, const void *in, const int64_t *pos, size_t seq, size_t n_heads,
               size_t d, float theta, FreqTable ft) {
    using F = Fmt<T>;
    const size_t half = d / 2;
    const size_t pairs = seq * n_heads * half;
    for (size_t k = size_t(blockIdx.x) * 256 + threadIdx.x; k < pairs;
         k += size_t(gridDim.x) * 256) {
        const size_t j = k % half;
        const size_t th = k / half; // token * n_heads + head
        const size_t tok = th / n_heads;
        const double ang = double(pos[tok]) * freqOf(ft, int(j), int(d), theta);
        double sn, c;
        sincos(ang, &sn, &c);
        const size_t base = th * d;
        const double A = F::get(in, base + j), B = F::get(in, base + j + half);
        F::put(out, base + j, float(A * c - B * sn));
        F::put(out, base + j + half, float(B * c + A * sn));
    }
}

template <typename T>
void launch(void *out, const void *in, const int64_t *pos, size_t seq, size_t nh, size_t d,
            float theta, hipStream_t s) {
    if (seq == 0 || nh == 0 || d == 0) return;
    constexpr int N = Fmt<T>::kVec;
    const size_t half = d / 2;
    FreqTable ft{};
    for (size_t j = 0; j < half && j < size_t(kMaxHalf); ++j) {
        // Same expression and libm call as rope_cpu.cpp:31.
        const float ex = 2.0f * float(j) / float(d);
        ft.f[j] = 1.0 / std::pow(double(theta), double(ex));
    }
    const bool vec = half % N == 0 && half <= size_t(kMaxHalf) && aligned16(out) && aligned16(in);
    if (vec) {
        const size_t per_tok = nh * (half / N);
        size_t tpb = std::max<size_t>(1, 1024 / per_tok);
        tpb = std::min(tpb, size_t(kLdsPairs) / half);
        tpb = std::max<size_t>(tpb, 1);
        if (tpb * per_tok <= size_t(INT32_MAX) && nh <= size_t(INT32_MAX)) {
            ropeVec<T><<<blocksFor(seq, tpb), 256, 0, s>>>(out, in, pos, seq, int(nh), int(d),
                                                           int(tpb), ft);
            return;
        }
    }
    const size_t pairs = seq * nh * half;
    const unsigned grid = unsigned(std::min<size_t>(blocksFor(pairs, 256), 65536));
    ropeScalar<T><<<grid, 256, 0, s>>>(out, in, pos, seq, nh, d, theta, ft);
}

} // namespace

void rope(void *out, const void *in, const int64_t *pos, size_t seq, size_t n_heads,
          size_t head_dim, float theta, llaisysDataType_t dt, hipStream_t s) {
    switch (dt) {
    case LLAISYS_DTYPE_F32: return launch<F32>(out, in, pos, seq, n_heads, head_dim, theta, s);
    case LLAISYS_DTYPE_BF16: return launch<BF16>(out, in, pos, seq, n_heads, head_dim, theta, s);
    case LLAISYS_DTYPE_F16: return launch<F16>(out, in, pos, seq, n_heads, head_dim, theta, s);
    default: return;
    }
}

} // namespace llaisys::kernels
