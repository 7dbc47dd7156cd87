// Strided copy between two layouts of one shape: out[i] = in[i] for every multi-index i.
//
// The reference's rearrange is a stub (src/ops/rearrange/op.cpp:4-6); its meaning is fixed by
// its signature and by Tensor::contiguous / Tensor::to (src/tensor/tensor.hpp:55-57), which
// need exactly this copy.  Bytes only -- no arithmetic -- so results are bit-exact.
//
// Host side: size-1 dimensions are dropped and neighbours that are contiguous in both
// layouts are merged, so most copies reach one of three kernels:
//  - rowCopy:   the innermost dimension is contiguous in both layouts: rows of R bytes are
//               copied in the widest unit (16 / 8 / 4 / 2 / 1 B) that divides R and the
//               base addresses; HBM-bound, 1 read + 1 write per byte.
//  - tileCopy128 / tileCopyVec / tileCopy: the output's contiguous dimension is strided in
//               the input, and another dimension is contiguous there (a transpose): tiles
//               through LDS, both sides coalesced, in 16-byte vectors when the shape and
//               alignment allow (128 x 128 tiles for 2-byte elements), else 32 x 32 elements
//               one per thread; HBM-bound.
//  - gatherCopy: anything else, one thread per element.
#include "common.hpp"
#include "launch.hpp"

#include <algorithm>
#include <cstring>
#include <type_traits>

namespace llaisys::kernels {

namespace {

constexpr int kMaxDims = 8;

struct Dims {
    int nd;
    int64_t shape[kMaxDims];
    int64_t sin[kMaxDims];  // element strides
    int64_t sout[kMaxDims];
};

// offsets of linear index `idx` over the first nd dims (row-major over `shape`)
__device__ __forceinline__ void offsets(const Dims &d, int nd, int64_t idx, int64_t &oi, int64_t &oo) {
    oi = 0;
    oo = 0;
    for (int k = nd - 1; k >= 0; --k) {
        const int64_t c = idx % d.shape[k];
        idx /= d.shape[k];
        oi += c * d.sin[k];
        oo += c * d.sout[k];
    }
}

// the offsets of `offsets` in 32-bit index arithmetic (every extent and the index < 2^32)
__device__ __forceinline__ void offsets32(const Dims &d, int nd, uint32_t idx, int64_t &oi, int64_t &oo) {
    oi = 0;
    oo = 0;
    for (int k = nd - 1; k >= 0; --k) {
        const uint32_t sh = uint32_t(d.shape[k]);
        const uint32_t c = idx % sh;
        idx /= sh;
        oi += int64_t(c) * d.sin[k];
        oo += int64_t(c) * d.sout[k];
    }
}

template <typename U, bool k32>
__global__ void __launch_bounds__(256)
    rowCopy(char *out, const char *in, Dims d, int64_t rows, int64_t units, int esize) {
    // d covers the outer dims (the row index); a row is `units` units of U, contiguous in both.
    // k32: rows * units < 2^31, so the index arithmetic runs in 32 bits (64-bit division is
    // a long instruction sequence on the GPU)
    const int64_t total = rows * units;
    for (int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x; t < total; t += int64_t(gridDim.x) * 256) {
        int64_t r, u, oi, oo;
        if constexpr (k32) {
            const uint32_t t32 = uint32_t(t), un = uint32_t(units);
            r = int64_t(t32 / un);
            u = int64_t(t32 % un);
            offsets32(d, d.nd, uint32_t(r), oi, oo);
        } else {
            r = t / units;
            u = t % units;
            offsets(d, d.nd, r, oi, oo);
        }
        __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const U *>(in + oi * esize) + u),
                                    reinterpret_cast<U *>(out + oo * esize) + u);
    }
}

// dims p (input-contiguous) and q (output-contiguous) tiled 32 x 32; the other dims of d
// (without p and q) index blockIdx.z
template <typename E>
__global__ void __launch_bounds__(256)
    tileCopy(E *out, const E *in, Dims rest, int64_t np, int64_t nq, int64_t sp_out, int64_t sq_in) {
    __shared__ E tile[32][33];
    int64_t oi, oo;
    offsets(rest, rest.nd, blockIdx.z, oi, oo);
    const int64_t p0 = int64_t(blockIdx.x) * 32, q0 = int64_t(blockIdx.y) * 32;
    const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;
    // read: consecutive threads walk p (contiguous in the input)
#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const int64_t p = p0 + tx, q = q0 + ty + k;
        if (p < np && q < nq) tile[ty + k][tx] = in[oi + p + q * sq_in];
    }
    __syncthreads();
    // write: consecutive threads walk q (contiguous in the output)
#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const int64_t q = q0 + tx, p = p0 + ty + k;
        if (p < np && q < nq) out[oo + q + p * sp_out] = tile[tx][ty + k];
    }
}

// The same transpose in 16-byte vectors on both sides, for 1-, 2- and 4-byte elements when
// np, nq, the strides and the bases keep every vector whole and aligned: a T x T tile (T =
// 64 for 1- and 2-byte elements, 32 for 4-byte) is read as rows of the input (p
// contiguous), held in LDS as tile[q][p], and written as rows of the output (q contiguous),
// each output vector gathered from VE LDS elements of one column.  Per byte moved, a
// sixteenth of the memory instructions of the element-wise tile.
template <typename E>
__global__ void __launch_bounds__(256)
    tileCopyVec(E *out, const E *in, Dims rest, int64_t np, int64_t nq, int64_t sp_out, int64_t sq_in) {
    constexpr int VE = 16 / int(sizeof(E));             // elements per vector
    constexpr int T = sizeof(E) == 4 ? 32 : 64;         // tile edge (elements)
    constexpr int VR = T / VE;                          // vectors per tile row
    constexpr int PAD = sizeof(E) == 4 ? 1 : (sizeof(E) == 2 ? 2 : 4); // 4 bytes: rows shift one bank
    __shared__ E tile[T][T + PAD];
    int64_t oi, oo;
    offsets(rest, rest.nd, blockIdx.z, oi, oo);
    const int64_t p0 = int64_t(blockIdx.x) * T, q0 = int64_t(blockIdx.y) * T;
#pragma unroll
    for (int k = threadIdx.x; k < T * VR; k += 256) {
        const int r = k / VR, v = k % VR; // tile row r = q offset, vector v along p
        const int64_t q = q0 + r, p = p0 + int64_t(v) * VE;
        if (q < nq && p < np) {
            const v4u x = *reinterpret_cast<const v4u *>(in + oi + p + q * sq_in);
            E e[VE];
            __builtin_memcpy(e, &x, 16);
#pragma unroll
            for (int j = 0; j < VE; ++j) tile[r][v * VE + j] = e[j];
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = threadIdx.x; k < T * VR; k += 256) {
        const int r = k / VR, v = k % VR; // output row r = p offset, vector v along q
        const int64_t p = p0 + r, q = q0 + int64_t(v) * VE;
        if (p < np && q < nq) {
            E e[VE];
#pragma unroll
            for (int j = 0; j < VE; ++j) e[j] = tile[v * VE + j][r];
            v4u x;
            __builtin_memcpy(&x, e, 16);
            *reinterpret_cast<v4u *>(out + oo + q + p * sp_out) = x;
        }
    }
}

// 2-byte elements, 16-byte vectors on both sides: 128 x 128 tiles (8 vectors per thread in
// flight), loads unconditional (clamped at ragged edges) and non-temporal, the tile written
// as 16-byte rows with chunk c of row r at c ^ ((r / 8) % 16) so that the transposed 2-byte
// reads of rows 8 apart fall in different banks, and the blocks ordered with the output's
// contiguous dimension fastest.  Measured on MI355X (8192 x 8192 bf16, rotating sets):
// 56.8 us against 62.6 us for tileCopyVec's 64 x 64 tiles (59.8 us with the input's
// contiguous dimension fastest; 63.5 us with padded rows instead of the swizzle).
__global__ void __launch_bounds__(256)
    tileCopy128(uint16_t *out, const uint16_t *in, Dims rest, int64_t np, int64_t nq, int64_t sp_out,
                int64_t sq_in) {
    constexpr int VE = 8, T = 128, VR = T / VE, NV = T * VR / 256;
    __shared__ __align__(16) uint16_t tile[T * T];
    int64_t oi, oo;
    offsets(rest, rest.nd, blockIdx.z, oi, oo);
    const int64_t q0 = int64_t(blockIdx.x) * T, p0 = int64_t(blockIdx.y) * T;
    v4u x[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) { // tile row r = q offset, vector v along p
        const int k = int(threadIdx.x) + 256 * i, r = k / VR, v = k % VR;
        const int64_t q = min(q0 + r, nq - 1), p = min(p0 + int64_t(v) * VE, np - VE);
        x[i] = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(in + oi + p + q * sq_in));
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int k = int(threadIdx.x) + 256 * i, r = k / VR, v = k % VR;
        *reinterpret_cast<v4u *>(&tile[r * T + (v ^ ((r >> 3) & (VR - 1))) * VE]) = x[i];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NV; ++i) { // output row p0 + r, vector v along q
        const int k = int(threadIdx.x) + 256 * i, r = k / VR, v = k % VR;
        uint16_t e[VE];
#pragma unroll
        for (int j = 0; j < VE; ++j) {
            const int row = v * VE + j;
            e[j] = tile[row * T + ((r / VE) ^ ((row >> 3) & (VR - 1))) * VE + r % VE];
        }
        const int64_t p = p0 + r, q = q0 + int64_t(v) * VE;
        v4u y;
        __builtin_memcpy(&y, e, 16);
        if (p < np && q < nq) __builtin_nontemporal_store(y, reinterpret_cast<v4u *>(out + oo + q + p * sp_out));
    }
}

template <typename E>
__global__ void __launch_bounds__(256)
    gatherCopy(E *out, const E *in, Dims d, int64_t n) {
    for (int64_t t = int64_t(blockIdx.x) * 256 + threadIdx.x; t < n; t += int64_t(gridDim.x) * 256) {
        int64_t oi, oo;
        offsets(d, d.nd, t, oi, oo);
        out[oo] = in[oi];
    }
}

unsigned gridFor(int64_t work) {
    return unsigned(std::min<int64_t>((work + 255) / 256, int64_t(256) * 64));
}

} // namespace

void rearrange(void *out, const void *in, size_t ndim, const size_t *shape, const ptrdiff_t *in_strides,
               const ptrdiff_t *out_strides, size_t esize, hipStream_t s) {
    // drop size-1 dims, then merge neighbours contiguous in both layouts
    Dims d{};
    int64_t n = 1;
    for (size_t k = 0; k < ndim; ++k) {
        n *= int64_t(shape[k]);
        if (shape[k] == 1) continue;
        const int64_t sh = int64_t(shape[k]), si = in_strides[k], so = out_strides[k];
        if (d.nd > 0 && d.sin[d.nd - 1] == sh * si && d.sout[d.nd - 1] == sh * so) {
            d.shape[d.nd - 1] *= sh;
            d.sin[d.nd - 1] = si;
            d.sout[d.nd - 1] = so;
        } else {
            d.shape[d.nd] = sh;
            d.sin[d.nd] = si;
            d.sout[d.nd] = so;
            ++d.nd;
        }
    }
    if (n == 0) return;
    char *o = static_cast<char *>(out);
    const char *i = static_cast<const char *>(in);
    if (d.nd == 0) { // one element
        d.nd = 1;
        d.shape[0] = 1;
        d.sin[0] = d.sout[0] = 1;
    }
    const int last = d.nd - 1;
    if (d.sin[last] == 1 && d.sout[last] == 1) {
        // rows: the innermost dim is contiguous in both
        const int64_t rowBytes = d.shape[last] * int64_t(esize);
        Dims outer = d;
        outer.nd = last;
        const int64_t rows = n / d.shape[last];
        int ub = 16;
        const auto fits = [&](int b) {
            if (rowBytes % b) return false;
            if ((reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(i)) % b) return false;
            for (int k = 0; k < outer.nd; ++k)
                if ((outer.sin[k] * int64_t(esize)) % b || (outer.sout[k] * int64_t(esize)) % b) return false;
            return true;
        };
        while (ub > 1 && !fits(ub)) ub /= 2;
        const int64_t units = rowBytes / ub;
        const unsigned g = gridFor(rows * units);
        const auto go = [&](auto k32) {
            constexpr bool K = decltype(k32)::value;
            switch (ub) {
            case 16: rowCopy<v4u, K><<<g, 256, 0, s>>>(o, i, outer, rows, units, int(esize)); break;
            case 8: rowCopy<uint64_t, K><<<g, 256, 0, s>>>(o, i, outer, rows, units, int(esize)); break;
            case 4: rowCopy<uint32_t, K><<<g, 256, 0, s>>>(o, i, outer, rows, units, int(esize)); break;
            case 2: rowCopy<uint16_t, K><<<g, 256, 0, s>>>(o, i, outer, rows, units, int(esize)); break;
            default: rowCopy<uint8_t, K><<<g, 256, 0, s>>>(o, i, outer, rows, units, int(esize)); break;
            }
        };
        // (the grid-stride index stays below total + grid * 256 <= total + 2^22)
        if (rows * units < (int64_t(1) << 31) - (int64_t(1) << 23))
            go(std::true_type{});
        else
            go(std::false_type{});
        return;
    }
    // transpose: output contiguous in dim q = last, input contiguous in some dim p != q
    int p = -1;
    for (int k = 0; k < last; ++k)
        if (d.sin[k] == 1) p = k;
    if (d.sout[last] == 1 && p >= 0 && (esize == 1 || esize == 2 || esize == 4 || esize == 8)) {
        Dims rest{};
        int64_t nz = 1;
        for (int k = 0; k < last; ++k) {
            if (k == p) continue;
            rest.shape[rest.nd] = d.shape[k];
            rest.sin[rest.nd] = d.sin[k];
            rest.sout[rest.nd] = d.sout[k];
            ++rest.nd;
            nz *= d.shape[k];
        }
        const int64_t np = d.shape[p], nq = d.shape[last], spo = d.sout[p], sqi = d.sin[last];
        // 16-byte vectors on both sides: every vector whole (np, nq multiples of its element
        // count) and aligned (bases, strides and the other dims' offsets)
        const int64_t ve = esize <= 4 ? 16 / int64_t(esize) : 0;
        bool vec = ve > 0 && np % ve == 0 && nq % ve == 0 && spo % ve == 0 && sqi % ve == 0 &&
                   (reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(i)) % 16 == 0;
        for (int k = 0; vec && k < rest.nd; ++k) vec = rest.sin[k] % ve == 0 && rest.sout[k] % ve == 0;
        const int64_t tv = esize == 4 ? 32 : 64;
        if (vec && esize == 2 && nz <= 65535 && (np + 127) / 128 <= 65535) {
            const dim3 grid(unsigned((nq + 127) / 128), unsigned((np + 127) / 128), unsigned(nz));
            tileCopy128<<<grid, 256, 0, s>>>(reinterpret_cast<uint16_t *>(o), reinterpret_cast<const uint16_t *>(i), rest,
                                            np, nq, spo, sqi);
            return;
        }
        if (vec && nz <= 65535 && (nq + tv - 1) / tv <= 65535) {
            const dim3 grid(unsigned((np + tv - 1) / tv), unsigned((nq + tv - 1) / tv), unsigned(nz));
            switch (esize) {
            case 1: tileCopyVec<uint8_t><<<grid, 256, 0, s>>>(reinterpret_cast<uint8_t *>(o), reinterpret_cast<const uint8_t *>(i), rest, np, nq, spo, sqi); break;
            case 2: tileCopyVec<uint16_t><<<grid, 256, 0, s>>>(reinterpret_cast<uint16_t *>(o), reinterpret_cast<const uint16_t *>(i), rest, np, nq, spo, sqi); break;
            default: tileCopyVec<uint32_t><<<grid, 256, 0, s>>>(reinterpret_cast<uint32_t *>(o), reinterpret_cast<const uint32_t *>(i), rest, np, nq, spo, sqi); break;
            }
            return;
        }
        if (nz <= 65535) {
            const dim3 grid(unsigned((d.shape[p] + 31) / 32), unsigned((d.shape[last] + 31) / 32), unsigned(nz));
            if (grid.y <= 65535) {
                switch (esize) {
                case 1: tileCopy<uint8_t><<<grid, 256, 0, s>>>(reinterpret_cast<uint8_t *>(o), reinterpret_cast<const uint8_t *>(i), rest, np, nq, spo, sqi); break;
                case 2: tileCopy<uint16_t><<<grid, 256, 0, s>>>(reinterpret_cast<uint16_t *>(o), reinterpret_cast<const uint16_t *>(i), rest, np, nq, spo, sqi); break;
                case 4: tileCopy<uint32_t><<<grid, 256, 0, s>>>(reinterpret_cast<uint32_t *>(o), reinterpret_cast<const uint32_t *>(i), rest, np, nq, spo, sqi); break;
                default: tileCopy<uint64_t><<<grid, 256, 0, s>>>(reinterpret_cast<uint64_t *>(o), reinterpret_cast<const uint64_t *>(i), rest, np, nq, spo, sqi); break;
                }
                return;
            }
        }
    }
    const unsigned g = gridFor(n);
    switch (esize) {
    case 1: gatherCopy<uint8_t><<<g, 256, 0, s>>>(reinterpret_cast<uint8_t *>(o), reinterpret_cast<const uint8_t *>(i), d, n); break;
    case 2: gatherCopy<uint16_t><<<g, 256, 0, s>>>(reinterpret_cast<uint16_t *>(o), reinterpret_cast<const uint16_t *>(i), d, n); break;
    case 4: gatherCopy<uint32_t><<<g, 256, 0, s>>>(reinterpret_cast<uint32_t *>(o), reinterpret_cast<const uint32_t *>(i), d, n); break;
    case 8: gatherCopy<uint64_t><<<g, 256, 0, s>>>(reinterpret_cast<uint64_t *>(o), reinterpret_cast<const uint64_t *>(i), d, n); break;
    default: break; // element sizes are 1, 2, 4 or 8 bytes
    }
}

} // namespace llaisys::kernels
