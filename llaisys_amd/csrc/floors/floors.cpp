// Copy-kernel floors for the per-layer ops (bench.py --floors runs this program).
//
// For each op the floor is the fastest of a few plain streaming kernels that move the op's
// exact HBM traffic (the same bytes read and written, 16-byte non-temporal accesses; 1, 2,
// 3 or 4 vectors per lane, blocks of 64 or 256 threads) with no arithmetic.  It is what the op's bytes cost on this GPU
// before any of the op's own work: an op at its floor can only get faster by moving fewer
// bytes.  Each case is timed over >= 1 GiB of rotating buffer sets, as back-to-back
// launches captured in one HIP graph (the way the config-4 chain runs), median of 9
// replays of 64 launches.  The config-4 chain floor replays the chain's 113 dependent
// launches (28 layers of add+rms_norm, RoPE + INT8 KV append, add+rms_norm, swiglu; then
// rms_norm and the row argmax) with each op replaced by a copy kernel of its traffic (one
// vector per lane, 256-thread blocks).
//
// Output: one JSON object {"case": us, ...} on stdout.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <vector>

namespace {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

void check(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        std::fprintf(stderr, "floors: %s: %s\n", what, hipGetErrorString(e));
        std::exit(1);
    }
}

// NR inputs, NW outputs of n vectors each (NW <= NR): out_j[i] = in_j[i] (^ in_{j+NW}[i]);
// U vectors per lane (all loads before any store), blocks of B threads
template <int NR, int NW, int U, int B>
__global__ void __launch_bounds__(B) stream(v4u *const *outs, const v4u *const *ins, size_t n) {
    const size_t first = size_t(blockIdx.x) * B * U + threadIdx.x;
    v4u r[U][NR];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = first + size_t(u) * B;
        if (i < n)
#pragma unroll
            for (int j = 0; j < NR; ++j) r[u][j] = __builtin_nontemporal_load(ins[j] + i);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const size_t i = first + size_t(u) * B;
        if (i >= n) continue;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            v4u v = r[u][j];
#pragma unroll
            for (int k = j + NW; k < NR; k += NW) v ^= r[u][k];
            __builtin_nontemporal_store(v, outs[j] + i);
        }
    }
}

// read 8 bytes, write 16, two vectors per lane 64 apart in 64-thread blocks: every store
// instruction writes one contiguous 1 KB (the INT8 dequantize layout)
__global__ void __launch_bounds__(64) stream12x2(v4u *out, const v2u *in, size_t n8) {
    const size_t v0 = size_t(blockIdx.x) * 128 + threadIdx.x, v1 = v0 + 64;
    const v2u a = __builtin_nontemporal_load(in + (v0 < n8 ? v0 : 0));
    const v2u b = __builtin_nontemporal_load(in + (v1 < n8 ? v1 : 0));
    if (v0 < n8) __builtin_nontemporal_store(v4u{a.x, a.y, a.x, a.y}, out + v0);
    if (v1 < n8) __builtin_nontemporal_store(v4u{b.x, b.y, b.x, b.y}, out + v1);
}

// read one vector, write two (a write-heavy stream: INT8 dequantize, 1 B in -> 2 B out)
__global__ void __launch_bounds__(256) stream12(v4u *out, const v4u *in, size_t n) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const v4u a = __builtin_nontemporal_load(in + i);
    __builtin_nontemporal_store(a, out + 2 * i);
    __builtin_nontemporal_store(a, out + 2 * i + 1);
}

// read only (argmax): a never-true compare keeps the loads
__global__ void __launch_bounds__(256) readOnly(const v4u *in, size_t n, v4u *sink) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const v4u a = __builtin_nontemporal_load(in + i);
    if (a.x == 0x12345678u && a.y == 0x9abcdef0u && a.z == 0x0fedcba9u) sink[0] = a;
}

// RoPE + INT8 KV append traffic: q copied, k and v read 16 B per lane and written as 8 B of
// codes, one f32 scale per 16 lanes
__global__ void __launch_bounds__(256) ropeKv(v4u *qo, const v4u *q, const v4u *k, const v4u *v, v2u *kc,
                                              v2u *vc, float *ks, float *vs, size_t nq, size_t nkv) {
    size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < nq) {
        __builtin_nontemporal_store(__builtin_nontemporal_load(q + i), qo + i);
        return;
    }
    i -= nq;
    const bool isk = i < nkv;
    if (!isk) i -= nkv;
    if (i >= nkv) return;
    const v4u a = __builtin_nontemporal_load((isk ? k : v) + i);
    __builtin_nontemporal_store(v2u{a.x ^ a.y, a.z ^ a.w}, (isk ? kc : vc) + i);
    if ((i & 15) == 0) (isk ? ks : vs)[i / 16] = __builtin_bit_cast(float, a.x);
}

unsigned blocks(size_t n) { return unsigned((n + 255) / 256); }

// device arrays of pointers (kernel arguments for stream<>)
struct PtrSet {
    v4u **d_outs = nullptr;
    const v4u **d_ins = nullptr;
};

struct Bench {
    hipStream_t s{};
    std::vector<void *> owned;
    void *alloc(size_t bytes) {
        void *p = nullptr;
        check(hipMalloc(&p, bytes), "hipMalloc");
        check(hipMemset(p, 0, bytes), "hipMemset");
        owned.push_back(p);
        return p;
    }
    void freeAll() {
        for (void *p : owned) (void)hipFree(p);
        owned.clear();
    }
    // sets of `bytes_per_set` so that the rotation covers >= 1 GiB (at least 2 sets)
    static int setsFor(size_t bytes_per_set) {
        return int(std::max<size_t>(2, std::min<size_t>(256, ((size_t(1) << 30) + bytes_per_set - 1) / bytes_per_set)));
    }
    // median us per call of fn(set), `per` calls per graph replay
    double time(int nsets, const std::function<void(int)> &fn, int per = 64) {
        for (int i = 0; i < 4; ++i) fn(i % nsets);
        hipGraph_t g;
        hipGraphExec_t ge;
        check(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal), "capture");
        for (int i = 0; i < per; ++i) fn(i % nsets);
        check(hipStreamEndCapture(s, &g), "end capture");
        check(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "instantiate");
        check(hipGraphLaunch(ge, s), "launch");
        check(hipStreamSynchronize(s), "sync");
        hipEvent_t a, b;
        check(hipEventCreate(&a), "event");
        check(hipEventCreate(&b), "event");
        std::vector<float> v;
        for (int r = 0; r < 9; ++r) {
            check(hipEventRecord(a, s), "record");
            check(hipGraphLaunch(ge, s), "launch");
            check(hipEventRecord(b, s), "record");
            check(hipEventSynchronize(b), "sync");
            float ms = 0.0f;
            check(hipEventElapsedTime(&ms, a, b), "elapsed");
            v.push_back(ms * 1e3f / per);
        }
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
        (void)hipGraphExecDestroy(ge);
        (void)hipGraphDestroy(g);
        std::sort(v.begin(), v.end());
        return v[v.size() / 2];
    }
    // fastest stream<NR, NW, U, B> over the shapes below, NR inputs / NW outputs of `bytes` each
    template <int NR, int NW>
    double streamFloor(size_t bytes) {
        const size_t n = bytes / 16;
        const int sets = setsFor(bytes * (NR + NW));
        std::vector<PtrSet> ps(sets);
        for (auto &p : ps) {
            v4u *outs[NW];
            const v4u *ins[NR];
            for (int j = 0; j < NW; ++j) outs[j] = static_cast<v4u *>(alloc(bytes));
            for (int j = 0; j < NR; ++j) ins[j] = static_cast<v4u *>(alloc(bytes));
            p.d_outs = static_cast<v4u **>(alloc(sizeof(outs)));
            p.d_ins = static_cast<const v4u **>(alloc(sizeof(ins)));
            check(hipMemcpy(p.d_outs, outs, sizeof(outs), hipMemcpyHostToDevice), "copy");
            check(hipMemcpy(p.d_ins, ins, sizeof(ins), hipMemcpyHostToDevice), "copy");
        }
        const auto shape = [&](auto u, auto b) {
            constexpr int U = decltype(u)::value, Bk = decltype(b)::value;
            const unsigned grid = unsigned((n + size_t(Bk) * U - 1) / (size_t(Bk) * U));
            return time(sets, [&](int i) { stream<NR, NW, U, Bk><<<grid, Bk, 0, s>>>(ps[i].d_outs, ps[i].d_ins, n); });
        };
        using std::integral_constant;
        double best = shape(integral_constant<int, 1>{}, integral_constant<int, 256>{});
        best = std::min(best, shape(integral_constant<int, 2>{}, integral_constant<int, 256>{}));
        best = std::min(best, shape(integral_constant<int, 4>{}, integral_constant<int, 256>{}));
        best = std::min(best, shape(integral_constant<int, 1>{}, integral_constant<int, 64>{}));
        best = std::min(best, shape(integral_constant<int, 3>{}, integral_constant<int, 64>{}));
        freeAll();
        return best;
    }
    double stream12Floor(size_t in_bytes) {
        const size_t n = in_bytes / 16;
        const int sets = setsFor(in_bytes * 3);
        std::vector<std::pair<v4u *, v4u *>> io(sets);
        for (auto &p : io) p = {static_cast<v4u *>(alloc(2 * in_bytes)), static_cast<v4u *>(alloc(in_bytes))};
        const size_t n8 = in_bytes / 8;
        const double us = std::min(
            time(sets, [&](int i) { stream12<<<blocks(n), 256, 0, s>>>(io[i].first, io[i].second, n); }),
            time(sets, [&](int i) {
                stream12x2<<<unsigned((n8 + 127) / 128), 64, 0, s>>>(io[i].first, reinterpret_cast<const v2u *>(io[i].second), n8);
            }));
        freeAll();
        return us;
    }
    double ropeKvFloor(size_t T) {
        const size_t qb = T * 12 * 128 * 2, kb = T * 2 * 128 * 2;
        const int sets = setsFor(2 * qb + 3 * kb);
        struct S { v4u *q, *k, *v, *qo; v2u *kc, *vc; float *ks, *vs; };
        std::vector<S> ss(sets);
        for (auto &x : ss) {
            x.q = static_cast<v4u *>(alloc(qb)), x.qo = static_cast<v4u *>(alloc(qb));
            x.k = static_cast<v4u *>(alloc(kb)), x.v = static_cast<v4u *>(alloc(kb));
            x.kc = static_cast<v2u *>(alloc(kb / 2)), x.vc = static_cast<v2u *>(alloc(kb / 2));
            x.ks = static_cast<float *>(alloc(T * 8)), x.vs = static_cast<float *>(alloc(T * 8));
        }
        const double us = time(sets, [&](int i) {
            const S &x = ss[i];
            ropeKv<<<blocks((qb + 2 * kb) / 16), 256, 0, s>>>(x.qo, x.q, x.k, x.v, x.kc, x.vc, x.ks, x.vs, qb / 16, kb / 16);
        });
        freeAll();
        return us;
    }
    double readFloor(size_t bytes) {
        const size_t n = bytes / 16;
        const int sets = setsFor(bytes);
        std::vector<v4u *> in(sets);
        for (auto &p : in) p = static_cast<v4u *>(alloc(bytes));
        v4u *sink = static_cast<v4u *>(alloc(64));
        const double us = time(sets, [&](int i) { readOnly<<<blocks(n), 256, 0, s>>>(in[i], n, sink); });
        freeAll();
        return us;
    }
};

// the config-4 chain with every op replaced by its copy kernel, as one graph; median ms
double chainFloor(Bench &B) {
    const size_t T = 2048, H = 1536, I = 8960, V = 151936;
    const size_t hb = T * H * 2, qb = T * 12 * 128 * 2, kb = T * 2 * 128 * 2, gb = T * I * 2;
    struct Layer {
        PtrSet n1, n2, sw;
        v4u *q, *k, *v, *qo;
        v2u *kc, *vc;
        float *ks, *vs;
    };
    auto v4 = [&](size_t b) { return static_cast<v4u *>(B.alloc(b)); };
    auto ptrs = [&](std::vector<v4u *> outs, std::vector<const v4u *> ins) {
        PtrSet p;
        p.d_outs = static_cast<v4u **>(B.alloc(outs.size() * sizeof(void *)));
        p.d_ins = static_cast<const v4u **>(B.alloc(ins.size() * sizeof(void *)));
        check(hipMemcpy(p.d_outs, outs.data(), outs.size() * sizeof(void *), hipMemcpyHostToDevice), "copy");
        check(hipMemcpy(p.d_ins, ins.data(), ins.size() * sizeof(void *), hipMemcpyHostToDevice), "copy");
        return p;
    };
    v4u *resid = v4(hb), *resid2 = v4(hb);
    std::vector<Layer> Ls(28);
    for (auto &l : Ls) {
        l.n1 = ptrs({v4(hb), resid2}, {v4(hb), resid});
        l.n2 = ptrs({v4(hb), resid}, {v4(hb), resid2});
        l.sw = ptrs({v4(gb)}, {v4(gb), v4(gb)});
        l.q = v4(qb), l.k = v4(kb), l.v = v4(kb), l.qo = v4(qb);
        l.kc = static_cast<v2u *>(B.alloc(kb / 2)), l.vc = static_cast<v2u *>(B.alloc(kb / 2));
        l.ks = static_cast<float *>(B.alloc(T * 8)), l.vs = static_cast<float *>(B.alloc(T * 8));
    }
    const PtrSet fin = ptrs({v4(hb)}, {resid});
    v4u *logits = v4(T * V * 2), *sink = v4(64);
    auto chain = [&]() {
        for (auto &l : Ls) {
            stream<2, 2, 1, 256><<<blocks(hb / 16), 256, 0, B.s>>>(l.n1.d_outs, l.n1.d_ins, hb / 16);
            ropeKv<<<blocks((qb + 2 * kb) / 16), 256, 0, B.s>>>(l.qo, l.q, l.k, l.v, l.kc, l.vc, l.ks, l.vs, qb / 16, kb / 16);
            stream<2, 2, 1, 256><<<blocks(hb / 16), 256, 0, B.s>>>(l.n2.d_outs, l.n2.d_ins, hb / 16);
            stream<2, 1, 1, 256><<<blocks(gb / 16), 256, 0, B.s>>>(l.sw.d_outs, l.sw.d_ins, gb / 16);
        }
        stream<1, 1, 1, 256><<<blocks(hb / 16), 256, 0, B.s>>>(fin.d_outs, fin.d_ins, hb / 16);
        readOnly<<<blocks(T * V * 2 / 16), 256, 0, B.s>>>(logits, T * V * 2 / 16, sink);
    };
    const double us = B.time(1, [&](int) { chain(); }, 4); // 4 chains (452 launches) per replay
    B.freeAll();
    return us * 1e-3;
}

} // namespace

int main() {
    Bench B;
    check(hipStreamCreate(&B.s), "stream");
    const size_t H = 1536, I = 8960;
    std::vector<std::pair<std::string, double>> out;
    // config 1 (bf16, 8192 tokens)
    const size_t tok = 8192 * H * 2;
    out.push_back({"rms_norm", B.streamFloor<1, 1>(tok)});
    out.push_back({"add_rms_norm", B.streamFloor<2, 2>(tok)});
    out.push_back({"embedding", B.streamFloor<1, 1>(tok)});
    out.push_back({"rope_qk", B.streamFloor<1, 1>(size_t(8192) * 14 * 128 * 2)});
    out.push_back({"swiglu", B.streamFloor<2, 1>(size_t(8192) * I * 2)});
    out.push_back({"argmax", B.readFloor(151936 * 2)});
    // config 3 (INT8): quantize reads 2 B and writes 1 B per element, dequantize the reverse
    const size_t w = size_t(8960) * 1536;
    out.push_back({"config3 quantize W[8960,1536]", B.streamFloor<2, 1>(w)});
    out.push_back({"config3 dequantize W[8960,1536]", B.stream12Floor(w)});
    // config-4 chain ops at 2048 tokens
    const size_t ctok = 2048 * H * 2;
    out.push_back({"chain add_rms_norm 2048", B.streamFloor<2, 2>(ctok)});
    out.push_back({"chain swiglu 2048", B.streamFloor<2, 1>(size_t(2048) * I * 2)});
    out.push_back({"chain rope_kv 2048", B.ropeKvFloor(2048)});
    out.push_back({"chain argmax_rows 2048", B.readFloor(size_t(2048) * 151936 * 2)});
    // config-4 chain
    out.push_back({"chain_ms", chainFloor(B)});
    std::printf("{");
    for (size_t i = 0; i < out.size(); ++i)
        std::printf("%s\"%s\": %.4f", i ? ", " : "", out[i].first.c_str(), out[i].second);
    std::printf("}\n");
    return 0;
}
