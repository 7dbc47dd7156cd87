#!/usr/bin/env python3
"""Benchmark of the LLAISYS per-layer ops on one MI355X.

Workload (the shape the metric is quoted on): Qwen2-1.5B layer ops in
bf16 at 8192 tokens -- embedding gather from [151936, 1536], rms_norm [8192, 1536], fused
residual add + rms_norm [8192, 1536], rope on q [8192, 12, 128] and k [8192, 2, 128],
swiglu [8192, 8960] and argmax over [1, 151936].  One step = one launch of each op over one
buffer set; 4 disjoint buffer sets (about 2.6 GB) rotate so that no step finds its inputs in
the 256 MB Infinity Cache.  Inputs are synthetic (seeded normal samples, the table
N(0, 0.02), norm weight N(1, 0.1)) and resident in HBM before timing starts.

value = algorithmic HBM bytes of the step (every input read once, every output written
once) / step time, in GB/s.  Per-op GB/s, the config-4 28-layer chain (2048-token prefill)
tokens/s, the roofline of the dominant kernel (swiglu) and the reference CPU ops timed on
this host are reported in the same JSON line.  Timing uses HIP events recorded on the
library's own stream (llaisysGetContextStream).
"""
import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "achieved HBM GB/s (% of MI355X peak) per op; layer-op tokens/s at Qwen2-1.5B"
PEAK_GBS = 8000.0  # MI355X HBM3E

T, H, V, NH, NKV, D, I = 8192, 1536, 151936, 12, 2, 128, 8960
NSETS = 4
REPS, WARMUP = 60, 10      # per-op timing: median of REPS launches after WARMUP
FOOTPRINT = 1 << 30         # bytes each per-op loop rotates through (4x the 256 MB MALL)
EAGER = False               # --eager: per-op cases launched one by one (kernel tracing)


def time_launches(hip, stream, fn, batch=64, reps=REPS, warmup=WARMUP):
    """Median and mean time in us of one call fn(i) over `reps` timed reps after `warmup`
    untimed calls.  A rep is a batch of `batch` consecutive calls bracketed by HIP events on
    the library stream (an event between single calls would add its own ~3 us to every
    interval); i keeps counting across reps, so the reps walk through every rotating buffer
    set of the case."""
    i = 0
    for _ in range(warmup):
        fn(i)
        i += 1
    evs = hip.events(reps + 1)
    hip.record(evs[0], stream)
    for r in range(reps):
        for _ in range(batch):
            fn(i)
            i += 1
        hip.record(evs[r + 1], stream)
    t = np.array([hip.elapsed_ms(evs[r], evs[r + 1]) * 1e3 / batch for r in range(reps)])
    return float(np.median(t)), float(t.mean())


def time_graph(L, hip, stream, fn, nbytes=None, batch=64, reps=REPS, warmup=2):
    """Median and mean time in us of one call fn(i), from replays of one HIP graph that holds
    n consecutive calls fn(0) .. fn(n - 1): n = 64, or the number of rotating buffer sets of
    a case of `nbytes` per call if that is larger, so every replay walks each set once.  The
    graph keeps host work out of the timed region: launched eagerly from Python, a call
    costs ~3.7 us of host time, more than a small kernel takes."""
    if EAGER:
        return time_launches(hip, stream, fn, batch=batch, reps=reps)
    n = batch if nbytes is None else max(batch, int(min(4096, -(-FOOTPRINT // max(1, nbytes)))))
    graph = L.Graph.capture()
    for i in range(n):
        fn(i)
    graph.end()
    for _ in range(warmup):
        graph.launch()
    evs = hip.events(reps + 1)
    hip.record(evs[0], stream)
    for r in range(reps):
        graph.launch()
        hip.record(evs[r + 1], stream)
    t = np.array([hip.elapsed_ms(evs[r], evs[r + 1]) * 1e3 / n for r in range(reps)])
    del graph
    return float(np.median(t)), float(t.mean())


def rate(name_us, nbytes, mean_us=None):
    gbs = nbytes / (name_us * 1e-6) / 1e9
    r = {"us": round(name_us, 3), "bytes": nbytes, "GB_s": round(gbs, 1),
         "frac_peak": round(gbs / PEAK_GBS, 4)}
    if mean_us is not None:
        r["mean_us"] = round(mean_us, 3)
    return r


class HipEvents:
    """hipEvent timing through the HIP runtime already loaded by libllaisys.so."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]

    def event(self):
        ev = ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(ev)) == 0
        return ev

    def events(self, n):
        if len(getattr(self, "_pool", [])) < n:
            self._pool = [self.event() for _ in range(n)]
        return self._pool[:n]

    def record(self, ev, stream):
        assert self.hip.hipEventRecord(ev, ctypes.c_void_p(stream)) == 0

    def elapsed_ms(self, a, b):
        assert self.hip.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value


def bf16(rng, shape, scale=1.0, loc=0.0):
    from llaisys_amd.hostfmt import f32_to_bf16
    return f32_to_bf16(loc + scale * rng.standard_normal(shape, dtype=np.float32))


class Workload:
    """Device buffers of the config-1 step: 4 rotating sets plus the shared table."""

    def __init__(self, L, seed=1):
        BF, I64 = L.DataType.BF16, L.DataType.I64
        dev = dict(device=L.DeviceType.AMD, device_id=0)
        rng = np.random.default_rng(seed)
        self.L = L
        self.table = L.Tensor.from_numpy(bf16(rng, (V, H), 0.02), BF, **dev)
        self.w = L.Tensor.from_numpy(bf16(rng, (H,), 0.1, 1.0), BF, **dev)
        self.pos = L.Tensor.from_numpy(np.arange(T, dtype=np.int64), **dev)
        host = {
            "x": bf16(rng, (T, H)), "r": bf16(rng, (T, H)),
            "q": bf16(rng, (T, NH, D)), "k": bf16(rng, (T, NKV, D)),
            "gate": bf16(rng, (T, I)), "up": bf16(rng, (T, I)),
            "logits": bf16(rng, (1, V)),
        }
        api = L.RuntimeAPI(L.DeviceType.AMD)
        self.sets = []
        for s in range(NSETS):
            b = {"ids": L.Tensor.from_numpy(rng.integers(0, V, size=T).astype(np.int64), **dev)}
            for name, arr in host.items():
                if s == 0:
                    b[name] = L.Tensor.from_numpy(arr, BF, **dev)
                else:  # same values, distinct addresses
                    b[name] = L.Tensor(arr.shape, BF, **dev)
                    api.memcpy_sync(b[name].data_ptr(), self.sets[0][name].data_ptr(), arr.nbytes,
                                    L.MemcpyKind.D2D)
            for name, shape in (("emb", (T, H)), ("y_rms", (T, H)), ("y", (T, H)), ("h", (T, H)),
                                ("q_out", (T, NH, D)), ("k_out", (T, NKV, D)), ("act", (T, I))):
                b[name] = L.Tensor(shape, BF, **dev)
            b["idx"] = L.Tensor((1,), I64, **dev)
            b["val"] = L.Tensor((1,), BF, **dev)
            self.sets.append(b)

    def extra_ops(self):
        """Reference-ABI forms measured beside the step (q and k RoPE as two calls)."""
        O = self.L.Ops
        return [
            ("rope_q", 2 * T * NH * D * 2 + T * 8, lambda b: O.rope(b["q_out"], b["q"], self.pos, 1e4)),
            ("rope_k", 2 * T * NKV * D * 2 + T * 8, lambda b: O.rope(b["k_out"], b["k"], self.pos, 1e4)),
        ]

    def ops(self):
        """(name, algorithmic bytes per launch, launch(set)) of one step."""
        O = self.L.Ops
        tok = T * H * 2
        return [
            ("embedding", T * 8 + 2 * tok, lambda b: O.embedding(b["emb"], b["ids"], self.table)),
            ("rms_norm", 2 * tok + H * 2, lambda b: O.rms_norm(b["y_rms"], b["x"], self.w, 1e-6)),
            ("add_rms_norm", 4 * tok + H * 2,
             lambda b: O.add_rms_norm(b["y"], b["h"], b["x"], b["r"], self.w, 1e-6)),
            ("rope_qk", 2 * T * (NH + NKV) * D * 2 + T * 8,
             lambda b: O.rope_qk(b["q_out"], b["q"], b["k_out"], b["k"], self.pos, 1e4)),
            ("swiglu", 3 * T * I * 2, lambda b: O.swiglu(b["act"], b["gate"], b["up"])),
            ("argmax", V * 2 + 8 + 2, lambda b: O.argmax(b["idx"], b["val"], b["logits"])),
        ]


class Chain:
    """Config 4: 28 Qwen2-1.5B layers of the per-layer ops at 2048 tokens, then the final
    norm and argmax over [2048, 151936] logits.  Random activations stand in for the
    GEMM / attention outputs; every layer has its own buffers."""

    TOK, LAYERS, MAXSEQ = 2048, 28, 2048

    def __init__(self, L, seed=4):
        BF, I8, F32 = L.DataType.BF16, L.DataType.I8, L.DataType.F32
        dev = dict(device=L.DeviceType.AMD, device_id=0)
        rng = np.random.default_rng(seed)
        t = self.TOK
        api = L.RuntimeAPI(L.DeviceType.AMD)
        self.L = L
        self.pos = L.Tensor.from_numpy(np.arange(t, dtype=np.int64), **dev)
        proto = {"attn": bf16(rng, (t, H)), "mlp": bf16(rng, (t, H)), "q": bf16(rng, (t, NH, D)),
                 "k": bf16(rng, (t, NKV, D)), "v": bf16(rng, (t, NKV, D)),
                 "gate": bf16(rng, (t, I)), "up": bf16(rng, (t, I))}
        first = {k: L.Tensor.from_numpy(a, BF, **dev) for k, a in proto.items()}
        self.layers = []
        for layer in range(self.LAYERS):
            b = {}
            for k, a in proto.items():
                if layer == 0:
                    b[k] = first[k]
                else:
                    b[k] = L.Tensor(a.shape, BF, **dev)
                    api.memcpy_sync(b[k].data_ptr(), first[k].data_ptr(), a.nbytes, L.MemcpyKind.D2D)
            b["w1"] = L.Tensor.from_numpy(bf16(rng, (H,), 0.1, 1.0), BF, **dev)
            b["w2"] = L.Tensor.from_numpy(bf16(rng, (H,), 0.1, 1.0), BF, **dev)
            for k, shape in (("n1", (t, H)), ("n2", (t, H)), ("q_out", (t, NH, D)),
                             ("k_out", (t, NKV, D)), ("act", (t, I))):
                b[k] = L.Tensor(shape, BF, **dev)
            for k in ("kc", "vc"):
                b[k] = L.Tensor((self.MAXSEQ, NKV, D), I8, **dev)
                b[k + "s"] = L.Tensor((self.MAXSEQ, NKV), F32, **dev)
            self.layers.append(b)
        self.resid = L.Tensor.from_numpy(bf16(rng, (t, H)), BF, **dev)
        self.wf = L.Tensor.from_numpy(bf16(rng, (H,), 0.1, 1.0), BF, **dev)
        self.final = L.Tensor((t, H), BF, **dev)
        self.logits = L.Tensor.from_numpy(bf16(rng, (t, V)), BF, **dev)
        self.tok_idx = L.Tensor((t,), L.DataType.I64, **dev)
        self.tok_val = L.Tensor((t,), BF, **dev)

    def bytes(self):
        t, e = self.TOK, 2
        norm = 4 * t * H * e + H * e
        # fused RoPE + INT8 KV append: q in/out, k and v in, codes and scales out
        rope = 2 * t * NH * D * e + t * 8
        kv = 2 * (t * NKV * D * e + t * NKV * D + t * NKV * 4)
        swi = 3 * t * I * e
        layer = 2 * norm + rope + kv + swi
        return self.LAYERS * layer + (2 * t * H * e + H * e) + (t * V * e + t * 8 + t * e)

    def run(self):
        O = self.L.Ops
        for b in self.layers:
            O.add_rms_norm(b["n1"], self.resid, b["attn"], self.resid, b["w1"], 1e-6)
            O.rope_kv_append_int8(b["q_out"], b["q"], b["k"], b["v"], self.pos, 1e6,
                                  b["kc"], b["kcs"], b["vc"], b["vcs"], 0)
            O.add_rms_norm(b["n2"], self.resid, b["mlp"], self.resid, b["w2"], 1e-6)
            O.swiglu(b["act"], b["gate"], b["up"])
        O.rms_norm(self.final, self.resid, self.wf, 1e-6)
        O.argmax_rows(self.tok_idx, self.tok_val, self.logits)


class DecodeChain:
    """One decode step of Qwen2-1.5B built from the library's entry points only (random
    weights, the reference's layer structure, src/models/qwen2/{layer,attention,mlp}.hpp):
    embedding; per layer add+rms_norm, q / k / v linear (with bias), fused RoPE + INT8 KV
    append at position CTX, attention over the CTX + 1 cached tokens (INT8 KV), o linear,
    add+rms_norm, gate / up linear, swiglu, down linear; then the final norm, the lm_head
    linear and a sample (T 0.8, top_k 50, top_p 0.8).  Projection weights are INT8 codes +
    per-channel scales (W8A16) or bf16; every layer has its own copies, so no cache serves
    them.  Like production Qwen2 decoders, q / k / v are one concatenated [2048, 1536]
    projection (with its bias) and gate / up one [17920, 1536] projection: one linear launch
    each, the one-row outputs split by slicing."""

    LAYERS, CTX = 28, 4096

    def __init__(self, L, int8_weights=True, seed=6, fused=True):
        BF, I8, F32, I64 = L.DataType.BF16, L.DataType.I8, L.DataType.F32, L.DataType.I64
        dev = dict(device=L.DeviceType.AMD, device_id=0)
        rng = np.random.default_rng(seed)
        api = L.RuntimeAPI(L.DeviceType.AMD)
        O = L.Ops
        self.L, self.int8, self.fused = L, int8_weights, fused
        QKV = (NH + 2 * NKV) * D
        shapes = {"qkv": (QKV, H), "o": (H, NH * D), "gate_up": (2 * I, H), "down": (H, I)}

        def copies(proto, n):
            out = [proto]
            for _ in range(n - 1):
                t = L.Tensor(proto.shape(), proto.dtype(), **dev)
                api.memcpy_sync(t.data_ptr(), proto.data_ptr(), proto.numel() * (1 if proto.dtype() == I8 else 2 if proto.dtype() == BF else 4), L.MemcpyKind.D2D)
                out.append(t)
            return out

        self.w = {}
        for name, shp in shapes.items():
            wb = L.Tensor.from_numpy(bf16(rng, shp, 0.02), BF, **dev)
            if int8_weights:
                q, sc = L.Tensor(shp, I8, **dev), L.Tensor((shp[0],), F32, **dev)
                O.quantize_int8(q, sc, wb)
                self.w[name] = list(zip(copies(q, self.LAYERS), copies(sc, self.LAYERS)))
            else:
                self.w[name] = [(t, None) for t in copies(wb, self.LAYERS)]
        self.bias = copies(L.Tensor.from_numpy(bf16(rng, (QKV,), 0.1), BF, **dev), self.LAYERS)
        self.norm = [(L.Tensor.from_numpy(bf16(rng, (H,), 0.1, 1.0), BF, **dev),
                      L.Tensor.from_numpy(bf16(rng, (H,), 0.1, 1.0), BF, **dev)) for _ in range(self.LAYERS)]
        # INT8 KV caches holding CTX tokens, one row more for the step's append
        kv0 = [L.Tensor.from_numpy(bf16(rng, (self.CTX, NKV, D)), BF, **dev) for _ in range(2)]
        self.cache = []
        for _ in range(self.LAYERS):
            c = {}
            for nm, src in (("k", kv0[0]), ("v", kv0[1])):
                c[nm] = L.Tensor((self.CTX + 1, NKV, D), I8, **dev)
                c[nm + "s"] = L.Tensor((self.CTX + 1, NKV), F32, **dev)
                O.kv_append_int8(c[nm], c[nm + "s"], src, 0)
            c["kview"] = c["k"].slice(0, 0, self.CTX + 1)
            c["vview"] = c["v"].slice(0, 0, self.CTX + 1)
            self.cache.append(c)
        self.table = L.Tensor.from_numpy(bf16(rng, (V, H), 0.02), BF, **dev)
        if int8_weights:
            lq, ls = L.Tensor((V, H), I8, **dev), L.Tensor((V,), F32, **dev)
            O.quantize_int8(lq, ls, L.Tensor.from_numpy(bf16(rng, (V, H), 0.02), BF, **dev))
            self.lm = (lq, ls)
        else:
            self.lm = (L.Tensor.from_numpy(bf16(rng, (V, H), 0.02), BF, **dev), None)
        self.wf = L.Tensor.from_numpy(bf16(rng, (H,), 0.1, 1.0), BF, **dev)
        self.ids = L.Tensor.from_numpy(np.array([12345], np.int64), **dev)
        self.pos = L.Tensor.from_numpy(np.array([self.CTX], np.int64), **dev)
        t = lambda shp, dt=BF: L.Tensor(shp, dt, **dev)
        self.x, self.n, self.prev = t((1, H)), t((1, H)), t((1, H))
        self.x2 = t((1, H))  # the fused ops write the residual stream ping-pong
        self.qkv = t((1, QKV))
        flat = self.qkv.view(QKV)
        self.qv = flat.slice(0, 0, NH * D).view(1, NH, D)
        self.kv = flat.slice(0, NH * D, (NH + NKV) * D).view(1, NKV, D)
        self.vv = flat.slice(0, (NH + NKV) * D, QKV).view(1, NKV, D)
        self.gu = t((1, 2 * I))
        gflat = self.gu.view(2 * I)
        self.g, self.u = gflat.slice(0, 0, I).view(1, I), gflat.slice(0, I, 2 * I).view(1, I)
        self.qr, self.att, self.o = t((1, NH, D)), t((1, NH, D)), t((1, H))
        self.a, self.d = t((1, I)), t((1, H))
        self.logits, self.tok = t((1, V)), t((1,), I64)
        self.zero = L.Tensor.from_numpy(np.zeros((1, H), np.uint16), BF, **dev)

    def _lin(self, out, x, pair, bias=None):
        O = self.L.Ops
        w, sc = pair
        if sc is None:
            O.linear(out, x, w, bias)
        else:
            O.linear_w8a16(out, x, w, sc, bias)

    def weight_bytes(self):
        per = sum(r * c for r, c in (((NH + 2 * NKV) * D, H), (H, NH * D), (2 * I, H), (H, I)))
        e = 1 if self.int8 else 2
        return self.LAYERS * per * e + V * H * e

    def run(self, seed=0):
        if self.fused:
            return self.run_fused(seed)
        O = self.L.Ops
        O.embedding(self.prev, self.ids, self.table)
        api_x = self.zero
        for l in range(self.LAYERS):
            c = self.cache[l]
            # x = prev + x (the first layer adds the embedding to zero); n = rms_norm(x)
            O.add_rms_norm(self.n, self.x, self.prev, api_x if l == 0 else self.x, self.norm[l][0], 1e-6)
            self._lin(self.qkv, self.n, self.w["qkv"][l], self.bias[l])
            self._attend(l)
            O.add_rms_norm(self.n, self.x, self.o, self.x, self.norm[l][1], 1e-6)
            self._lin(self.gu, self.n, self.w["gate_up"][l])
            O.swiglu(self.a, self.g, self.u)
            self._lin(self.prev, self.a, self.w["down"][l])
        O.add_rms_norm(self.n, self.x, self.prev, self.x, self.wf, 1e-6)
        self._lin(self.logits, self.n, self.lm)
        O.random_sample(self.tok, self.logits, 0.8, 50, 0.8, seed)

    def _attend(self, l):
        """RoPE + INT8 KV append, attention over the cache, o projection -> self.o."""
        O, c = self.L.Ops, self.cache[l]
        O.rope_kv_append_int8(self.qr, self.qv, self.kv, self.vv, self.pos, 1e6,
                              c["k"], c["ks"], c["v"], c["vs"], self.CTX)
        O.self_attention_int8kv(self.att, self.qr, c["kview"], c["ks"], c["vview"], c["vs"],
                                1.0 / np.sqrt(D))
        self._lin(self.o, self.att.view(1, NH * D), self.w["o"][l])

    def run_fused(self, seed=0):
        """The same step with the norms fused into the projections after them and swiglu
        into the gate / up projection (llaisysRmsNormLinear): 7 launches per layer."""
        O = self.L.Ops
        O.embedding(self.prev, self.ids, self.table)
        cur, nxt = self.zero, self.x
        for l in range(self.LAYERS):
            w, sc = self.w["qkv"][l]
            O.rms_norm_linear(self.qkv, self.prev, self.norm[l][0], 1e-6, w, sc, self.bias[l],
                              residual=cur, residual_out=nxt)
            cur, nxt = nxt, (self.x2 if nxt is self.x else self.x)
            self._attend(l)
            w, sc = self.w["gate_up"][l]
            O.rms_norm_linear(self.a, self.o, self.norm[l][1], 1e-6, w, sc, residual=cur,
                              residual_out=nxt, swiglu=True)
            cur, nxt = nxt, (self.x2 if nxt is self.x else self.x)
            self._lin(self.prev, self.a, self.w["down"][l])
        O.add_rms_norm(self.n, nxt, self.prev, cur, self.wf, 1e-6)
        self._lin(self.logits, self.n, self.lm)
        O.random_sample(self.tok, self.logits, 0.8, 50, 0.8, seed)


class Pool:
    """Disjoint buffer sets cut from one allocation per tensor (slice + view keep the byte
    offset), filled with seeded normal samples; enough sets that one pass over them moves
    >= 1 GiB (FOOTPRINT), so the 256 MB Infinity Cache does not serve the timed launches."""

    def __init__(self, L, rng):
        self.L, self.rng = L, rng
        self.dev = dict(device=L.DeviceType.AMD, device_id=0)
        self.api = L.RuntimeAPI(L.DeviceType.AMD)
        self.keep = []

    def sets_for(self, nbytes, cap=4096):
        return int(max(4, min(cap, -(-FOOTPRINT // max(1, nbytes)))))

    def fill(self, shape, dtype, sets, scale=1.0, loc=0.0):
        """`sets` tensors of `shape`; the first is sampled, the others copy it."""
        L = self.L
        n = int(np.prod(shape))
        big = L.Tensor((sets * n,), dtype, **self.dev)
        self.keep.append(big)
        if dtype == L.DataType.BF16:
            host = bf16(self.rng, (n,), scale, loc)
        elif dtype == L.DataType.F32:
            host = (loc + scale * self.rng.standard_normal(n, dtype=np.float32)).astype(np.float32)
        else:
            raise ValueError(dtype)
        first = big.slice(0, 0, n)
        first.load(host.ctypes.data_as(ctypes.c_void_p))
        out = []
        for k in range(sets):
            t = big.slice(0, k * n, (k + 1) * n).view(*shape)
            if k:
                self.api.memcpy_sync(t.data_ptr(), first.data_ptr(), host.nbytes, L.MemcpyKind.D2D)
            out.append(t)
        return out

    def empty(self, shape, dtype, sets):
        L = self.L
        n = int(np.prod(shape))
        big = L.Tensor((sets * n,), dtype, **self.dev)
        self.keep.append(big)
        return [big.slice(0, k * n, (k + 1) * n).view(*shape) for k in range(sets)]

    def ints(self, values_list):
        return [self.L.Tensor.from_numpy(v, **self.dev) for v in values_list]


def config1_ops(L, rng):
    """(op, algorithmic bytes per launch, launch(i)) for the config-1 ops one at a time,
    each over its own >= 1 GiB of rotating buffer sets; the reference-ABI rope (q and k as
    two calls) is timed beside the fused launch."""
    O, BF, I64 = L.Ops, L.DataType.BF16, L.DataType.I64
    P = Pool(L, rng)
    tok = T * H * 2
    cases = []
    table = P.fill((V, H), BF, 1, 0.02)[0]
    w = P.fill((H,), BF, 1, 0.1, 1.0)[0]
    pos = L.Tensor.from_numpy(np.arange(T, dtype=np.int64), **P.dev)

    b = T * 8 + 2 * tok
    s = P.sets_for(b)
    ids = P.ints([rng.integers(0, V, size=T).astype(np.int64) for _ in range(s)])
    emb = P.empty((T, H), BF, s)
    cases.append(("embedding", b, lambda i, s=s: O.embedding(emb[i % s], ids[i % s], table)))

    b = 2 * tok + H * 2
    s = P.sets_for(b)
    x, y = P.fill((T, H), BF, s), P.empty((T, H), BF, s)
    cases.append(("rms_norm", b, lambda i, s=s: O.rms_norm(y[i % s], x[i % s], w, 1e-6)))

    b = 4 * tok + H * 2
    s = P.sets_for(b)
    xa, ra = P.fill((T, H), BF, s), P.fill((T, H), BF, s)
    ya, ha = P.empty((T, H), BF, s), P.empty((T, H), BF, s)
    cases.append(("add_rms_norm", b,
                  lambda i, s=s: O.add_rms_norm(ya[i % s], ha[i % s], xa[i % s], ra[i % s], w, 1e-6)))

    b = 2 * T * (NH + NKV) * D * 2 + T * 8
    s = P.sets_for(b)
    q, k = P.fill((T, NH, D), BF, s), P.fill((T, NKV, D), BF, s)
    qo, ko = P.empty((T, NH, D), BF, s), P.empty((T, NKV, D), BF, s)
    cases.append(("rope_qk", b, lambda i, s=s: O.rope_qk(qo[i % s], q[i % s], ko[i % s], k[i % s], pos, 1e4)))
    cases.append(("rope_q", 2 * T * NH * D * 2 + T * 8, lambda i, s=s: O.rope(qo[i % s], q[i % s], pos, 1e4)))
    cases.append(("rope_k", 2 * T * NKV * D * 2 + T * 8, lambda i, s=s: O.rope(ko[i % s], k[i % s], pos, 1e4)))

    b = 3 * T * I * 2
    s = P.sets_for(b)
    g, u, act = P.fill((T, I), BF, s), P.fill((T, I), BF, s), P.empty((T, I), BF, s)
    cases.append(("swiglu", b, lambda i, s=s: O.swiglu(act[i % s], g[i % s], u[i % s])))

    b = V * 2 + 8 + 2
    s = P.sets_for(b)
    lg = P.fill((1, V), BF, s)
    mi, mv = P.empty((1,), I64, 1)[0], P.empty((1,), BF, 1)[0]
    cases.append(("argmax", b, lambda i, s=s: O.argmax(mi, mv, lg[i % s])))
    return cases, P


def config_ops(L, rng):
    """(config, op, algorithmic bytes per launch, launches per call, launch(i)) for the
    parity configs other than the headline one (2 and 3)."""
    O, BF, F32, I8, I64 = L.Ops, L.DataType.BF16, L.DataType.F32, L.DataType.I8, L.DataType.I64
    P = Pool(L, rng)
    cases = []

    # config 0: Qwen2-1.5B shapes, f32, 128 tokens
    t0, V0 = 128, 151936
    table = P.fill((V0, H), F32, 1, 0.02)[0]
    s = P.sets_for(t0 * H * 4 * 2)
    ids = P.ints([rng.integers(0, V0, size=t0).astype(np.int64) for _ in range(s)])
    emb = P.empty((t0, H), F32, s)
    cases.append(("config0", "embedding f32 128x1536", t0 * 8 + 2 * t0 * H * 4, 1,
                  lambda i: O.embedding(emb[i % s], ids[i % s], table)))
    x, y = P.fill((t0, H), F32, s), P.empty((t0, H), F32, s)
    w = P.fill((H,), F32, 1, 0.1, 1.0)[0]
    cases.append(("config0", "rms_norm f32 [128,1536]", 2 * t0 * H * 4 + H * 4, 1,
                  lambda i: O.rms_norm(y[i % s], x[i % s], w, 1e-6)))
    sq = P.sets_for(t0 * 14 * 128 * 4 * 2)
    q, k = P.fill((t0, NH, D), F32, sq), P.fill((t0, NKV, D), F32, sq)
    qo, ko = P.empty((t0, NH, D), F32, sq), P.empty((t0, NKV, D), F32, sq)
    pos0 = L.Tensor.from_numpy(np.arange(t0, dtype=np.int64), **P.dev)
    cases.append(("config0", "rope q+k f32 [128,12+2,128]", 2 * t0 * (NH + NKV) * D * 4 + t0 * 8, 1,
                  lambda i: O.rope_qk(qo[i % sq], q[i % sq], ko[i % sq], k[i % sq], pos0, 1e4)))
    ss = P.sets_for(3 * t0 * I * 4)
    g, u, a = P.fill((t0, I), F32, ss), P.fill((t0, I), F32, ss), P.empty((t0, I), F32, ss)
    cases.append(("config0", "swiglu f32 [128,8960]", 3 * t0 * I * 4, 1,
                  lambda i: O.swiglu(a[i % ss], g[i % ss], u[i % ss])))
    sa = P.sets_for(V0 * 4)
    lg = P.fill((1, V0), F32, sa)
    mi, mv = P.empty((1,), I64, 1)[0], P.empty((1,), F32, 1)[0]
    cases.append(("config0", "argmax f32 [1,151936] (latency)", V0 * 4 + 12, 1,
                  lambda i: O.argmax(mi, mv, lg[i % sa])))

    # config 2: Llama-8B shapes, bf16, 16384 tokens (4 sets: >= 1 GiB per loop)
    t2, H2, I2, V2 = 16384, 4096, 14336, 128256
    n2 = 4
    x2, y2 = P.fill((t2, H2), BF, n2), P.empty((t2, H2), BF, n2)
    w2 = P.fill((H2,), BF, 1, 0.1, 1.0)[0]
    cases.append(("config2", "rms_norm [16384,4096]", 2 * t2 * H2 * 2 + H2 * 2, 1,
                  lambda i: O.rms_norm(y2[i % n2], x2[i % n2], w2, 1e-5)))
    q2, k2 = P.fill((t2, 32, D), BF, n2), P.fill((t2, 8, D), BF, n2)
    qo2, ko2 = P.empty((t2, 32, D), BF, n2), P.empty((t2, 8, D), BF, n2)
    pos2 = L.Tensor.from_numpy(np.arange(t2, dtype=np.int64), **P.dev)
    cases.append(("config2", "rope q+k [16384,32+8,128] theta 5e5", 2 * t2 * 40 * D * 2 + t2 * 8, 1,
                  lambda i: O.rope_qk(qo2[i % n2], q2[i % n2], ko2[i % n2], k2[i % n2], pos2, 5e5)))
    g2, u2, a2 = P.fill((t2, I2), BF, n2), P.fill((t2, I2), BF, n2), P.empty((t2, I2), BF, n2)
    cases.append(("config2", "swiglu [16384,14336]", 3 * t2 * I2 * 2, 1,
                  lambda i: O.swiglu(a2[i % n2], g2[i % n2], u2[i % n2])))
    table2 = P.fill((V2, H2), BF, 1, 0.02)[0]
    ids2 = P.ints([rng.integers(0, V2, size=t2).astype(np.int64) for _ in range(n2)])
    emb2 = P.empty((t2, H2), BF, n2)
    cases.append(("config2", "embedding [128256,4096] x 16384 ids", t2 * 8 + 2 * t2 * H2 * 2, 1,
                  lambda i: O.embedding(emb2[i % n2], ids2[i % n2], table2)))

    # config 3: INT8 weights (per output channel) and KV cache (per token and head)
    for rows, cols in ((8960, 1536), (1536, 8960)):
        sw = P.sets_for(rows * cols * 3)
        wt = P.fill((rows, cols), BF, sw, 0.02)
        qc, sc = P.empty((rows, cols), I8, sw), P.empty((rows,), F32, sw)
        dq = P.empty((rows, cols), BF, sw)
        nb = rows * cols * 3 + rows * 4
        cases.append(("config3", f"quantize W[{rows},{cols}]", nb, 1,
                      lambda i, wt=wt, qc=qc, sc=sc, sw=sw: O.quantize_int8(qc[i % sw], sc[i % sw], wt[i % sw])))
        cases.append(("config3", f"dequantize W[{rows},{cols}]", nb, 1,
                      lambda i, dq=dq, qc=qc, sc=sc, sw=sw: O.dequantize_int8(dq[i % sw], qc[i % sw], sc[i % sw])))
    tk = 32768
    skv = P.sets_for(2 * tk * 2 * D * 3)
    kv_k, kv_v = P.fill((tk, 2, D), BF, skv), P.fill((tk, 2, D), BF, skv)
    ckq, cks = P.empty((tk, 2, D), I8, skv), P.empty((tk, 2), F32, skv)
    cvq, cvs = P.empty((tk, 2, D), I8, skv), P.empty((tk, 2), F32, skv)
    dk, dv = P.empty((tk, 2, D), BF, skv), P.empty((tk, 2, D), BF, skv)
    kvb = 2 * (tk * 2 * D * 2 + tk * 2 * D + tk * 2 * 4)

    def append(i):
        O.kv_append_int8(ckq[i % skv], cks[i % skv], kv_k[i % skv], 0)
        O.kv_append_int8(cvq[i % skv], cvs[i % skv], kv_v[i % skv], 0)

    def read(i):
        O.dequantize_int8(dk[i % skv], ckq[i % skv], cks[i % skv])
        O.dequantize_int8(dv[i % skv], cvq[i % skv], cvs[i % skv])

    def append_pair(i):
        j = i % skv
        O.kv_append_int8_pair(ckq[j], cks[j], cvq[j], cvs[j], kv_k[j], kv_v[j], 0)

    def read_pair(i):
        j = i % skv
        O.dequantize_int8_pair(dk[j], ckq[j], cks[j], dv[j], cvq[j], cvs[j])

    cases.append(("config3", "KV append k+v [32768,2,128] (pair, 1 launch)", kvb, 1, append_pair))
    cases.append(("config3", "KV dequant read k+v [32768,2,128] (pair, 1 launch)", kvb, 1, read_pair))
    cases.append(("config3", "KV append k+v [32768,2,128] (2 launches)", kvb, 2, append))
    cases.append(("config3", "KV dequant read k+v [32768,2,128] (2 launches)", kvb, 2, read))
    return cases, P


PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


def attention_ops(L, rng):
    """(name, kind, amount per launch, launch(i)) for self-attention at Qwen2-1.5B heads
    (12 q / 2 kv, head_dim 128): one-token decode over a 32768-token cache, INT8 and bf16
    (kind "bytes": K and V read once + q + out), and a 2048-token causal prefill (kind
    "flops": 4 * heads * head_dim * visible keys summed over the queries)."""
    O, BF, F32, I8 = L.Ops, L.DataType.BF16, L.DataType.F32, L.DataType.I8
    P = Pool(L, rng)
    nh, nkv, d, tk = 12, 2, 128, 32768
    sk = P.sets_for(tk * nkv * d * 2 * 2)
    q1 = P.fill((1, nh, d), BF, sk)
    kb, vb = P.fill((tk, nkv, d), BF, sk), P.fill((tk, nkv, d), BF, sk)
    kq, vq = P.empty((tk, nkv, d), I8, sk), P.empty((tk, nkv, d), I8, sk)
    ks, vs = P.empty((tk, nkv), F32, sk), P.empty((tk, nkv), F32, sk)
    for j in range(sk):
        O.kv_append_int8_pair(kq[j], ks[j], vq[j], vs[j], kb[j], vb[j], 0)
    o1 = P.empty((1, nh, d), BF, 1)[0]
    sc = 1.0 / np.sqrt(d)
    qo = 2 * nh * d * 2
    ops = [
        ("decode INT8 KV [32768, 2, 128], 12 q heads", "bytes", tk * nkv * (d + 4) * 2 + qo,
         lambda i: O.self_attention_int8kv(o1, q1[i % sk], kq[i % sk], ks[i % sk], vq[i % sk], vs[i % sk], sc)),
        ("decode bf16 KV [32768, 2, 128], 12 q heads", "bytes", tk * nkv * d * 2 * 2 + qo,
         lambda i: O.self_attention(o1, q1[i % sk], kb[i % sk], vb[i % sk], sc)),
    ]
    tp = 2048
    qp = P.fill((tp, nh, d), BF, 1)[0]
    kp, vp = P.fill((tp, nkv, d), BF, 1)[0], P.fill((tp, nkv, d), BF, 1)[0]
    op_ = P.empty((tp, nh, d), BF, 1)[0]
    ops.append(("prefill 2048 tokens causal, 12 q / 2 kv heads, bf16", "flops",
                4 * nh * d * tp * (tp + 1) // 2,
                lambda i: O.self_attention(op_, qp, kp, vp, sc)))
    kpq, kps = P.empty((tp, nkv, d), I8, 1)[0], P.empty((tp, nkv), F32, 1)[0]
    vpq, vps = P.empty((tp, nkv, d), I8, 1)[0], P.empty((tp, nkv), F32, 1)[0]
    O.kv_append_int8_pair(kpq, kps, vpq, vps, kp, vp, 0)
    ops.append(("prefill 2048 tokens causal, 12 q / 2 kv heads, INT8 KV", "flops",
                4 * nh * d * tp * (tp + 1) // 2,
                lambda i: O.self_attention_int8kv(op_, qp, kpq, kps, vpq, vps, sc)))
    return ops, P


def time_cases(L, hip, stream, e0, e1, steps, cases):
    """Times (name, kind, amount per launch, launch(i)) cases with HIP events on the library
    stream; kind "bytes" is rated against HBM, "flops" against the bf16 MFMA peak."""
    res = {}
    for name, kind, amount, fn in cases:
        us, mean = time_graph(L, hip, stream, fn)
        if kind == "bytes":
            res[name] = dict(rate(us, amount, mean), bound="hbm")
        else:
            tf = amount / (us * 1e-6) / 1e12
            res[name] = {"us": round(us, 3), "mean_us": round(mean, 3), "flops": amount,
                         "TFLOP_s": round(tf, 2), "frac_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                         "bound": "mfma (bf16 dense peak)"}
    assert L.take_device_error() == 0
    return res


def measure_attention(L, hip, stream, e0, e1, steps):
    """Times the attention_ops cases."""
    print("bench: building attention buffers", file=sys.stderr, flush=True)
    aops, apool = attention_ops(L, np.random.default_rng(11))
    res = time_cases(L, hip, stream, e0, e1, steps, aops)
    del aops, apool
    print("bench: attention " + json.dumps(res), file=sys.stderr, flush=True)
    return res


def linear_ops(L, rng):
    """(name, kind, amount per launch, launch(i)) for the Qwen2-1.5B projections: decode
    (one token: HBM-bound on the weights; bytes = weights (+ scales) + x + out) and a
    2048-token prefill (MFMA-bound; flops = 2 * rows * in * out), dense bf16 and W8A16 (INT8
    codes + per-channel scales from llaisysQuantizeInt8 of the bf16 weights)."""
    O, BF, F32, I8 = L.Ops, L.DataType.BF16, L.DataType.F32, L.DataType.I8
    P = Pool(L, rng)
    ops = []

    def weights(out_f, in_f, sets):
        w = P.fill((out_f, in_f), BF, sets, 0.02)
        q, sc = P.empty((out_f, in_f), I8, sets), P.empty((out_f,), F32, sets)
        for j in range(sets):
            O.quantize_int8(q[j], sc[j], w[j])
        return w, q, sc

    for label, in_f, out_f in (("gate/up [8960, 1536]", H, I), ("down [1536, 8960]", I, H)):
        sets = P.sets_for(out_f * in_f * 2)
        w, q, sc = weights(out_f, in_f, sets)
        x1 = P.fill((1, in_f), BF, sets)
        o1 = P.empty((1, out_f), BF, 1)[0]
        io = (in_f + out_f) * 2
        ops.append((f"decode 1 token, {label}, bf16 weights", "bytes", out_f * in_f * 2 + io,
                    lambda i, x1=x1, w=w, o1=o1, n=sets: O.linear(o1, x1[i % n], w[i % n])))
        ops.append((f"decode 1 token, {label}, INT8 weights (W8A16)", "bytes", out_f * (in_f + 4) + io,
                    lambda i, x1=x1, q=q, sc=sc, o1=o1, n=sets: O.linear_w8a16(o1, x1[i % n], q[i % n], sc[i % n])))
        tp = 2048
        xp = P.fill((tp, in_f), BF, 1)[0]
        op_ = P.empty((tp, out_f), BF, 1)[0]
        fl = 2 * tp * in_f * out_f
        ops.append((f"prefill 2048 tokens, {label}, bf16 weights", "flops", fl,
                    lambda i, xp=xp, w=w, op_=op_: O.linear(op_, xp, w[0])))
        ops.append((f"prefill 2048 tokens, {label}, INT8 weights (W8A16)", "flops", fl,
                    lambda i, xp=xp, q=q, sc=sc, op_=op_: O.linear_w8a16(op_, xp, q[0], sc[0])))
    # lm_head: sets sized by the INT8 codes (234 MB alone would sit in the 256 MB Infinity Cache)
    nl = P.sets_for(V * H)
    wl, ql, scl = weights(V, H, nl)
    xl, ol = P.fill((1, H), BF, 1)[0], P.empty((1, V), BF, 1)[0]
    ops.append(("decode 1 token, lm_head [151936, 1536], bf16 weights", "bytes", V * H * 2 + (H + V) * 2,
                lambda i: O.linear(ol, xl, wl[i % nl])))
    ops.append(("decode 1 token, lm_head [151936, 1536], INT8 weights (W8A16)", "bytes",
                V * (H + 4) + (H + V) * 2, lambda i: O.linear_w8a16(ol, xl, ql[i % nl], scl[i % nl])))
    return ops, P


def measure_linear(L, hip, stream, e0, e1, steps):
    """Times the linear_ops cases."""
    print("bench: building linear buffers", file=sys.stderr, flush=True)
    lops, lpool = linear_ops(L, np.random.default_rng(13))
    res = time_cases(L, hip, stream, e0, e1, steps, lops)
    del lops, lpool
    print("bench: linear " + json.dumps(res), file=sys.stderr, flush=True)
    return res


def rearrange_ops(L, rng):
    """(name, "bytes", bytes per launch, launch(i)) for the strided copy behind
    Tensor::contiguous: q [2048, 12, 128] bf16 to head-major (rows of 256 B) and a
    [8192, 8192] bf16 transpose (LDS tiles); bytes = read + write."""
    O, BF = L.Ops, L.DataType.BF16
    P = Pool(L, rng)
    ops = []
    for label, shape, perm in (("q [2048, 12, 128] -> [12, 2048, 128] bf16", (2048, 12, 128), (1, 0, 2)),
                               ("transpose [8192, 8192] bf16", (8192, 8192), (1, 0))):
        n = int(np.prod(shape))
        sets = P.sets_for(2 * n * 2)
        src = [t.permute(*perm) for t in P.fill(shape, BF, sets)]
        dst = P.empty(src[0].shape(), BF, sets)
        ops.append((f"rearrange {label}", "bytes", 2 * n * 2,
                    lambda i, src=src, dst=dst, k=sets: O.rearrange(dst[i % k], src[i % k])))
    return ops, P


def sample_ops(L, rng):
    """(name, "bytes", logits bytes per launch, launch(i)) for llaisysRandomSample over one
    row of the Qwen2 vocabulary (bf16): the reference generate() defaults (T 0.8, top_p 0.8)
    with top_k 50 and 1024, and the greedy case (argmax).  Latency-bound (one 297 KB row)."""
    O, BF, I64 = L.Ops, L.DataType.BF16, L.DataType.I64
    P = Pool(L, rng)
    sets = 16
    lg = P.fill((1, V), BF, sets, 3.0)
    out = P.empty((1,), I64, 1)[0]
    return [(f"sample 1 x {V} bf16, T 0.8, top_k {k}, top_p 0.8", "bytes", V * 2,
             lambda i, k=k: O.random_sample(out, lg[i % sets], 0.8, k, 0.8, i)) for k in (50, 1024)] + [
        (f"sample 1 x {V} bf16, greedy (argmax)", "bytes", V * 2,
         lambda i: O.random_sample(out, lg[i % sets], 0.0, 50, 0.8, i))], P


def measure_rearrange(L, hip, stream, e0, e1, steps):
    print("bench: building rearrange and sampling buffers", file=sys.stderr, flush=True)
    rops, rpool = rearrange_ops(L, np.random.default_rng(17))
    sops, spool = sample_ops(L, np.random.default_rng(19))
    res = time_cases(L, hip, stream, e0, e1, steps, rops + sops)
    del rops, rpool, sops, spool
    print("bench: rearrange " + json.dumps(res), file=sys.stderr, flush=True)
    return res


def measure_decode(L, hip, stream, e0, e1, graphs=True, int8_only=False):
    """One Qwen2-1.5B decode step (DecodeChain) at context 4096, replayed as one HIP graph
    (graphs=False: eager launches, for kernel tracing), with INT8 and with bf16 projection
    weights, each with the norms and swiglu fused into the projections and as separate
    launches: ms per token, tokens/s, and the weight bytes streamed per token against HBM.
    int8_only: the fused INT8 chain alone."""
    res = {}
    variants = [(True, True), (True, False), (False, True), (False, False)]
    for int8, fused in variants:
        if int8_only and not (int8 and fused):
            continue
        label = ("INT8 weights (W8A16), INT8 KV" if int8 else "bf16 weights, INT8 KV") + \
            ("" if fused else ", norms and swiglu as separate launches")
        print(f"bench: building decode chain ({label})", file=sys.stderr, flush=True)
        dc = DecodeChain(L, int8, fused=fused)
        for i in range(2):
            dc.run(i)
        graph = None
        if graphs:
            graph = L.Graph.capture()
            dc.run(7)
            graph.end()
        step = graph.launch if graphs else dc.run
        for _ in range(3):
            step()
        nrep = 20
        hip.record(e0, stream)
        for _ in range(nrep):
            step()
        hip.record(e1, stream)
        ms = hip.elapsed_ms(e0, e1) / nrep
        wb = dc.weight_bytes()
        res[label] = {"ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
                      "weight_bytes": wb, "weight_GB_s": round(wb / (ms * 1e-3) / 1e9, 1),
                      "frac_peak": round(wb / (ms * 1e-3) / 1e9 / PEAK_GBS, 4),
                      "context": DecodeChain.CTX, "layers": DecodeChain.LAYERS,
                      "launch": "one HIP graph" if graphs else "eager"}
        assert L.take_device_error() == 0
        del graph, dc
    print("bench: decode " + json.dumps(res), file=sys.stderr, flush=True)
    return res


def cpu_baseline(seconds):
    """The oracle's restatement of the reference CPU ops (oracle/, pinned bit for bit to the
    compiled reference by tests/test_oracle.py; the reference itself never travels to the
    GPU box) on a row sample of config 1, single thread pinned to one core; GB/s with the
    same bytes formula as the GPU."""
    import oracle
    rng = np.random.default_rng(7)
    rows, srows, stok = 512, 128, 512
    x, r = bf16(rng, (rows, H)), bf16(rng, (rows, H))
    w = bf16(rng, (H,), 0.1, 1.0)
    q, k = bf16(rng, (stok, NH, D)), bf16(rng, (stok, NKV, D))
    pos = np.arange(stok, dtype=np.int64)
    g, u = bf16(rng, (srows, I)), bf16(rng, (srows, I))
    table = bf16(rng, (V, H), 0.02)
    ids = rng.integers(0, V, size=T).astype(np.int64)
    logits = bf16(rng, (1, V))
    tok = rows * H * 2
    work_bytes = ((T * 8 + 2 * T * H * 2) + (2 * tok + H * 2) + (4 * tok + H * 2)
                  + (2 * stok * (NH + NKV) * D * 2 + 2 * stok * 8) + 3 * srows * I * 2 + (V * 2 + 10))
    sample = (f"config-1 ops on a sample: embedding 8192 ids, rms_norm and add+rms_norm "
              f"{rows} rows, rope q+k {stok} tokens, swiglu {srows} rows, argmax [1,{V}]")

    def step():
        oracle.embedding(ids, table)
        oracle.rms_norm(x, w, 1e-6)
        oracle.add_rms_norm(x, r, w, 1e-6)
        oracle.rope(q, pos, 1e4)
        oracle.rope(k, pos, 1e4)
        oracle.swiglu(g, u)
        oracle.argmax(logits)
    kind = "port"
    saved = os.sched_getaffinity(0)
    os.sched_setaffinity(0, {min(saved)})
    try:
        step()
        n, t0 = 0, time.perf_counter()
        while True:
            step()
            n += 1
            el = time.perf_counter() - t0
            if el >= seconds:
                break
    finally:
        os.sched_setaffinity(0, saved)
    return {"value": round(work_bytes * n / el / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": sample + f"; {n} reps in {el:.1f} s", "cpu_model": _cpu_model()}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def summary_of(per_op, chain, configs):
    """Per-op fraction of peak (config 1), chain ms and tokens/s (config 4), config-3 fractions."""
    out = {"config1_frac_peak": {k: v["frac_peak"] for k, v in per_op.items()},
           "config1_us": {k: v["us"] for k, v in per_op.items()}}
    if chain is not None:
        out["chain_ms"] = chain["ms"]
        out["chain_tokens_per_s"] = chain["tokens_per_s"]
    if configs is not None and "config3" in configs:
        out["config3_frac_peak"] = {k: v["frac_peak"] for k, v in configs["config3"].items()}
    return out


def copy_floors():
    """Copy-kernel floors of the ops' traffic (llaisys_amd/csrc/floors/floors.cpp, built next
    to libllaisys.so): us per launch of a plain streaming kernel moving each op's bytes, and
    the config-4 chain with every op replaced by its copy kernel (ms).  Run as a child
    process on the same GPU; None when the program is missing."""
    exe = ROOT / "llaisys_amd" / "libllaisys" / "llaisys_floors"
    if not exe.is_file():
        return None
    import subprocess
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        print("bench: floors failed: " + r.stderr[-500:], file=sys.stderr, flush=True)
        return None
    return json.loads(r.stdout.strip().splitlines()[-1])


def traffic_of(kernel):
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (scaled by
    the counters' reading on a device copy of known size), read from profiles/traffic.txt
    ('<op> <fetch_bytes> <write_bytes>'), or None."""
    path = ROOT / "profiles" / "traffic.txt"
    if not path.is_file():
        return None
    for line in path.read_text().splitlines():
        parts = line.split("#", 1)[0].split()
        if len(parts) == 3 and parts[0] == kernel:
            return int(float(parts[1]) + float(parts[2]))
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-chain", action="store_true")
    ap.add_argument("--no-floors", action="store_true", help="skip the copy-kernel floors")
    ap.add_argument("--no-configs", action="store_true", help="skip configs 0, 2 and 3")
    ap.add_argument("--no-attention", action="store_true", help="skip the self-attention lines")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the self-attention lines (profiling); prints their JSON")
    ap.add_argument("--chain-only", action="store_true", help="only the config-4 chain: --steps graph replays (profiling), then its timing as JSON")
    ap.add_argument("--no-linear", action="store_true", help="skip the linear and rearrange lines")
    ap.add_argument("--decode", action="store_true",
                    help="also time the decode-step chain (model orchestration, off by default)")
    ap.add_argument("--no-decode", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode-step chain; prints its JSON")
    ap.add_argument("--decode-eager", action="store_true",
                    help="with --decode-only: the fused INT8 chain only, eager launches (kernel tracing)")
    ap.add_argument("--linear-only", action="store_true",
                    help="only the linear and rearrange lines (profiling); prints their JSON")
    ap.add_argument("--eager", action="store_true",
                    help="time per-op cases as eager launches instead of graph replays "
                         "(rocprofv3 kernel tracing of graph replays crashes the host process)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="3 dispatches of a 256 MiB device copy (counter calibration), then 3 of "
                         "each config-1 op, for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the per-layer "
              "ops shard by rows with no exchange; see the sharding notes)", file=sys.stderr)
        sys.exit(2)

    import llaisys_amd as L
    assert L.RuntimeAPI(L.DeviceType.AMD).get_device_count() >= 1, "no AMD GPU"
    hip = HipEvents()
    stream = L.context_stream(L.DeviceType.AMD, 0)
    api = L.RuntimeAPI(L.DeviceType.AMD)
    if args.chain_only:
        ch = Chain(L)
        graph = L.Graph.capture()
        ch.run()
        graph.end()
        for _ in range(args.steps):
            graph.launch()
        api.device_synchronize()
        us, us_mean = time_launches(hip, stream, lambda i: graph.launch(), batch=4)
        print(json.dumps({"chain_ms": round(us * 1e-3, 4), "chain_ms_mean": round(us_mean * 1e-3, 4),
                          "tokens_per_s": round(Chain.TOK / (us * 1e-6)),
                          "frac_peak": round(ch.bytes() / (us * 1e-6) / 1e9 / PEAK_GBS, 4)}))
        return
    if args.decode_only:
        print(json.dumps({"decode": measure_decode(L, hip, stream, hip.event(), hip.event(),
                                                   graphs=not args.decode_eager,
                                                   int8_only=args.decode_eager)}), flush=True)
        return
    if args.linear_only:
        res = measure_linear(L, hip, stream, e0=hip.event(), e1=hip.event(), steps=args.steps)
        res.update(measure_rearrange(L, hip, stream, e0=hip.event(), e1=hip.event(), steps=args.steps))
        print(json.dumps({"linear": res}), flush=True)
        return
    if args.attention_only:
        print(json.dumps({"attention": measure_attention(L, hip, stream, e0=hip.event(), e1=hip.event(),
                                                         steps=args.steps)}), flush=True)
        return
    print("bench: building config-1 buffers", file=sys.stderr, flush=True)
    wl = Workload(L)
    if args.traffic_probe:
        n = 256 << 20
        src, dst = L.Tensor((n,), L.DataType.U8, device=L.DeviceType.AMD), L.Tensor((n,), L.DataType.U8, device=L.DeviceType.AMD)
        for _ in range(3):
            api.memcpy_sync(dst.data_ptr(), src.data_ptr(), n, L.MemcpyKind.D2D)
        for name, _, fn in wl.ops():
            for i in range(3):
                fn(wl.sets[i % NSETS])
            api.device_synchronize()
        # then the chain's fused RoPE + INT8 KV append (2048 tokens) and the config-3
        # quantize / dequantize of W[8960, 1536], 3 dispatches each
        BF, I8, F32 = L.DataType.BF16, L.DataType.I8, L.DataType.F32
        dev = dict(device=L.DeviceType.AMD, device_id=0)
        rng = np.random.default_rng(5)
        t = Chain.TOK
        q, k, v = (L.Tensor.from_numpy(bf16(rng, shp), BF, **dev) for shp in ((t, NH, D), (t, NKV, D), (t, NKV, D)))
        qo, pos = L.Tensor((t, NH, D), BF, **dev), L.Tensor.from_numpy(np.arange(t, dtype=np.int64), **dev)
        kc, vc = L.Tensor((t, NKV, D), I8, **dev), L.Tensor((t, NKV, D), I8, **dev)
        ks, vs = L.Tensor((t, NKV), F32, **dev), L.Tensor((t, NKV), F32, **dev)
        w = L.Tensor.from_numpy(bf16(rng, (I, H), 0.02), BF, **dev)
        wq, wsc, wd = L.Tensor((I, H), I8, **dev), L.Tensor((I,), F32, **dev), L.Tensor((I, H), BF, **dev)
        for _ in range(3):
            L.Ops.rope_kv_append_int8(qo, q, k, v, pos, 1e6, kc, ks, vc, vs, 0)
        # the chain's add + rms_norm at 2048 rows (the one-vector-per-lane row kernel)
        x2, r2 = (L.Tensor.from_numpy(bf16(rng, (t, H)), BF, **dev) for _ in range(2))
        y2, h2 = L.Tensor((t, H), BF, **dev), L.Tensor((t, H), BF, **dev)
        nw = L.Tensor.from_numpy(bf16(rng, (H,), 0.1, 1.0), BF, **dev)
        for _ in range(3):
            L.Ops.add_rms_norm(y2, h2, x2, r2, nw, 1e-6)
        for _ in range(3):
            L.Ops.quantize_int8(wq, wsc, w)
        for _ in range(3):
            L.Ops.dequantize_int8(wd, wq, wsc)
        api.device_synchronize()
        print(json.dumps({"probe": "copy 256 MiB x3, then each config-1 op x3, RoPE+KV append (2048 "
                                   "tokens) x3, add+rms_norm [2048,1536] x3, quantize / dequantize "
                                   "W[8960,1536] x3",
                          "ops": {name: b for name, b, _ in wl.ops()}}))
        return
    ops = wl.ops()
    step_bytes = sum(b for _, b, _ in ops)

    def step(i):
        s = wl.sets[i % NSETS]
        for _, _, fn in ops:
            fn(s)

    for i in range(args.warmup):
        step(i)
    api.device_synchronize()
    e0, e1 = hip.event(), hip.event()
    t0 = time.perf_counter()
    hip.record(e0, stream)
    for i in range(args.steps):
        step(i)
    hip.record(e1, stream)
    api.device_synchronize()
    wall = time.perf_counter() - t0
    ms_step = hip.elapsed_ms(e0, e1) / args.steps
    assert L.take_device_error() == 0

    del wl
    print("bench: building config-1 per-op buffers", file=sys.stderr, flush=True)
    c1, c1pool = config1_ops(L, np.random.default_rng(3))
    per_op = {}
    for name, nbytes, fn in c1:
        med, mean = time_graph(L, hip, stream, fn, nbytes)
        per_op[name] = rate(med, nbytes, mean)
    assert L.take_device_error() == 0
    del c1, c1pool
    print("bench: per-op " + json.dumps(per_op), file=sys.stderr, flush=True)

    chain = None
    if not args.no_chain:
        print("bench: building config-4 chain buffers", file=sys.stderr, flush=True)
        ch = Chain(L)
        us_eager, _ = time_launches(hip, stream, lambda i: ch.run(), batch=2, reps=10, warmup=2)
        ms_eager = us_eager * 1e-3
        graph = L.Graph.capture()
        ch.run()
        graph.end()
        us, us_mean = time_launches(hip, stream, lambda i: graph.launch(), batch=4)
        ms = us * 1e-3
        del graph
        cb = ch.bytes()
        chain = {"workload": "config 4: 28 Qwen2-1.5B layers, 2048-token prefill, bf16, INT8 KV "
                             "append, final rms_norm + argmax over [2048, 151936]; replayed "
                             "as one HIP graph",
                 "ms": round(ms, 4), "ms_mean": round(us_mean * 1e-3, 4),
                 "timing": "median over 60 reps of 4 graph replays, after 10",
                 "tokens_per_s": round(Chain.TOK / (ms * 1e-3)),
                 "bytes": cb, "GB_s": round(cb / (ms * 1e-3) / 1e9, 1),
                 "frac_peak": round(cb / (ms * 1e-3) / 1e9 / PEAK_GBS, 4),
                 "ms_eager_launches": round(ms_eager, 4),
                 "tokens_per_s_eager": round(Chain.TOK / (ms_eager * 1e-3))}
        assert L.take_device_error() == 0
        del ch

    configs = None
    if not args.no_configs:
        print("bench: building config 0 / 2 / 3 buffers", file=sys.stderr, flush=True)
        cases, pool = config_ops(L, np.random.default_rng(9))
        configs = {}
        for cfg, name, nbytes, launches, fn in cases:
            med, mean = time_graph(L, hip, stream, fn, nbytes)
            configs.setdefault(cfg, {})[name] = dict(rate(med, nbytes, mean), launches=launches)
        assert L.take_device_error() == 0
        del cases, pool
        print("bench: configs " + json.dumps(configs), file=sys.stderr, flush=True)

    attention = None
    if not args.no_attention:
        attention = measure_attention(L, hip, stream, e0, e1, args.steps)
    decode = None
    if args.decode and not args.no_decode:
        decode = measure_decode(L, hip, stream, e0, e1)
    linear = None
    if not args.no_linear:
        linear = measure_linear(L, hip, stream, e0, e1, args.steps)
        linear.update(measure_rearrange(L, hip, stream, e0, e1, args.steps))

    floors = None if args.no_floors else copy_floors()
    if floors:
        print("bench: floors " + json.dumps(floors), file=sys.stderr, flush=True)
        for name, r in per_op.items():
            if name in floors:
                r["copy_floor_us"] = floors[name]
                r["frac_of_copy_floor"] = round(floors[name] / r["us"], 4)
        if chain is not None and "chain_ms" in floors:
            chain["copy_floor_ms"] = floors["chain_ms"]
            chain["frac_of_copy_floor"] = round(floors["chain_ms"] / chain["ms"], 4)
        if configs is not None:
            for key in ("config3 quantize W[8960,1536]", "config3 dequantize W[8960,1536]"):
                name = key.split(" ", 1)[1]
                r = configs.get("config3", {}).get(name)
                if r is not None and key in floors:
                    r["copy_floor_us"] = floors[key]
                    r["frac_of_copy_floor"] = round(floors[key] / r["us"], 4)

    dom = per_op["swiglu"]
    roof = {"kernel": "swiglu binaryVec<BF16> [8192, 8960]", "bound": "hbm",
            "achieved": dom["GB_s"], "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(dom["GB_s"] / PEAK_GBS, 4), "traffic": traffic_of("swiglu")}
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)

    value = step_bytes / (ms_step * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded normal activations, N(0,0.02) table), resident in HBM",
        "config": {"workload": "config 1: Qwen2-1.5B layer ops, bf16, 8192 tokens (embedding, "
                               "rms_norm, add+rms_norm, rope q+k (fused launch), swiglu, argmax [1,151936])",
                   "tokens": T, "hidden": H, "intermediate": I, "vocab": V,
                   "buffer_sets": NSETS, "parallelism": "single GPU"},
        "frac_peak": round(value / PEAK_GBS, 4),
        "tokens_per_s": round(T / (ms_step * 1e-3)),
        "wall_s_timed": round(wall, 3),
        "roofline": roof, "cpu_baseline": cpu,
        "attention": attention, "linear": linear, "decode": decode,
        "configs": configs,
        # the detailed hot-path figures last, and a compact summary at the very end, so that
        # a reader that keeps only the tail of the line still sees every per-op fraction
        "per_op": per_op, "chain": chain,
        "summary": summary_of(per_op, chain, configs),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
