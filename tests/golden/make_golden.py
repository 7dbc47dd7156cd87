"""Writes tests/golden/golden.npz: inputs and outputs of the REFERENCE CPU library.

Run in the build container, where `make -C oracle ref` compiled the reference's own
sources (/root/reference/src) into oracle/_ref/libllaisys_ref.so.  The script drives that
library through its C ABI (tensorCreate / tensorLoad / llaisys* ops on CPU tensors) with
this repository's ctypes binding; nothing of the reference's Python package is imported.

    python tests/golden/make_golden.py

Every case is seeded (numpy PCG64, seed per case); bf16 inputs are f32 samples rounded
with the reference rule, f16 inputs are numpy float16 casts.  Shapes follow the
reference's own op tests (test/ops/*.py) plus Qwen2-1.5B-sized rows and large RoPE
positions.  The fixture is data only: inputs and expected outputs.
"""
import ctypes
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from llaisys_amd.hostfmt import f32_to_bf16  # noqa: E402
from llaisys_amd.libllaisys import DataType, DeviceType, bind  # noqa: E402
from llaisys_amd.tensor import Tensor  # noqa: E402

OUT = Path(__file__).parent / "golden.npz"
DT = {"f32": DataType.F32, "bf16": DataType.BF16, "f16": DataType.F16}


def sample(rng, shape, dtype, scale=1.0, loc=0.0):
    x = (loc + scale * rng.standard_normal(shape)).astype(np.float32)
    if dtype == "bf16":
        return f32_to_bf16(x)
    if dtype == "f16":
        return x.astype(np.float16)
    return x


class Ref:
    def __init__(self, lib):
        self.lib = lib
        self.keep = []  # host tensors stay alive until the case is done

    def h(self, arr, dtype=None):
        t = self.t(arr, dtype)
        self.keep.append(t)
        return t.lib_tensor()

    def t(self, arr, dtype=None):
        return Tensor.from_numpy(arr, dtype, device=DeviceType.CPU, lib=self.lib)

    def empty(self, shape, dtype):
        return Tensor(shape, dtype, DeviceType.CPU, lib=self.lib)


def main():
    lib = oracle.reference_library()
    if lib is None:
        sys.exit("oracle/_ref/libllaisys_ref.so not built: run make -C oracle ref")
    bind(lib)
    R = Ref(lib)
    g = {}
    seed = [0]

    def rng():
        seed[0] += 1
        return np.random.default_rng(1000 + seed[0])

    for dt in ("f32", "bf16", "f16"):
        # rms_norm: reference test shapes (1,4), plus Qwen2 / Llama rows
        for shape, eps in (((1, 4), 1e-5), ((7, 1536), 1e-6), ((3, 4096), 1e-5), ((5, 1000), 1e-5)):
            r = rng()
            x = sample(r, shape, dt)
            w = sample(r, shape[-1:], dt, 0.1, 1.0)
            y = R.empty(shape, DT[dt])
            lib.llaisysRmsNorm(y.lib_tensor(), R.h(x, DT[dt]), R.h(w, DT[dt]), ctypes.c_float(eps))
            key = f"rms_norm/{dt}/{shape[0]}x{shape[1]}"
            g.update({f"{key}/x": x, f"{key}/w": w, f"{key}/eps": np.float32(eps), f"{key}/y": y.numpy()})

        # add: reference test shapes
        for shape in ((2, 3), (16, 1536)):
            r = rng()
            a, b = sample(r, shape, dt), sample(r, shape, dt)
            c = R.empty(shape, DT[dt])
            lib.llaisysAdd(c.lib_tensor(), R.h(a, DT[dt]), R.h(b, DT[dt]))
            key = f"add/{dt}/{shape[0]}x{shape[1]}"
            g.update({f"{key}/a": a, f"{key}/b": b, f"{key}/c": c.numpy()})

        # rope: reference test (2,1,4) pos 0..2; Qwen2 heads; late positions; theta 5e5; odd half
        for shape, p0, theta in (((2, 1, 4), 0, 1e4), ((16, 12, 128), 0, 1e4), ((8, 2, 128), 8184, 1e4),
                                 ((4, 8, 128), 16380, 5e5), ((3, 2, 6), 5, 1e4)):
            r = rng()
            x = sample(r, shape, dt)
            pos = np.arange(p0, p0 + shape[0], dtype=np.int64)
            y = R.empty(shape, DT[dt])
            lib.llaisysROPE(y.lib_tensor(), R.h(x, DT[dt]), R.h(pos, DataType.I64), ctypes.c_float(theta))
            key = f"rope/{dt}/{shape[0]}x{shape[1]}x{shape[2]}@{p0}"
            g.update({f"{key}/x": x, f"{key}/pos": pos, f"{key}/theta": np.float32(theta), f"{key}/y": y.numpy()})

        # swiglu: reference test (2,3), a Qwen2 row block, a wide gate range
        for shape, gs in (((2, 3), 1.0), ((2, 8960), 1.0), ((16, 256), 8.0)):
            r = rng()
            gt, up = sample(r, shape, dt, gs), sample(r, shape, dt)
            y = R.empty(shape, DT[dt])
            lib.llaisysSwiGLU(y.lib_tensor(), R.h(gt, DT[dt]), R.h(up, DT[dt]))
            key = f"swiglu/{dt}/{shape[0]}x{shape[1]}"
            g.update({f"{key}/gate": gt, f"{key}/up": up, f"{key}/y": y.numpy()})

        # argmax: random, planted ties (first wins), NaN later (ignored), NaN first, all -inf
        n = 4096
        r = rng()
        base = sample(r, (n,), dt).astype(np.float32 if dt == "f32" else sample(r, (1,), dt).dtype)
        cases = {"rand": base.copy()}
        tie = base.copy()
        hi = np.float32(50.0)
        hv = f32_to_bf16(hi).reshape(-1)[0] if dt == "bf16" else (np.float16(hi) if dt == "f16" else hi)
        tie[[700, 123, 3000]] = hv
        cases["tie"] = tie
        nanl = base.copy()
        nanv = f32_to_bf16(np.float32(np.nan)).reshape(-1)[0] if dt == "bf16" else (np.float16(np.nan) if dt == "f16" else np.float32(np.nan))
        nanl[[5, 77]] = nanv
        cases["nan_later"] = nanl
        nan0 = base.copy()
        nan0[0] = nanv
        cases["nan_first"] = nan0
        ninf = f32_to_bf16(np.float32(-np.inf)).reshape(-1)[0] if dt == "bf16" else (np.float16(-np.inf) if dt == "f16" else np.float32(-np.inf))
        cases["all_neg_inf"] = np.full(17, ninf, dtype=base.dtype)
        if dt == "bf16":
            cases["vocab"] = sample(r, (151936,), dt)
        for name, v in cases.items():
            mi, mv = R.empty((1,), DataType.I64), R.empty((1,), DT[dt])
            lib.llaisysArgmax(mi.lib_tensor(), mv.lib_tensor(), R.h(v, DT[dt]))
            key = f"argmax/{dt}/{name}"
            g.update({f"{key}/vals": v, f"{key}/idx": mi.numpy(), f"{key}/val": mv.numpy()})

    for dt in ("f32", "bf16"):
        # embedding: reference test (50 ids into 512 x 4096 scaled to 512 x 64), I32 and I64
        for idt, npi in ((DataType.I32, np.int32), (DataType.I64, np.int64)):
            r = rng()
            w = sample(r, (512, 64), dt, 0.02)
            idx = r.integers(0, 512, size=50).astype(npi)
            out = R.empty((50, 64), DT[dt])
            lib.llaisysEmbedding(out.lib_tensor(), R.h(idx, idt), R.h(w, DT[dt]))
            key = f"embedding/{dt}/{idt.name}"
            g.update({f"{key}/w": w, f"{key}/idx": idx, f"{key}/out": out.numpy()})

    # self_attention: the reference test shapes (test/ops/self_attention.py: qlen, kvlen, nh,
    # nkvh, hd = (2,2,1,1,4), (5,11,4,2,8)), a Qwen2-1.5B GQA decode row and prefill block
    # (12 q heads on 2 kv heads, head_dim 128), a single key, and seq_len > total_len (the
    # reference's size_t current_pos wraps, so the early queries see every key).  Seeds are
    # their own sequence, so the cases above keep their values.
    sa_seed = [0]

    def sa_rng():
        sa_seed[0] += 1
        return np.random.default_rng(5000 + sa_seed[0])

    for dt in ("f32", "bf16", "f16"):
        for ql, kl, nh, nkvh, hd in ((2, 2, 1, 1, 4), (5, 11, 4, 2, 8), (1, 37, 12, 2, 128),
                                     (16, 16, 12, 2, 128), (4, 1, 2, 1, 8), (3, 2, 2, 1, 8)):
            r = sa_rng()
            q = sample(r, (ql, nh, hd), dt)
            k = sample(r, (kl, nkvh, hd), dt)
            v = sample(r, (kl, nkvh, hd), dt)
            scale = np.float32(1.0 / hd ** 0.5)
            out = R.empty((ql, nh, hd), DT[dt])
            lib.llaisysSelfAttention(out.lib_tensor(), R.h(q, DT[dt]), R.h(k, DT[dt]), R.h(v, DT[dt]),
                                     ctypes.c_float(scale))
            key = f"self_attention/{dt}/{ql}x{kl}x{nh}x{nkvh}x{hd}"
            g.update({f"{key}/q": q, f"{key}/k": k, f"{key}/v": v, f"{key}/scale": scale,
                      f"{key}/out": out.numpy()})

    # linear: the reference test's small shape (x scale 0.1, w scale 0.01, bias N(0, 1)),
    # a Qwen2 row block with and without bias (the reference's "no bias" is a bias tensor
    # with no elements, op.cpp:22), and an odd in_features.  Own seed sequence.
    li_seed = [0]

    def li_rng():
        li_seed[0] += 1
        return np.random.default_rng(7000 + li_seed[0])

    for dt in ("f32", "bf16", "f16"):
        for rows, in_f, out_f, use_bias in ((2, 4, 3, True), (16, 1536, 64, True), (5, 96, 40, False),
                                            (3, 77, 9, True)):
            r = li_rng()
            x = sample(r, (rows, in_f), dt, 0.1)
            w = sample(r, (out_f, in_f), dt, 0.01)
            b = sample(r, (out_f,), dt) if use_bias else sample(r, (0,), dt)
            out = R.empty((rows, out_f), DT[dt])
            lib.llaisysLinear(out.lib_tensor(), R.h(x, DT[dt]), R.h(w, DT[dt]), R.h(b, DT[dt]))
            key = f"linear/{dt}/{rows}x{in_f}x{out_f}{'b' if use_bias else ''}"
            g.update({f"{key}/x": x, f"{key}/w": w, f"{key}/bias": b, f"{key}/out": out.numpy()})

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({OUT.stat().st_size / 1e6:.2f} MB, {len(g)} arrays)")


if __name__ == "__main__":
    main()
