"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the parity checker.

1. Golden vectors written by the compiled reference library (tests/golden/golden.npz):
   the oracle must reproduce every reference output bit for bit.
2. Where the reference library is built in this container (oracle/_ref), random shapes
   are compared with it directly.
3. The functions without a reference counterpart (INT8 quantize / dequantize / KV append,
   fused add + rms_norm, row-wise argmax) are pinned by closed forms: exactly known
   quotients and ties, invariants and compositions of already-pinned functions.
"""
import ctypes

import numpy as np
import pytest

import oracle
from llaisys_amd.hostfmt import bf16_to_f32, f32_to_bf16
from numerics import assert_exact

# ---- 1. reference golden vectors ----------------------------------------------------


def test_golden_rms_norm(golden):
    n = 0
    for (op, dt, case), c in golden.items():
        if op == "rms_norm":
            assert_exact(oracle.rms_norm(c["x"], c["w"], float(c["eps"])), c["y"], f"{dt} {case}")
            n += 1
    assert n == 12


def test_golden_add(golden):
    for (op, dt, case), c in golden.items():
        if op == "add":
            assert_exact(oracle.add(c["a"], c["b"]), c["c"], f"{dt} {case}")


def test_golden_rope(golden):
    n = 0
    for (op, dt, case), c in golden.items():
        if op == "rope":
            assert_exact(oracle.rope(c["x"], c["pos"], float(c["theta"])), c["y"], f"{dt} {case}")
            n += 1
    assert n == 15


def test_golden_swiglu(golden):
    for (op, dt, case), c in golden.items():
        if op == "swiglu":
            assert_exact(oracle.swiglu(c["gate"], c["up"]), c["y"], f"{dt} {case}")


def test_golden_embedding(golden):
    for (op, dt, case), c in golden.items():
        if op == "embedding":
            out, st = oracle.embedding(c["idx"], c["w"])
            assert st == 0
            assert_exact(out, c["out"], f"{dt} {case}")


def test_golden_argmax(golden):
    n = 0
    for (op, dt, case), c in golden.items():
        if op == "argmax":
            i, v = oracle.argmax(c["vals"])
            assert i == c["idx"][0], f"{dt} {case}"
            assert_exact(np.array([v]), c["val"], f"{dt} {case}")
            n += 1
    assert n == 16


# ---- 2. direct comparison with the compiled reference --------------------------------

@pytest.fixture(scope="module")
def ref():
    lib = oracle.reference_library()
    if lib is None:
        pytest.skip("reference library not built here (needs /root/reference)")
    from llaisys_amd.libllaisys import bind
    return bind(lib)


def _ref_call(lib, fn, outs, ins, *scalars):
    from llaisys_amd.libllaisys import DataType, DeviceType
    from llaisys_amd.tensor import Tensor
    keep = [Tensor.from_numpy(a, dt, device=DeviceType.CPU, lib=lib) for a, dt in ins]
    res = [Tensor(shape, dt, DeviceType.CPU, lib=lib) for shape, dt in outs]
    getattr(lib, fn)(*[t.lib_tensor() for t in res], *[t.lib_tensor() for t in keep], *scalars)
    return [t.numpy() for t in res]


@pytest.mark.parametrize("seed", range(6))
def test_random_shapes_match_reference(ref, seed):
    from llaisys_amd.libllaisys import DataType
    rng = np.random.default_rng(seed)
    for dt, conv in ((DataType.F32, lambda a: a), (DataType.BF16, f32_to_bf16),
                     (DataType.F16, lambda a: a.astype(np.float16))):
        rows, cols = int(rng.integers(1, 9)), int(rng.integers(1, 700))
        x = conv(rng.standard_normal((rows, cols)).astype(np.float32) * 3)
        w = conv(rng.standard_normal(cols).astype(np.float32))
        eps = float(rng.choice([1e-5, 1e-6]))
        (y,) = _ref_call(ref, "llaisysRmsNorm", [((rows, cols), dt)], [(x, dt), (w, dt)], ctypes.c_float(eps))
        assert_exact(oracle.rms_norm(x, w, eps), y, "rms_norm")
        (y,) = _ref_call(ref, "llaisysSwiGLU", [((rows, cols), dt)], [(x, dt), (x[::-1].copy(), dt)])
        assert_exact(oracle.swiglu(x, x[::-1].copy()), y, "swiglu")
        seq, nh, half = int(rng.integers(1, 6)), int(rng.integers(1, 4)), int(rng.integers(1, 70))
        q = conv(rng.standard_normal((seq, nh, 2 * half)).astype(np.float32))
        pos = rng.integers(0, 40000, size=seq).astype(np.int64)
        theta = float(rng.choice([1e4, 5e5, 1e6]))
        (y,) = _ref_call(ref, "llaisysROPE", [(q.shape, dt)], [(q, dt), (pos, DataType.I64)], ctypes.c_float(theta))
        assert_exact(oracle.rope(q, pos, theta), y, "rope")
        nkvh = int(rng.integers(1, 3))
        nh, hd = nkvh * int(rng.integers(1, 4)), int(rng.integers(1, 40))
        ql, kl = int(rng.integers(1, 7)), int(rng.integers(1, 30))
        qa = conv(rng.standard_normal((ql, nh, hd)).astype(np.float32))
        ka = conv(rng.standard_normal((kl, nkvh, hd)).astype(np.float32))
        va = conv(rng.standard_normal((kl, nkvh, hd)).astype(np.float32))
        sc = float(1.0 / np.sqrt(hd))
        (y,) = _ref_call(ref, "llaisysSelfAttention", [((ql, nh, hd), dt)], [(qa, dt), (ka, dt), (va, dt)],
                         ctypes.c_float(sc))
        assert_exact(oracle.self_attention(qa, ka, va, sc), y, "self_attention")


# ---- 3. closed forms -------------------------------------------------------------------

def test_bf16_rounding_rule():
    L = oracle.lib()
    cases = {
        0x3F808000: 0x3F80,  # exact tie, even LSB stays
        0x3F818000: 0x3F82,  # exact tie, odd LSB rounds up
        0x3F807FFF: 0x3F80,  # below half
        0x3F808001: 0x3F81,  # above half
        0x7F7FFFFF: 0x7F80,  # overflow rounds to +inf
        0xFF7FFFFF: 0xFF80,
        0x00000000: 0x0000,
        0x80000000: 0x8000,
    }
    for bits, want in cases.items():
        f = np.array([bits], dtype=np.uint32).view(np.float32)[0]
        assert L.orc_f32_to_bf16(float(f)) == want, hex(bits)
    # exhaustive widening: bf16 -> f32 is a 16-bit shift
    b = np.arange(1 << 16, dtype=np.uint32)
    f = bf16_to_f32(b.astype(np.uint16))
    assert np.array_equal(f.view(np.uint32), b << 16)
    # the host helper used to build inputs follows the same rule
    x = np.random.default_rng(1).standard_normal(10000).astype(np.float32)
    assert all(L.orc_f32_to_bf16(float(v)) == h for v, h in zip(x[:500], f32_to_bf16(x[:500])))


def test_f16_truncation_rule():
    L = oracle.lib()
    # f32 -> f16 truncates the mantissa (reference types.cpp:54-55)
    one_plus = np.float32(1.0) + np.float32(2.0 ** -11) * np.float32(1.9)  # above the f16 half-ulp
    assert L.orc_f32_to_f16(float(one_plus)) == 0x3C00
    assert L.orc_f32_to_f16(70000.0) == 0x7C00
    assert L.orc_f32_to_f16(float("nan")) == 0x7E00
    # f16 -> f32 is exact for every pattern (compare with numpy's exact widening)
    h = np.arange(1 << 16, dtype=np.uint16)
    fin = np.isfinite(h.view(np.float16))
    got = np.array([L.orc_f16_to_f32(int(v)) for v in h[fin][::97]], dtype=np.float32)
    assert np.array_equal(got, h[fin][::97].view(np.float16).astype(np.float32))


def test_rms_norm_closed_form():
    # a constant row c gives y_j = w_j * c / sqrt(c^2 + eps) (up to f32 rounding)
    for c, eps in ((0.5, 1e-6), (3.0, 1e-5), (1e-3, 1e-6)):
        x = np.full((2, 1536), c, dtype=np.float32)
        w = np.linspace(0.5, 1.5, 1536).astype(np.float32)
        y = oracle.rms_norm(x, w, eps)
        exact = w.astype(np.float64) * c / np.sqrt(c * c + eps)
        assert np.allclose(y, exact, rtol=2e-6), (c, eps)
    # eps matters: for tiny rows the result is x*w/sqrt(eps)
    x = np.full((1, 64), 1e-8, dtype=np.float32)
    y = oracle.rms_norm(x, np.ones(64, np.float32), 1e-2)
    assert np.allclose(y, 1e-8 / np.sqrt(1e-2), rtol=1e-5)


def test_rope_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 3, 16)).astype(np.float32)
    # position 0 is the identity
    assert_exact(oracle.rope(x, np.zeros(4, np.int64), 1e4), x)
    # head_dim 2: a single pair rotated by angle p (freq = theta^0 = 1)
    x2 = rng.standard_normal((5, 1, 2)).astype(np.float32)
    p = np.arange(5, dtype=np.int64) * 7
    y = oracle.rope(x2, p, 1e4)
    a, b = x2[:, 0, 0].astype(np.float64), x2[:, 0, 1].astype(np.float64)
    assert np.allclose(y[:, 0, 0], a * np.cos(p) - b * np.sin(p), rtol=1e-6, atol=1e-7)
    assert np.allclose(y[:, 0, 1], b * np.cos(p) + a * np.sin(p), rtol=1e-6, atol=1e-7)
    # rotation preserves the norm of every (j, j + d/2) pair, and pairs are (j, j+d/2)
    pos = np.arange(4, dtype=np.int64) * 1000
    y = oracle.rope(x, pos, 1e4)
    nx = x[..., :8] ** 2 + x[..., 8:] ** 2
    ny = y[..., :8] ** 2 + y[..., 8:] ** 2
    assert np.allclose(nx, ny, rtol=1e-5)
    # frequency j uses theta^(-2j/d): pair j=4 of d=16 at p=1 turns by 1e4^-0.5 = 0.01
    e = np.zeros((1, 1, 16), np.float32)
    e[0, 0, 4] = 1.0
    y = oracle.rope(e, np.ones(1, np.int64), 1e4)
    assert np.isclose(y[0, 0, 4], np.cos(0.01), rtol=1e-7) and np.isclose(y[0, 0, 12], np.sin(0.01), rtol=1e-6)


def test_swiglu_closed_forms():
    g = np.array([0.0, 40.0, -40.0, 1.0, -2.5], np.float32)
    u = np.array([3.0, 2.0, 5.0, 1.0, 4.0], np.float32)
    y = oracle.swiglu(g, u)
    assert y[0] == 0.0 and y[1] == 80.0 and abs(y[2]) < 1e-15
    silu = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    assert np.allclose(y[3:], (u * silu)[3:], rtol=1e-6)


def _pow2_row(k, odd):
    """Row with amax = 127 * 2^-k, so scale = 2^-k exactly and x / scale = odd / 2."""
    s = np.float32(2.0 ** -k)
    row = np.concatenate([[127 * s], odd.astype(np.float32) * s / 2]).astype(np.float32)
    return row, s


def test_int8_quantize_exact_quotients():
    odd = np.arange(-253, 254, 2)  # quotients -126.5 .. 126.5: every half-integer tie
    for k in (0, 4, 9):
        row, s = _pow2_row(k, odd)
        q, scale = oracle.quantize_int8(row[None, :])
        assert scale[0] == s
        assert q[0, 0] == 127
        half = odd / 2
        want = np.where(np.abs(half - np.floor(half)) == 0.5,
                        2 * np.round(half / 2), np.round(half))  # ties to even
        assert np.array_equal(q[0, 1:], want.astype(np.int8))
    # exact multiples give their multiplier; -amax gives -127
    s = np.float32(0.25)
    row = np.array([-127, -3, 0, 5, 126], np.float32) * s
    q, scale = oracle.quantize_int8(row[None, :])
    assert scale[0] == s and q.tolist() == [[-127, -3, 0, 5, 126]]


def test_int8_special_rows():
    rows = np.zeros((3, 8), np.float32)
    rows[1, 3] = np.nan
    rows[1, 5] = -2.0
    rows[2, :] = [1, -1, np.nan, 0.5, 0, 0, 0, 0]
    q, s = oracle.quantize_int8(rows)
    assert s[0] == 0 and not q[0].any()                     # all-zero row
    assert s[1] == np.float32(2.0) / np.float32(127.0)      # NaN ignored by amax
    assert q[1, 3] == 0 and q[1, 5] == -127                 # NaN code is 0
    assert q[2].tolist() == [127, -127, 0, 64, 0, 0, 0, 0]  # 63.5 rounds to even 64


def test_int8_roundtrip_bound_and_dequant():
    rng = np.random.default_rng(7)
    for dt in ("f32", "bf16"):
        x = rng.standard_normal((64, 128)).astype(np.float32)
        x[rng.random(x.shape) < 0.01] *= 20
        xin = x if dt == "f32" else f32_to_bf16(x)
        xf = xin if dt == "f32" else bf16_to_f32(xin)
        q, s = oracle.quantize_int8(xin)
        assert np.array_equal(s, np.abs(xf).max(axis=1) / np.float32(127))
        assert (np.abs(q).max(axis=1) == 127).all()
        deq = oracle.dequantize_int8(q, s, np.float32)
        assert np.array_equal(deq, q.astype(np.float32) * s[:, None])
        assert (np.abs(deq - xf) <= s[:, None] / 2 * (1 + 1e-6)).all()
        deq16 = oracle.dequantize_int8(q, s, np.uint16)
        assert np.array_equal(deq16, f32_to_bf16(deq))


def test_kv_append_writes_only_its_rows():
    rng = np.random.default_rng(9)
    kv = f32_to_bf16(rng.standard_normal((5, 2, 128)).astype(np.float32))
    cq = np.full((16, 2, 128), 99, np.int8)
    cs = np.full((16, 2), -1, np.float32)
    assert oracle.kv_append_int8(cq, cs, kv, 7) == 0
    q, s = oracle.quantize_int8(kv)
    assert np.array_equal(cq[7:12], q) and np.array_equal(cs[7:12], s)
    assert (cq[:7] == 99).all() and (cq[12:] == 99).all() and (cs[:7] == -1).all()
    assert oracle.kv_append_int8(cq, cs, kv, 12) == -1  # 12 + 5 > 16


def test_fused_add_rms_norm_is_the_composition(golden):
    # residual stream = the reference add (golden), output = rms_norm of that sum
    for (op, dt, case), c in golden.items():
        if op == "add" and case == "16x1536":
            w = np.ones(1536, dtype=c["a"].dtype) if dt != "bf16" else f32_to_bf16(np.ones(1536, np.float32))
            y, h = oracle.add_rms_norm(c["a"], c["b"], w, 1e-6)
            assert_exact(h, c["c"], dt)
            assert_exact(y, oracle.rms_norm(c["c"], w, 1e-6), dt)


def test_argmax_rows_is_rowwise_argmax(golden):
    vals = golden[("argmax", "bf16", "rand")]["vals"].reshape(4, 1024)
    idx, val = oracle.argmax_rows(vals)
    for r in range(4):
        i, v = oracle.argmax(vals[r])
        assert idx[r] == i and val[r] == v


def test_embedding_out_of_range():
    w = np.arange(12, dtype=np.float32).reshape(4, 3)
    out, st = oracle.embedding(np.array([1, 4], np.int64), w)
    assert st == -1 and np.array_equal(out[0], w[1])
    _, st = oracle.embedding(np.array([-1], np.int32), w)
    assert st == -1


# ---- self_attention ------------------------------------------------------------------

def test_golden_self_attention(golden):
    n = 0
    for (op, dt, case), c in golden.items():
        if op == "self_attention":
            got = oracle.self_attention(c["q"], c["k"], c["v"], float(c["scale"]))
            assert_exact(got, c["out"], f"{dt} {case}")
            n += 1
    assert n == 18


def _f32(a):
    return bf16_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)


def _attention_f64(q, k, v, scale):
    """Textbook causal GQA attention in f64 (the query at total - seq + i sees keys <= it)."""
    q, k, v = _f32(q).astype(np.float64), _f32(k).astype(np.float64), _f32(v).astype(np.float64)
    seq, nh, d = q.shape
    total, nkvh, _ = k.shape
    g = nh // nkvh
    out = np.zeros((seq, nh, v.shape[2]))
    for h in range(nh):
        for i in range(seq):
            cur = total - seq + i
            vis = total if cur < 0 else min(cur + 1, total)
            s = k[:vis, h // g] @ q[i, h] * scale
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ v[:vis, h // g]
    return out


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_self_attention_against_f64(dt):
    # GQA, causal offset total - seq, against the textbook formula in f64
    rng = np.random.default_rng(3)
    mk = lambda shape: f32_to_bf16(rng.standard_normal(shape).astype(np.float32)) if dt == "bf16" \
        else rng.standard_normal(shape).astype(np.float32)
    q, k, v = mk((7, 6, 16)), mk((19, 2, 16)), mk((19, 2, 16))
    got = _f32(oracle.self_attention(q, k, v, 0.25))
    exp = _attention_f64(q, k, v, 0.25)
    tol = 1e-5 if dt == "f32" else 2 ** -7
    assert np.abs(got - exp).max() <= tol * np.abs(exp).max()


def test_self_attention_closed_forms():
    rng = np.random.default_rng(4)
    # one key: softmax is exactly 1, the output is exactly v[0] of the head's kv head
    q = rng.standard_normal((3, 4, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 8)).astype(np.float32)
    v = rng.standard_normal((1, 2, 8)).astype(np.float32)
    out = oracle.self_attention(q, k, v, 0.3)
    for h in range(4):
        assert np.array_equal(out[:, h], np.broadcast_to(v[0, h // 2], (3, 8)))
    # equal keys: uniform weights over the visible keys -> prefix means of v
    total, seq = 9, 4
    k = np.ones((total, 1, 8), np.float32)
    v = rng.standard_normal((total, 1, 8)).astype(np.float32)
    q = rng.standard_normal((seq, 1, 8)).astype(np.float32)
    out = oracle.self_attention(q, k, v, 1.0)
    for i in range(seq):
        vis = total - seq + i + 1
        assert np.allclose(out[i, 0], v[:vis, 0].mean(0), rtol=1e-6, atol=1e-6)
    # causality: keys and values after a query's position do not change its output
    q = rng.standard_normal((5, 2, 8)).astype(np.float32)
    k = rng.standard_normal((12, 1, 8)).astype(np.float32)
    v = rng.standard_normal((12, 1, 8)).astype(np.float32)
    base = oracle.self_attention(q, k, v, 0.5)
    k2, v2 = k.copy(), v.copy()
    k2[9:] = 100.0
    v2[9:] = -100.0
    moved = oracle.self_attention(q, k2, v2, 0.5)
    assert np.array_equal(base[:2], moved[:2])      # queries at 7, 8 see keys 0..8 only
    assert not np.array_equal(base[2:], moved[2:])  # later queries see the changed keys
    # GQA mapping: q head h uses kv head h // (nh / nkvh), as a run with that head alone
    q = rng.standard_normal((3, 6, 8)).astype(np.float32)
    k = rng.standard_normal((10, 2, 8)).astype(np.float32)
    v = rng.standard_normal((10, 2, 8)).astype(np.float32)
    full = oracle.self_attention(q, k, v, 0.4)
    for h in range(6):
        one = oracle.self_attention(q[:, h:h + 1].copy(), k[:, h // 3:h // 3 + 1].copy(),
                                    v[:, h // 3:h // 3 + 1].copy(), 0.4)
        assert np.array_equal(full[:, h], one[:, 0])


def test_self_attention_int8kv_is_the_composition():
    rng = np.random.default_rng(6)
    q = f32_to_bf16(rng.standard_normal((4, 6, 16)).astype(np.float32))
    k = f32_to_bf16(rng.standard_normal((10, 2, 16)).astype(np.float32))
    v = f32_to_bf16(rng.standard_normal((10, 2, 16)).astype(np.float32))
    kq, ks = oracle.quantize_int8(k)
    vq, vs = oracle.quantize_int8(v)
    got = oracle.self_attention_int8kv(q, kq, ks, vq, vs, 0.25)
    exp = oracle.self_attention(q, oracle.dequantize_int8(kq, ks, np.uint16),
                                oracle.dequantize_int8(vq, vs, np.uint16), 0.25)
    assert_exact(got, exp)


# ---- linear and the W8A16 rule -----------------------------------------------------------

def test_golden_linear(golden):
    n = 0
    for (op, dt, case), c in golden.items():
        if op == "linear":
            b = c["bias"] if c["bias"].size else None
            assert_exact(oracle.linear(c["x"], c["w"], b), c["out"], f"{dt} {case}")
            n += 1
    assert n == 12


@pytest.mark.parametrize("seed", range(4))
def test_linear_random_shapes_match_reference(ref, seed):
    from llaisys_amd.libllaisys import DataType
    rng = np.random.default_rng(100 + seed)
    for dt, conv in ((DataType.F32, lambda a: a), (DataType.BF16, f32_to_bf16),
                     (DataType.F16, lambda a: a.astype(np.float16))):
        rows, in_f, out_f = int(rng.integers(1, 9)), int(rng.integers(1, 300)), int(rng.integers(1, 40))
        x = conv(rng.standard_normal((rows, in_f)).astype(np.float32))
        w = conv((0.05 * rng.standard_normal((out_f, in_f))).astype(np.float32))
        b = conv(rng.standard_normal(out_f).astype(np.float32))
        (y,) = _ref_call(ref, "llaisysLinear", [((rows, out_f), dt)], [(x, dt), (w, dt), (b, dt)])
        assert_exact(oracle.linear(x, w, b), y, "linear")


def test_linear_w8a16_closed_forms():
    rng = np.random.default_rng(12)
    x = f32_to_bf16(rng.standard_normal((6, 200)).astype(np.float32))
    codes = rng.integers(-127, 128, size=(30, 200)).astype(np.int8)
    bias = f32_to_bf16(rng.standard_normal(30).astype(np.float32))
    # scale 1: exactly the reference linear with the codes as weights (codes are exact in bf16)
    w = f32_to_bf16(codes.astype(np.float32))
    ones = np.ones(30, np.float32)
    assert_exact(oracle.linear_w8a16(x, codes, ones, bias), oracle.linear(x, w, bias))
    # power-of-two scales only shift the exponent of the f32 sum: scale 2^k, no bias, f32 out
    xf = bf16_to_f32(x)
    base = oracle.linear_w8a16(xf, codes, ones)
    for k in (-7, 3):
        sc = np.full(30, 2.0 ** k, np.float32)
        assert np.array_equal(oracle.linear_w8a16(xf, codes, sc), base * np.float32(2.0 ** k))
    # against f64: the products are exact, so the sum is within f32 accumulation error
    sc = (0.01 * rng.random(30) + 1e-3).astype(np.float32)
    got = oracle.linear_w8a16(xf, codes, sc, bias=None)
    exp = (xf.astype(np.float64) @ codes.T.astype(np.float64)) * sc.astype(np.float64)
    assert np.abs(got - exp).max() <= 1e-5 * np.abs(exp).max()


# ---- random sampling (no reference kernel; rule in oracle/oracle.h) ------------------------

def test_sample_exp2_against_math():
    ts = np.concatenate([-np.linspace(0, 120, 2000), -np.random.default_rng(3).random(500) * 30])
    for t in ts.astype(np.float32):
        got, exp = oracle.sample_exp2(t), 2.0 ** float(t)
        assert abs(got - exp) <= 2e-7 * exp, (t, got, exp)
    assert oracle.sample_exp2(-126.5) == 0.0 and oracle.sample_exp2(float("nan")) == 0.0


def test_splitmix64_known_answers():
    # the first three outputs of splitmix64 seeded with 0 (Steele, Lea and Flood 2014)
    gamma = 0x9E3779B97F4A7C15
    assert oracle.splitmix64(0) == 0xE220A8397B1DCDAF
    assert oracle.splitmix64(gamma) == 0x6E789E6AA1B965F4
    assert oracle.splitmix64(2 * gamma) == 0x06C45D188009454F


def _sample_rule(x, temperature, top_k, top_p, seed):
    """The sampling rule restated with Python integers (independent of oracle.c's loops)."""
    x = np.asarray(x, np.float32)
    if temperature <= 0 or top_k == 1:
        return int(np.argmax(x))
    inv = np.float32(1.0) / np.float32(temperature)
    z = (x * inv).astype(np.float32)
    z = np.where(np.isnan(z), np.float32(-np.inf), z).astype(np.float32)  # NaN orders as -inf
    bits = z.view(np.uint32).astype(np.int64)
    key = np.where(bits & 0x80000000, (~bits) & 0xFFFFFFFF, bits | 0x80000000)
    order = sorted(range(len(z)), key=lambda i: (-int(key[i]), i))[:min(top_k, len(z))]
    zmax = z[order[0]]
    with np.errstate(invalid="ignore"):
        d = [np.float32(0.0) if key[i] == key[order[0]] else np.float32(z[i] - zmax) for i in order]
    w = [int(np.float32(oracle.sample_exp2(di * np.float32(1.4426950408889634))) * np.float32(2 ** 31))
         for di in d]
    cum = np.cumsum(w, dtype=object)
    W = int(cum[-1])
    kept = len(order)
    if top_p < 1:
        target = max(1, int(float(np.float32(top_p)) * W)) if top_p > 0 else 1
        kept = next(j for j in range(len(order)) if cum[j] >= target) + 1
    wk = int(cum[kept - 1])
    r = ((oracle.splitmix64(seed) >> 40) * wk) >> 24
    return order[next(j for j in range(kept) if cum[j] > r)]


def test_random_sample_matches_the_rule_restated():
    rng = np.random.default_rng(21)
    for case in range(60):
        V = int(rng.integers(2, 400))
        x = (rng.standard_normal(V) * rng.choice([0.5, 3.0, 10.0])).astype(np.float32)
        if case % 3 == 0:  # ties
            x = np.round(x).astype(np.float32)
        T = float(rng.choice([0.0, 0.3, 0.8, 1.0, 2.5]))
        k = int(rng.choice([1, 2, 7, 50, 1024]))
        p = float(rng.choice([0.0, 0.2, 0.8, 0.95, 1.0]))
        seed = int(rng.integers(0, 2 ** 62))
        got = oracle.random_sample(x, T, k, p, seed)[0]
        assert got == _sample_rule(x, T, k, p, seed), (case, V, T, k, p)


def test_random_sample_nan_and_infinite_logits():
    """NaN logits order as -inf (never drawn while a number is among the candidates);
    infinite maxima share the mass equally; an all -inf / NaN row still draws a candidate."""
    rng = np.random.default_rng(23)
    x = rng.standard_normal(64).astype(np.float32)
    x[[3, 10, 40]] = np.nan
    x[11] = -np.nan
    for seed in range(200):
        got = oracle.random_sample(x, 0.8, 50, 0.9, seed)[0]
        assert not np.isnan(x[got])
        assert got == _sample_rule(x, 0.8, 50, 0.9, seed)
    y = x.copy()
    y[[5, 20]] = np.inf
    draws = [oracle.random_sample(y, 1.0, 8, 0.95, s)[0] for s in range(400)]
    assert set(draws) == {5, 20}
    assert 120 < draws.count(5) < 280
    for s in range(50):
        assert oracle.random_sample(y, 1.0, 8, 0.95, s)[0] == _sample_rule(y, 1.0, 8, 0.95, s)
    z = np.full(16, -np.inf, np.float32)
    z[[2, 9]] = np.nan
    draws = {oracle.random_sample(z, 1.0, 4, 1.0, s)[0] for s in range(100)}
    assert draws == {0, 1, 2, 3}  # the four lowest indices, equal weights
    for s in range(20):
        assert oracle.random_sample(z, 1.0, 4, 0.5, s)[0] == _sample_rule(z, 1.0, 4, 0.5, s)


def test_random_sample_greedy_cases_are_argmax():
    rng = np.random.default_rng(22)
    x = rng.standard_normal((5, 300)).astype(np.float32)
    x[2, 17] = x[2, 250] = x[2].max() + 1  # tie: the lower index wins
    am = np.argmax(x, axis=1)
    assert np.array_equal(oracle.random_sample(x, 0.0, 50, 0.9, 1), am)
    assert np.array_equal(oracle.random_sample(x, 0.8, 1, 0.9, 1), am)
    assert np.array_equal(oracle.random_sample(x, 0.8, 50, 0.0, 1), am)  # top_p <= 0: the top element
    with pytest.raises(ValueError):
        oracle.random_sample(x, 0.8, 2000, 0.9, 1)


def _chi2_ok(counts, probs, n):
    exp = np.asarray(probs) * n
    m = exp > 0
    assert counts[~m].sum() == 0, "sampled an excluded token"
    chi2 = float((((counts[m] - exp[m]) ** 2) / exp[m]).sum())
    dof = int(m.sum()) - 1
    return chi2 < dof + 6 * np.sqrt(2 * max(dof, 1)) + 10


def test_random_sample_distribution():
    x = np.array([2.0, 1.0, 0.5, 0.0, -1.0, 3.0, 0.2, -0.3], np.float32)
    n = 20000
    for T, k, p in ((1.0, 8, 1.0), (0.7, 3, 1.0), (1.0, 8, 0.6), (2.0, 5, 0.9)):
        z = x.astype(np.float64) / T
        order = np.argsort(-z, kind="stable")[:k]
        pr = np.exp(z[order] - z[order].max())
        pr /= pr.sum()
        keep = len(order) if p >= 1 else int(np.searchsorted(np.cumsum(pr), p - 1e-12) + 1)
        probs = np.zeros(len(x))
        probs[order[:keep]] = pr[:keep] / pr[:keep].sum()
        counts = np.bincount([oracle.random_sample(x, T, k, p, s)[0] for s in range(n)], minlength=len(x))
        assert _chi2_ok(counts, probs, n), (T, k, p, counts, probs * n)


def test_cast_is_the_reference_conversions_composed():
    """orc_cast (types.hpp:116-139) against the pinned scalar rules, composed in numpy:
    f32 -> bf16 round-half-even without a NaN case, f32 -> f16 truncation, exact widening,
    identity for equal types; special values and ties included."""
    rng = np.random.default_rng(51)
    f = (rng.standard_normal(4000) * 10.0 ** rng.integers(-8, 8, 4000)).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -3e-45, 65504.0, 65520.0, 1e6],
                       np.float32)
    raw = np.array([0x7FC00001, 0x7F800001, 0xFFC00000, 0x3F808000, 0x3F818000, 0x3F807FFF],
                   np.uint32).view(np.float32)
    f = np.concatenate([f, special, raw])
    bf = oracle.cast(f, oracle.BF16)
    assert np.array_equal(bf, f32_to_bf16(f))
    assert np.array_equal(oracle.cast(bf, oracle.F32).view(np.uint32), bf16_to_f32(bf).view(np.uint32))
    h = oracle.cast(f, oracle.F16)
    exp_h = np.array([oracle.lib().orc_f32_to_f16(float(v)) for v in f], np.uint16)
    assert np.array_equal(h.view(np.uint16), exp_h)
    assert h.view(np.uint16)[np.where(f == np.float32(65520.0))[0][0]] == 0x7BFF  # truncates, no overflow to inf
    wide = np.array([oracle.lib().orc_f16_to_f32(int(v)) for v in h.view(np.uint16)], np.float32)
    assert np.array_equal(oracle.cast(h, oracle.F32).view(np.uint32), wide.view(np.uint32))
    # bf16 <-> f16 go through f32
    assert np.array_equal(oracle.cast(bf, oracle.F16).view(np.uint16),
                          oracle.cast(bf16_to_f32(bf), oracle.F16).view(np.uint16))
    assert np.array_equal(oracle.cast(h, oracle.BF16), f32_to_bf16(oracle.cast(h, oracle.F32)))
    for a in (f, bf, h):  # same type: the bits themselves
        code = {np.float32: oracle.F32, np.uint16: oracle.BF16, np.float16: oracle.F16}[a.dtype.type]
        assert np.array_equal(oracle.cast(a, code).view(np.uint8), a.view(np.uint8))
