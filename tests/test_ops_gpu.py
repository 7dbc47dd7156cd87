"""Parity of the gfx950 kernels with the CPU oracle and the reference golden vectors.

Every test calls the ops through the C ABI (llaisys_amd.Ops -> libllaisys.so) on device
AMD:0 and compares with oracle/ (itself pinned to the reference, tests/test_oracle.py)
under the rules of tests/numerics.py: integer work bit-exact, f32 1e-5 relative, bf16 and
f16 within 2 ulps.  Shapes: the reference tests' own, the BASELINE configs (full size where
the single-thread oracle finishes in seconds) and edge cases that take the scalar kernels
(ragged rows, unaligned slices) or the boundary paths (empty, NaN / tie / -inf, out-of-range
ids, appends at the cache end).
"""
import zlib

import numpy as np
import pytest

import llaisys_amd as L
import oracle
from llaisys_amd.hostfmt import bf16_to_f32, f32_to_bf16
from numerics import assert_attention_close, assert_close, assert_exact, assert_linear_close

pytestmark = pytest.mark.gpu

AMD = dict(device=L.DeviceType.AMD, device_id=0)
DTS = {"f32": L.DataType.F32, "bf16": L.DataType.BF16, "f16": L.DataType.F16}


@pytest.fixture(scope="module", autouse=True)
def gpu_present():
    n = L.RuntimeAPI(L.DeviceType.AMD).get_device_count()
    assert n >= 1, "no AMD GPU visible: the gpu tests need the HIP path"


def sample(rng, shape, dt, scale=1.0, loc=0.0):
    x = (loc + scale * rng.standard_normal(shape, dtype=np.float32)).astype(np.float32)
    return {"f32": x, "bf16": f32_to_bf16(x), "f16": x.astype(np.float16)}[dt]


def seed_of(*args):
    """Deterministic per-case seed (str hashes are salted per process)."""
    return zlib.crc32(repr(args).encode())


def dev(a, dt=None):
    return L.Tensor.from_numpy(a, dt, **AMD)


def empty(shape, dt):
    return L.Tensor(shape, dt, **AMD)


def no_device_error():
    assert L.take_device_error() == 0


# ---- reference golden vectors -------------------------------------------------------

def test_golden_vectors_on_gpu(golden):
    checked = 0
    for (op, dt, case), c in golden.items():
        what = f"{op}/{dt}/{case}"
        if op == "rms_norm":
            y = empty(c["x"].shape, DTS[dt])
            L.Ops.rms_norm(y, dev(c["x"], DTS[dt]), dev(c["w"], DTS[dt]), float(c["eps"]))
            assert_close(y.numpy(), c["y"], what)
        elif op == "add":
            out = empty(c["a"].shape, DTS[dt])
            L.Ops.add(out, dev(c["a"], DTS[dt]), dev(c["b"], DTS[dt]))
            assert_exact(out.numpy(), c["c"], what)  # one rounding of an exact f32 sum
        elif op == "rope":
            y = empty(c["x"].shape, DTS[dt])
            L.Ops.rope(y, dev(c["x"], DTS[dt]), dev(c["pos"]), float(c["theta"]))
            assert_close(y.numpy(), c["y"], what)
        elif op == "swiglu":
            y = empty(c["gate"].shape, DTS[dt])
            L.Ops.swiglu(y, dev(c["gate"], DTS[dt]), dev(c["up"], DTS[dt]))
            assert_close(y.numpy(), c["y"], what)
        elif op == "embedding":
            out = empty(c["out"].shape, DTS[dt])
            L.Ops.embedding(out, dev(c["idx"]), dev(c["w"], DTS[dt]))
            assert_exact(out.numpy(), c["out"], what)
        elif op == "argmax":
            i, v = empty((1,), L.DataType.I64), empty((1,), DTS[dt])
            L.Ops.argmax(i, v, dev(c["vals"], DTS[dt]))
            assert_exact(i.numpy(), c["idx"], what)
            assert_exact(v.numpy(), c["val"], what)
        elif op == "self_attention":
            out = empty(c["out"].shape, DTS[dt])
            L.Ops.self_attention(out, dev(c["q"], DTS[dt]), dev(c["k"], DTS[dt]), dev(c["v"], DTS[dt]),
                                 float(c["scale"]))
            assert_attention_close(out.numpy(), c["out"], c["v"], what)
        elif op == "linear":
            out = empty(c["out"].shape, DTS[dt])
            L.Ops.linear(out, dev(c["x"], DTS[dt]), dev(c["w"], DTS[dt]), dev(c["bias"], DTS[dt]))
            assert_linear_close(out.numpy(), c["out"], c["x"], c["w"], what)
        else:
            continue
        checked += 1
    assert checked == len(golden)
    no_device_error()


# ---- rms_norm and the fused residual variant -----------------------------------------

RMS_SHAPES = [
    ((1, 4), 1e-5), ((512, 4096), 1e-5),        # reference test shapes
    ((128, 1536), 1e-6),                        # config 0 (f32) / Qwen2 hidden
    ((8192, 1536), 1e-6),                       # config 1
    ((64, 8960), 1e-6),                         # 1024-lane rows
    ((65, 1536), 1e-6), ((100, 4096), 1e-5),    # one vector per lane, one row per block
    ((33, 1000), 1e-5), ((5, 20000), 1e-5),     # ragged / wider than the register plan
    ((3, 8), 1e-5), ((2, 100000), 1e-6),        # tiny, huge rows (scalar kernel)
]


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape,eps", RMS_SHAPES)
def test_rms_norm(dt, shape, eps):
    rng = np.random.default_rng(seed_of(shape, dt))
    x, w = sample(rng, shape, dt), sample(rng, shape[-1:], dt, 0.1, 1.0)
    y = empty(shape, DTS[dt])
    L.Ops.rms_norm(y, dev(x, DTS[dt]), dev(w, DTS[dt]), eps)
    got, exp = y.numpy(), oracle.rms_norm(x, w, eps)
    if dt == "f32" and shape[-1] > 16384:
        # The reference sums 1e5 squares left to right in f32; that sum alone drifts by up
        # to ~1e-5 relative, while the kernel's tree sum stays near the exact value.  Both
        # are checked: 1e-5 against the f64-accumulated value, 3e-5 against the oracle.
        xf = x.astype(np.float64)
        exact = (xf * w) / np.sqrt((xf * xf).mean(axis=-1, keepdims=True) + eps)
        assert np.abs(got - exact).max() <= 1e-5 * np.abs(exact).max()
        assert (np.abs(got - exp) <= 3e-5 * np.abs(exp)).all()
        return
    assert_close(got, exp, f"rms_norm {dt} {shape}")


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", [(8192, 1536), (2048, 1536), (300, 4096), (65, 1536), (7, 4096),
                                   (9, 1000), (1, 12)])
def test_add_rms_norm(dt, shape):
    rng = np.random.default_rng(11)
    x, r = sample(rng, shape, dt), sample(rng, shape, dt)
    w = sample(rng, shape[-1:], dt, 0.1, 1.0)
    y, h = empty(shape, DTS[dt]), empty(shape, DTS[dt])
    L.Ops.add_rms_norm(y, h, dev(x, DTS[dt]), dev(r, DTS[dt]), dev(w, DTS[dt]), 1e-6)
    ey, eh = oracle.add_rms_norm(x, r, w, 1e-6)
    assert_exact(h.numpy(), eh, "residual")  # the residual stream is bit-exact
    assert_close(y.numpy(), ey, "normed")


def test_add_rms_norm_in_place_residual():
    rng = np.random.default_rng(12)
    x, r = sample(rng, (256, 1536), "bf16"), sample(rng, (256, 1536), "bf16")
    w = sample(rng, (1536,), "bf16", 0.1, 1.0)
    tr = dev(r, L.DataType.BF16)
    y = empty((256, 1536), L.DataType.BF16)
    L.Ops.add_rms_norm(y, tr, dev(x, L.DataType.BF16), tr, dev(w, L.DataType.BF16), 1e-6)
    ey, eh = oracle.add_rms_norm(x, r, w, 1e-6)
    assert_exact(tr.numpy(), eh)
    assert_close(y.numpy(), ey)


def test_rms_norm_unaligned_slice_takes_the_scalar_path():
    rng = np.random.default_rng(13)
    x = sample(rng, (9, 1536), "bf16")
    w = sample(rng, (1536,), "bf16", 0.1, 1.0)
    big = dev(np.concatenate([np.zeros(3, np.uint16), x.reshape(-1)]), L.DataType.BF16)
    xs = big.slice(0, 3, 3 + x.size).view(9, 1536)  # 6-byte offset: not 16-byte aligned
    y = empty((9, 1536), L.DataType.BF16)
    L.Ops.rms_norm(y, xs, dev(w, L.DataType.BF16), 1e-6)
    assert_close(y.numpy(), oracle.rms_norm(x, w, 1e-6))


# ---- rope ------------------------------------------------------------------------------

ROPE = [
    ((2, 1, 4), 0, 1e4),            # reference test
    ((512, 4, 4096), 512, 1e4),     # reference test (head_dim 4096: scalar kernel)
    ((128, 12, 128), 0, 1e4),       # config 0 q
    ((128, 2, 128), 0, 1e4),        # config 0 k
    ((8192, 12, 128), 0, 1e4),      # config 1 q
    ((8192, 2, 128), 0, 1e4),       # config 1 k
    ((64, 32, 128), 16320, 5e5),    # config 2 heads, late positions
    ((7, 3, 6), 3, 1e4),            # odd half-dim
    ((5, 4, 64), 100000, 1e6),
    # one wave per token over one instruction, 1/4 of the lanes busy (one 128-wide head, two
    # 64-wide heads), and 1/8 (one 64-wide head: tokens packed per block)
    ((33, 1, 128), 70, 1e4),
    ((40, 2, 64), 0, 1e6),
    ((41, 1, 64), 5, 1e4),
    # half-pair layout at other widths: head_dim 256 (the widest), 16 (two-lane groups,
    # eight rows fill a quarter wave), and 8 rows of 128 (16-byte chunks over one wave
    # instruction); two 16-wide heads fall back to ropeVec
    ((9, 3, 256), 11, 1e4),
    ((13, 8, 16), 0, 1e4),
    ((13, 2, 16), 0, 1e4),
    ((19, 8, 128), 3, 1e4),
    # tokens packed per row instruction (one tensor filling 1/2 or 1/4 of it), ragged counts
    ((8193, 2, 128), 7, 1e4),
    ((8191, 1, 128), 0, 1e4),
    # one tensor of 9-15 rows per token, 4 tokens per wave as flat row runs (16-bit types):
    # the last wave's group ragged, 5 and 7 row instructions per wave
    ((8195, 12, 128), 5, 1e4),
    ((8190, 9, 128), 3, 1e4),
    ((8189, 14, 128), 0, 1e6),
]


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape,p0,theta", ROPE)
def test_rope(dt, shape, p0, theta):
    if shape == (512, 4, 4096) and dt != "bf16":
        pytest.skip("one dtype is enough for the 8M-element reference shape")
    rng = np.random.default_rng(seed_of(shape, dt))
    x = sample(rng, shape, dt)
    pos = np.arange(p0, p0 + shape[0], dtype=np.int64)
    y = empty(shape, DTS[dt])
    L.Ops.rope(y, dev(x, DTS[dt]), dev(pos), theta)
    assert_close(y.numpy(), oracle.rope(x, pos, theta), f"rope {dt} {shape}")


@pytest.mark.parametrize("shape", [(300, 2, 128), (8194, 12, 128)])
def test_rope_shuffled_positions(shape):
    """Random positions: a lane that took a neighbouring token's (cos, sin) pairs would
    show (the flat row runs of the second shape put several tokens in one row instruction)."""
    rng = np.random.default_rng(14)
    x = sample(rng, shape, "bf16")
    pos = rng.integers(0, 32768, size=shape[0]).astype(np.int64)
    y = empty(x.shape, L.DataType.BF16)
    L.Ops.rope(y, dev(x, L.DataType.BF16), dev(pos), 1e4)
    assert_close(y.numpy(), oracle.rope(x, pos, 1e4))


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("seq,nhq,nhk", [
    (8192, 12, 2),   # q + k, four tokens per wave
    (8192, 2, 0),    # k alone, two tokens per row instruction
    (8192, 12, 0),   # q alone, four tokens per wave as flat row runs (16-bit types)
    (64, 12, 2),     # two waves per token
])
def test_rope_far_angles(dt, seq, nhq, nhk):
    """Positions up to 2^40: angles beyond the reduced-argument range (|angle| > 2^30) take
    the device library's sincos inside each kernel layout; every fourth position is small,
    so waves mix both paths."""
    rng = np.random.default_rng(seed_of(seq, nhq, nhk, dt))
    pos = rng.integers(0, 2 ** 40, size=seq).astype(np.int64)
    pos[::4] = rng.integers(0, 4096, size=len(pos[::4]))
    q = sample(rng, (seq, nhq, 128), dt)
    qo = empty(q.shape, DTS[dt])
    if nhk:
        k = sample(rng, (seq, nhk, 128), dt)
        ko = empty(k.shape, DTS[dt])
        L.Ops.rope_qk(qo, dev(q, DTS[dt]), ko, dev(k, DTS[dt]), dev(pos), 1e4)
        assert_close(ko.numpy(), oracle.rope(k, pos, 1e4), "k")
    else:
        L.Ops.rope(qo, dev(q, DTS[dt]), dev(pos), 1e4)
    assert_close(qo.numpy(), oracle.rope(q, pos, 1e4), "q")


# ---- swiglu / add ------------------------------------------------------------------------

@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape,gs", [((2, 3), 1.0), ((512, 4096), 1.0), ((128, 8960), 1.0),
                                      ((8192, 8960), 1.0), ((33, 1001), 6.0)])
def test_swiglu(dt, shape, gs):
    if shape == (8192, 8960) and dt == "f16":
        pytest.skip("covered in f32 and bf16")
    rng = np.random.default_rng(seed_of(shape, dt))
    g, u = sample(rng, shape, dt, gs), sample(rng, shape, dt)
    y = empty(shape, DTS[dt])
    L.Ops.swiglu(y, dev(g, DTS[dt]), dev(u, DTS[dt]))
    assert_close(y.numpy(), oracle.swiglu(g, u), f"swiglu {dt} {shape}")


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", [(2, 3), (512, 4096), (13, 1001)])
def test_add(dt, shape):
    rng = np.random.default_rng(5)
    a, b = sample(rng, shape, dt), sample(rng, shape, dt)
    c = empty(shape, DTS[dt])
    L.Ops.add(c, dev(a, DTS[dt]), dev(b, DTS[dt]))
    assert_exact(c.numpy(), oracle.add(a, b))


# ---- embedding ---------------------------------------------------------------------------

_TABLES = {}


def table(vocab, dim, dt):
    """Embedding tables are built once per shape (the Qwen2 table is 233M elements)."""
    key = (vocab, dim, dt)
    if key not in _TABLES:
        _TABLES.clear()
        w = sample(np.random.default_rng(vocab + dim), (vocab, dim), dt, 0.02)
        _TABLES[key] = (w, dev(w, DTS[dt]))
    return _TABLES[key]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("vocab,dim", [(151936, 1536), (512, 4096), (1000, 3), (300, 1001)])
@pytest.mark.parametrize("n", [1, 50, 128, 8192])
@pytest.mark.parametrize("idt", [np.int32, np.int64])
def test_embedding(dt, vocab, dim, n, idt):
    rng = np.random.default_rng(vocab + dim + n)
    w, tw = table(vocab, dim, dt)
    idx = rng.integers(0, vocab, size=n).astype(idt)
    idx[: min(n, 3)] = [0, vocab - 1, 0][: min(n, 3)]
    out = empty((n, dim), DTS[dt])
    L.Ops.embedding(out, dev(idx), tw)
    exp, st = oracle.embedding(idx, w)
    assert st == 0
    assert_exact(out.numpy(), exp)
    no_device_error()


def test_embedding_out_of_range_sets_the_device_error():
    w = sample(np.random.default_rng(0), (64, 256), "bf16")
    idx = np.array([3, 64, -1, 5], np.int64)
    out = dev(np.zeros((4, 256), np.uint16), L.DataType.BF16)
    L.Ops.embedding(out, dev(idx), dev(w, L.DataType.BF16))
    assert L.take_device_error() == 1
    got = out.numpy()
    assert np.array_equal(got[0], w[3]) and np.array_equal(got[3], w[5])
    assert not got[1].any() and not got[2].any()  # out-of-range rows untouched
    assert L.take_device_error() == 0  # the error word was cleared
    # Qwen2 rows (8 ids per wavefront): bad ids inside full and partial groups
    w2 = sample(np.random.default_rng(1), (1000, 1536), "bf16")
    idx2 = np.arange(40, dtype=np.int64) * 7
    idx2[[5, 17, 38]] = [1000, -3, 2 ** 40]
    out2 = dev(np.zeros((40, 1536), np.uint16), L.DataType.BF16)
    L.Ops.embedding(out2, dev(idx2), dev(w2, L.DataType.BF16))
    assert L.take_device_error() == 1
    got2 = out2.numpy()
    good = np.ones(40, bool)
    good[[5, 17, 38]] = False
    assert np.array_equal(got2[good], w2[idx2[good]])
    assert not got2[~good].any()


# ---- argmax ------------------------------------------------------------------------------

@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n", [1, 4, 4096, 151936, 8193, 3_000_001])
@pytest.mark.parametrize("idt", [L.DataType.I64, L.DataType.I32])
def test_argmax_flat(dt, n, idt):
    rng = np.random.default_rng(n)
    v = sample(rng, (n,), dt)
    i, m = empty((1,), idt), empty((1,), DTS[dt])
    L.Ops.argmax(i, m, dev(v, DTS[dt]))
    ei, ev = oracle.argmax(v, np.int64 if idt == L.DataType.I64 else np.int32)
    assert i.numpy()[0] == ei
    assert_exact(m.numpy(), np.array([ev]))


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_argmax_ties_nans_and_infs(dt):
    rng = np.random.default_rng(3)
    n = 151936
    base = sample(rng, (n,), dt)
    hi = sample(rng, (1,), dt, 0, 9.0)[0]
    nan = sample(rng, (1,), dt, 0, np.nan)[0]
    ninf = sample(rng, (1,), dt, 0, -np.inf)[0]
    cases = []
    t = base.copy(); t[[90000, 4097, 150000, 4096 + 8 * 256]] = hi; cases.append(t)  # ties across blocks
    t = base.copy(); t[[1, 5000, 151935]] = nan; cases.append(t)                     # NaN never wins
    t = base.copy(); t[0] = nan; cases.append(t)                                      # NaN at 0 wins
    cases.append(np.full(n, ninf, dtype=base.dtype))                                 # all -inf -> 0
    t = np.full(n, ninf, dtype=base.dtype); t[77777] = nan; cases.append(t)
    t = np.full(n, hi, dtype=base.dtype); cases.append(t)                            # all equal -> 0
    for k, v in enumerate(cases):
        i, m = empty((1,), L.DataType.I64), empty((1,), DTS[dt])
        L.Ops.argmax(i, m, dev(v, DTS[dt]))
        ei, ev = oracle.argmax(v)
        assert i.numpy()[0] == ei, (dt, k)
        assert_exact(m.numpy(), np.array([ev]), f"{dt} case {k}")
        # the row variant agrees on the same data
        ri, rm = empty((2,), L.DataType.I64), empty((2,), DTS[dt])
        L.Ops.argmax_rows(ri, rm, dev(np.stack([v, v[::-1]]), DTS[dt]))
        eri, erm = oracle.argmax_rows(np.stack([v, v[::-1]]))
        assert np.array_equal(ri.numpy(), eri)
        assert_exact(rm.numpy(), erm)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("rows,cols", [(2048, 151936), (3, 1001), (64, 7), (1, 151936)])
def test_argmax_rows(dt, rows, cols):
    rng = np.random.default_rng(rows * cols)
    v = sample(rng, (rows, cols), dt)
    v[1 % rows, 10 % cols] = v[1 % rows].max()  # a tie in row 1
    i, m = empty((rows,), L.DataType.I32), empty((rows,), DTS[dt])
    L.Ops.argmax_rows(i, m, dev(v, DTS[dt]))
    ei, ev = oracle.argmax_rows(v, np.int32)
    assert_exact(i.numpy(), ei)
    assert_exact(m.numpy(), ev)


# ---- INT8 quantization -------------------------------------------------------------------

def with_outliers(rng, shape, dt, scale):
    x = (scale * rng.standard_normal(shape)).astype(np.float32)
    x[rng.random(shape) < 0.01] *= 20
    return {"f32": x, "bf16": f32_to_bf16(x), "f16": x.astype(np.float16)}[dt]


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", [(8960, 1536), (1536, 8960), (4096, 128), (5, 1001), (3, 20000), (7, 8),
                                   # one wave per row with a partial last lane group (125 / 129
                                   # bf16 vectors, 250 f32), and exactly 256 bf16 vectors
                                   (33, 1000), (17, 1032), (9, 2048),
                                   # one-wavefront blocks of 4 / 8 / 16 / 32-lane groups with
                                   # partial groups (bf16: 4, 25, 9, 1 vectors; f32: 8, 50, 18, 2)
                                   (301, 32), (65, 200), (130, 72), (3, 8),
                                   # one wave per row in one-wavefront blocks, 8 / 12 / 18
                                   # vectors per lane (bf16: 512, 750, 1025 vectors)
                                   (5, 4096), (3, 6000), (4, 8200)])
def test_quantize_dequantize(dt, shape):
    rng = np.random.default_rng(shape[0])
    x = with_outliers(rng, shape, dt, 0.02)
    x[0] = 0  # an all-zero row
    q, s = empty(shape, L.DataType.I8), empty(shape[:-1], L.DataType.F32)
    tx = dev(x, DTS[dt])
    L.Ops.quantize_int8(q, s, tx)
    eq, es = oracle.quantize_int8(x)
    assert_exact(q.numpy(), eq, "codes")
    assert_exact(s.numpy(), es, "scales")
    out = empty(shape, DTS[dt])
    L.Ops.dequantize_int8(out, q, s)
    assert_exact(out.numpy(), oracle.dequantize_int8(eq, es, x.dtype), "dequant")


def test_quantize_exact_ties_on_gpu():
    # scale = 2^-4 exactly; quotients k + 0.5 must round half to even, bit-exact
    s = np.float32(2.0 ** -4)
    odd = np.arange(-253, 254, 2)
    row = np.concatenate([[127 * s], odd.astype(np.float32) * s / 2, np.zeros(512 - 255, np.float32)])
    x = np.tile(row.astype(np.float32), (4, 1))
    x[2, 7] = np.nan
    q, sc = empty(x.shape, L.DataType.I8), empty((4,), L.DataType.F32)
    L.Ops.quantize_int8(q, sc, dev(x))
    eq, es = oracle.quantize_int8(x)
    assert_exact(q.numpy(), eq)
    assert_exact(sc.numpy(), es)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_kv_append(dt):
    rng = np.random.default_rng(21)
    max_seq, nkvh, d = 32768, 2, 128
    cq = dev(np.full((max_seq, nkvh, d), 7, np.int8))
    cs = dev(np.full((max_seq, nkvh), -1.0, np.float32))
    host_q = np.full((max_seq, nkvh, d), 7, np.int8)
    host_s = np.full((max_seq, nkvh), -1.0, np.float32)
    for pos, ntok in ((0, 2048), (2048, 1), (5000, 27768), (32767, 1)):
        kv = with_outliers(rng, (ntok, nkvh, d), dt, 1.0)
        L.Ops.kv_append_int8(cq, cs, dev(kv, DTS[dt]), pos)
        assert oracle.kv_append_int8(host_q, host_s, kv, pos) == 0
    assert_exact(cq.numpy(), host_q)
    assert_exact(cs.numpy(), host_s)
    # dequantized read of the whole cache
    out = empty((max_seq, nkvh, d), DTS[dt])
    L.Ops.dequantize_int8(out, cq, cs)
    assert_exact(out.numpy(), oracle.dequantize_int8(host_q, host_s, np.uint16 if dt == "bf16" else np.float32))


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("pos, ntok", [(0, 2048), (5000, 1), (31000, 1768)])
def test_kv_append_pair_equals_two_appends(dt, pos, ntok):
    """llaisysKVAppendInt8Pair: one launch for k and v, bit-identical to two
    llaisysKVAppendInt8 calls and to the oracle, rows outside pos .. pos+ntok untouched;
    then llaisysDequantizeInt8Pair of both caches against two single dequantizations."""
    rng = np.random.default_rng(pos + ntok)
    max_seq, nkvh, d = 32768, 2, 128
    k = with_outliers(rng, (ntok, nkvh, d), dt, 1.0)
    v = with_outliers(rng, (ntok, nkvh, d), dt, 1.0)
    k[0, 1] = 0  # an all-zero (token, head) row
    fill_q, fill_s = np.full((max_seq, nkvh, d), 7, np.int8), np.full((max_seq, nkvh), -1.0, np.float32)
    kc, ks, vc, vs = dev(fill_q), dev(fill_s), dev(fill_q), dev(fill_s)
    L.Ops.kv_append_int8_pair(kc, ks, vc, vs, dev(k, DTS[dt]), dev(v, DTS[dt]), pos)
    hk_q, hk_s, hv_q, hv_s = fill_q.copy(), fill_s.copy(), fill_q.copy(), fill_s.copy()
    assert oracle.kv_append_int8(hk_q, hk_s, k, pos) == 0
    assert oracle.kv_append_int8(hv_q, hv_s, v, pos) == 0
    assert_exact(kc.numpy(), hk_q, "k codes")
    assert_exact(ks.numpy(), hk_s, "k scales")
    assert_exact(vc.numpy(), hv_q, "v codes")
    assert_exact(vs.numpy(), hv_s, "v scales")
    # the single-tensor entry point writes the same bytes
    kc1, ks1 = dev(fill_q), dev(fill_s)
    L.Ops.kv_append_int8(kc1, ks1, dev(k, DTS[dt]), pos)
    assert_exact(kc1.numpy(), kc.numpy(), "pair vs single codes")
    assert_exact(ks1.numpy(), ks.numpy(), "pair vs single scales")
    # paired dequantized read of the appended rows of both caches
    sl = lambda t: t.slice(0, pos, pos + ntok)
    ko, vo = empty((ntok, nkvh, d), DTS[dt]), empty((ntok, nkvh, d), DTS[dt])
    L.Ops.dequantize_int8_pair(ko, sl(kc), sl(ks), vo, sl(vc), sl(vs))
    et = np.uint16 if dt == "bf16" else (np.float16 if dt == "f16" else np.float32)
    assert_exact(ko.numpy(), oracle.dequantize_int8(hk_q[pos:pos + ntok], hk_s[pos:pos + ntok], et), "k read")
    assert_exact(vo.numpy(), oracle.dequantize_int8(hv_q[pos:pos + ntok], hv_s[pos:pos + ntok], et), "v read")


def test_quant_pairs_unaligned_and_empty():
    """Pair entry points on shapes the vector kernels do not take (odd rows, an odd byte
    offset) and with an empty second job."""
    rng = np.random.default_rng(5)
    a = with_outliers(rng, (9, 3, 7), "bf16", 1.0)
    b = with_outliers(rng, (9, 3, 7), "bf16", 1.0)
    qa, sa = empty((20, 3, 7), L.DataType.I8), empty((20, 3), L.DataType.F32)
    qb, sb = empty((20, 3, 7), L.DataType.I8), empty((20, 3), L.DataType.F32)
    L.Ops.kv_append_int8_pair(qa, sa, qb, sb, dev(a, L.DataType.BF16), dev(b, L.DataType.BF16), 3)
    for q, s, x in ((qa, sa, a), (qb, sb, b)):
        eq, es = oracle.quantize_int8(x.reshape(-1, 7))
        assert_exact(q.numpy()[3:12].reshape(-1, 7), eq)
        assert_exact(s.numpy()[3:12].reshape(-1), es)
    # empty second job, and outputs that start at an odd element
    oa, ob = empty((9, 3, 7), L.DataType.BF16), empty((0, 3, 7), L.DataType.BF16)
    qz, sz = empty((0, 3, 7), L.DataType.I8), empty((0, 3), L.DataType.F32)
    L.Ops.dequantize_int8_pair(oa, qa.slice(0, 3, 12), sa.slice(0, 3, 12), ob, qz, sz)
    eq, es = oracle.quantize_int8(a.reshape(-1, 7))
    assert_exact(oa.numpy().reshape(-1, 7), oracle.dequantize_int8(eq, es, np.uint16))


# ---- config-size properties ----------------------------------------------------------------

def test_config2_shapes_properties():
    """Llama-8B shapes (config 2) checked through size-independent properties."""
    rng = np.random.default_rng(2)
    BF = L.DataType.BF16
    # rms_norm [16384, 4096]: every row of the output has rms ~= rms(w) and matches
    # the oracle on a sample of rows
    x = sample(rng, (16384, 4096), "bf16")
    w = sample(rng, (4096,), "bf16", 0.1, 1.0)
    y = empty(x.shape, BF)
    L.Ops.rms_norm(y, dev(x, BF), dev(w, BF), 1e-5)
    got = y.numpy()
    rows = rng.choice(16384, 64, replace=False)
    assert_close(got[rows], oracle.rms_norm(x[rows], w, 1e-5))
    # rope q[16384, 32, 128], theta 5e5: norm of every pair preserved; position 0 identity
    q = sample(rng, (16384, 32, 128), "bf16")
    pos = np.arange(16384, dtype=np.int64)
    yq = empty(q.shape, BF)
    L.Ops.rope(yq, dev(q, BF), dev(pos), 5e5)
    gq = yq.numpy()
    assert np.array_equal(gq[0], q[0])
    qa, qb = bf16_to_f32(q[..., :64]), bf16_to_f32(q[..., 64:])
    ya, yb = bf16_to_f32(gq[..., :64]), bf16_to_f32(gq[..., 64:])
    n0, n1 = qa ** 2 + qb ** 2, ya ** 2 + yb ** 2
    assert np.allclose(n0, n1, rtol=2e-2, atol=1e-3)
    assert_close(gq[-4:], oracle.rope(q[-4:], pos[-4:], 5e5))
    no_device_error()


def test_config2_swiglu_full():
    """swiglu [16384, 14336] bf16 (config 2), every element against the oracle
    (reference src/ops/swiglu/cpu/swiglu_cpu.cpp:15-20)."""
    rng = np.random.default_rng(21)
    BF = L.DataType.BF16
    g, u = sample(rng, (16384, 14336), "bf16"), sample(rng, (16384, 14336), "bf16")
    y = empty(g.shape, BF)
    L.Ops.swiglu(y, dev(g, BF), dev(u, BF))
    got = y.numpy()
    for r0 in range(0, 16384, 4096):  # chunks bound the oracle's host memory
        assert_close(got[r0:r0 + 4096], oracle.swiglu(g[r0:r0 + 4096], u[r0:r0 + 4096]), f"rows {r0}+")
    no_device_error()


def test_config2_embedding_full():
    """Embedding from a [128256, 4096] bf16 table with 16384 int64 ids (config 2):
    bit-exact against table[ids] (a gather is its own oracle,
    src/ops/embedding/cpu/embedding_cpu.cpp:16-22), first and last rows included."""
    rng = np.random.default_rng(22)
    BF = L.DataType.BF16
    table = sample(rng, (128256, 4096), "bf16", 0.02)
    ids = rng.integers(0, 128256, size=16384).astype(np.int64)
    ids[:2] = (0, 128255)
    out = empty((16384, 4096), BF)
    L.Ops.embedding(out, dev(ids), dev(table, BF))
    assert_exact(out.numpy(), table[ids])
    no_device_error()


def test_config2_rope_qk_full():
    """RoPE q [16384, 32, 128] and k [16384, 8, 128] bf16, theta 5e5, positions
    0..16383 (config 2) through the fused q/k launch and the reference-ABI single-tensor
    launch: every element against the oracle (src/ops/rope/cpu/rope_cpu.cpp:28-44)."""
    rng = np.random.default_rng(23)
    BF = L.DataType.BF16
    q, k = sample(rng, (16384, 32, 128), "bf16"), sample(rng, (16384, 8, 128), "bf16")
    pos = np.arange(16384, dtype=np.int64)
    tq, tk, tp = dev(q, BF), dev(k, BF), dev(pos)
    qo, ko = empty(q.shape, BF), empty(k.shape, BF)
    L.Ops.rope_qk(qo, tq, ko, tk, tp, 5e5)
    eq, ek = oracle.rope(q, pos, 5e5), oracle.rope(k, pos, 5e5)
    assert_close(qo.numpy(), eq, "q (fused q/k)")
    assert_close(ko.numpy(), ek, "k (fused q/k)")
    ko2 = empty(k.shape, BF)
    L.Ops.rope(ko2, tk, tp, 5e5)
    assert_close(ko2.numpy(), ek, "k (llaisysROPE)")
    no_device_error()


# ---- fused q/k RoPE ------------------------------------------------------------------------

@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("seq,nhq,nhk,d,p0,theta", [
    (8192, 12, 2, 128, 0, 1e4),       # config 1
    (2048, 12, 2, 128, 0, 1e6),       # config 4 (Qwen2 theta)
    (300, 32, 8, 128, 16000, 5e5),    # config 2 heads
    (5, 3, 1, 6, 2, 1e4),             # odd half-dim: scalar kernels
    (17, 64, 64, 128, 7, 1e4),        # more items per token than the register plan holds
    (8195, 12, 2, 128, 5, 1e4),       # four tokens per wave, the last wave's group ragged
])
def test_rope_qk_equals_two_ropes(dt, seq, nhq, nhk, d, p0, theta):
    rng = np.random.default_rng(seed_of(seq, nhq, dt))
    q, k = sample(rng, (seq, nhq, d), dt), sample(rng, (seq, nhk, d), dt)
    pos = np.arange(p0, p0 + seq, dtype=np.int64)
    qo, ko = empty(q.shape, DTS[dt]), empty(k.shape, DTS[dt])
    L.Ops.rope_qk(qo, dev(q, DTS[dt]), ko, dev(k, DTS[dt]), dev(pos), theta)
    assert_close(qo.numpy(), oracle.rope(q, pos, theta), "q")
    assert_close(ko.numpy(), oracle.rope(k, pos, theta), "k")


# ---- HIP graph capture ---------------------------------------------------------------------

def test_graph_replays_match_eager():
    """A captured layer (fused norm, RoPE q/k, INT8 KV append, swiglu, argmax) replayed
    three times, with eager work and synchronisation between replays; every replay must
    reproduce the eager results (the outputs are cleared before each replay)."""
    rng = np.random.default_rng(31)
    BF, I8, F32, I64 = L.DataType.BF16, L.DataType.I8, L.DataType.F32, L.DataType.I64
    t = 256
    x, r = sample(rng, (t, 1536), "bf16"), sample(rng, (t, 1536), "bf16")
    w = sample(rng, (1536,), "bf16", 0.1, 1.0)
    q, k = sample(rng, (t, 12, 128), "bf16"), sample(rng, (t, 2, 128), "bf16")
    g, u = sample(rng, (t, 8960), "bf16"), sample(rng, (t, 8960), "bf16")
    logits = sample(rng, (4, 151936), "bf16")
    pos = np.arange(t, dtype=np.int64)
    tx, tr, tw, tq, tk, tg, tu, tl, tp = (dev(a, BF if a.dtype == np.uint16 else None)
                                          for a in (x, r, w, q, k, g, u, logits, pos))
    outs = {"y": empty((t, 1536), BF), "h": empty((t, 1536), BF), "qo": empty(q.shape, BF),
            "ko": empty(k.shape, BF), "kc": empty((t, 2, 128), I8), "ks": empty((t, 2), F32),
            "act": empty((t, 8960), BF), "ri": empty((4,), I64), "rv": empty((4,), BF),
            "fi": empty((1,), I64), "fv": empty((1,), BF)}

    def layer():
        o = outs
        L.Ops.add_rms_norm(o["y"], o["h"], tx, tr, tw, 1e-6)
        L.Ops.rope_qk(o["qo"], tq, o["ko"], tk, tp, 1e6)
        L.Ops.kv_append_int8(o["kc"], o["ks"], o["ko"], 0)
        L.Ops.swiglu(o["act"], tg, tu)
        L.Ops.argmax_rows(o["ri"], o["rv"], tl)
        L.Ops.argmax(o["fi"], o["fv"], tl)

    layer()
    eager = {name: tt.numpy() for name, tt in outs.items()}
    graph = L.Graph.capture()
    layer()
    graph.end()
    api = L.RuntimeAPI(L.DeviceType.AMD)
    for replay in range(3):
        for tt in outs.values():  # clear every output with an eager copy
            z = np.zeros(tt.shape(), dtype=tt.numpy().dtype)
            api.memcpy_sync(tt.data_ptr(), z.ctypes.data, z.nbytes, L.MemcpyKind.H2D)
        scratch = empty((t, 8960), BF)
        L.Ops.swiglu(scratch, tu, tg)  # unrelated eager work between replays
        api.device_synchronize()
        graph.launch()
        api.device_synchronize()
        for name, tt in outs.items():
            assert_exact(tt.numpy(), eager[name], f"replay {replay}: {name}")
    no_device_error()


def test_graph_replays_sampling_and_int8_prefill():
    """Random sampling (histogram state left zero by each launch, top_k 50 and 1024) and a
    bf16 prefill over an INT8 cache (the caches dequantized into the workspace, then the bf16
    kernel) captured in one graph: three replays with eager work between them must equal
    the eager results."""
    BF, I64 = L.DataType.BF16, L.DataType.I64
    rng = np.random.default_rng(41)
    logits = dev(sample(rng, (2, 151936), "bf16"), BF)
    kv = f32_to_bf16(rng.standard_normal((2, 300, 2, 128)).astype(np.float32))
    kq, ks = oracle.quantize_int8(kv[0])
    vq, vs = oracle.quantize_int8(kv[1])
    tq = dev(sample(rng, (64, 12, 128), "bf16"), BF)
    tkq, tks, tvq, tvs = dev(kq), dev(ks), dev(vq), dev(vs)
    s50, s1k, att = empty((2,), I64), empty((2,), I64), empty((64, 12, 128), BF)

    def ops():
        L.Ops.random_sample(s50, logits, 0.8, 50, 0.8, 1234)
        L.Ops.random_sample(s1k, logits, 1.0, 1024, 0.95, 99)
        L.Ops.self_attention_int8kv(att, tq, tkq, tks, tvq, tvs, 0.0883883)

    ops()
    eager = [t.numpy() for t in (s50, s1k, att)]
    graph = L.Graph.capture()
    ops()
    graph.end()
    api = L.RuntimeAPI(L.DeviceType.AMD)
    for replay in range(3):
        # eager work between replays: other samples and a decode attention
        L.Ops.random_sample(empty((2,), I64), logits, 0.7, 40, 1.0, replay)
        L.Ops.self_attention_int8kv(empty((1, 12, 128), BF), dev(sample(rng, (1, 12, 128), "bf16"), BF),
                                    tkq, tks, tvq, tvs, 0.0883883)
        api.device_synchronize()
        for t in (s50, s1k, att):
            z = np.zeros(t.shape(), dtype=t.numpy().dtype)
            api.memcpy_sync(t.data_ptr(), z.ctypes.data, z.nbytes, L.MemcpyKind.H2D)
        graph.launch()
        api.device_synchronize()
        for name, t, e in zip(("top_k 50", "top_k 1024", "int8 prefill"), (s50, s1k, att), eager):
            assert_exact(t.numpy(), e, f"replay {replay}: {name}")
    del graph
    no_device_error()


def test_graph_keeps_its_workspace_after_growth(monkeypatch):
    """A graph whose kernels use the library scratch (the flat argmax's counter, the
    decode attention's partials) stays valid after a later eager op grows the scratch:
    captured in a fresh thread (its own stream and scratch) with no capture reservation,
    then a long decode attention run eagerly needs more scratch than the graph captured,
    and three replays must still equal the eager results."""
    import threading
    monkeypatch.setenv("LLAISYS_GRAPH_WORKSPACE_BYTES", "0")
    BF, I64 = L.DataType.BF16, L.DataType.I64
    rng = np.random.default_rng(37)
    logits = sample(rng, (1, 151936), "bf16")
    q1, k1, v1 = (sample(rng, s, "bf16") for s in ((1, 12, 128), (64, 2, 128), (64, 2, 128)))
    qb, kb, vb = (sample(rng, s, "bf16") for s in ((4, 12, 128), (32768, 2, 128), (32768, 2, 128)))
    errors = []

    def body():
        try:
            tl = dev(logits, BF)
            tq, tk, tv = dev(q1, BF), dev(k1, BF), dev(v1, BF)
            fi, fv, ao = empty((1,), I64), empty((1,), BF), empty((1, 12, 128), BF)

            def ops():
                L.Ops.argmax(fi, fv, tl)
                L.Ops.self_attention(ao, tq, tk, tv, 0.0883883)

            ops()
            eager = [t.numpy() for t in (fi, fv, ao)]
            graph = L.Graph.capture()
            ops()
            graph.end()
            # 4 queries x 12 heads over 32768 keys: partials beyond the captured scratch
            big = empty((4, 12, 128), BF)
            L.Ops.self_attention(big, dev(qb, BF), dev(kb, BF), dev(vb, BF), 0.0883883)
            api = L.RuntimeAPI(L.DeviceType.AMD)
            api.device_synchronize()
            for replay in range(3):
                for t in (fi, fv, ao):
                    z = np.zeros(t.shape(), dtype=t.numpy().dtype)
                    api.memcpy_sync(t.data_ptr(), z.ctypes.data, z.nbytes, L.MemcpyKind.H2D)
                graph.launch()
                api.device_synchronize()
                for name, t, e in zip(("idx", "val", "attn"), (fi, fv, ao), eager):
                    assert_exact(t.numpy(), e, f"replay {replay}: {name}")
            del graph
            assert L.take_device_error() == 0
        except BaseException as e:  # re-raised in the test thread
            errors.append(e)

    th = threading.Thread(target=body)
    th.start()
    th.join()
    if errors:
        raise errors[0]


# ---- fused RoPE + INT8 KV append ---------------------------------------------------------

@pytest.mark.parametrize("dt", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("seq,nq,nk,d,pos0,max_seq,theta", [
    (2048, 12, 2, 128, 0, 2048, 1e6),     # config 4 layer
    (8192, 12, 2, 128, 0, 8192, 1e4),     # config 1 shape
    (300, 32, 8, 128, 100, 1024, 5e5),    # Llama-8B heads, append at an offset
    (1, 12, 2, 128, 4095, 4096, 1e6),     # one decode token at the cache end
    (7, 3, 1, 6, 2, 16, 1e4),             # odd half-dim: composed fallback
    (9, 64, 64, 128, 0, 9, 1e4),          # more rows per token than the fused plan holds
])
def test_rope_kv_append_equals_composition(dt, seq, nq, nk, d, pos0, max_seq, theta):
    """The fused op equals llaisysROPEQK followed by two llaisysKVAppendInt8, bit for bit,
    and that composition matches the oracle (rope within tolerance, codes exact on the
    GPU's own rope'd k)."""
    rng = np.random.default_rng(seed_of(seq, nq, dt))
    T = DTS[dt]
    q, k, v = sample(rng, (seq, nq, d), dt), sample(rng, (seq, nk, d), dt), sample(rng, (seq, nk, d), dt)
    pos = np.arange(pos0, pos0 + seq, dtype=np.int64)
    tq, tk, tv, tp = dev(q, T), dev(k, T), dev(v, T), dev(pos)

    def caches():
        return (dev(np.full((max_seq, nk, d), 5, np.int8)), dev(np.full((max_seq, nk), -2.0, np.float32)),
                dev(np.full((max_seq, nk, d), 5, np.int8)), dev(np.full((max_seq, nk), -2.0, np.float32)))

    kc, ks, vc, vs = caches()
    qo = empty(q.shape, T)
    L.Ops.rope_kv_append_int8(qo, tq, tk, tv, tp, theta, kc, ks, vc, vs, pos0)
    # composition through the separate entry points
    kc2, ks2, vc2, vs2 = caches()
    qo2, ko2 = empty(q.shape, T), empty(k.shape, T)
    L.Ops.rope_qk(qo2, tq, ko2, tk, tp, theta)
    L.Ops.kv_append_int8(kc2, ks2, ko2, pos0)
    L.Ops.kv_append_int8(vc2, vs2, tv, pos0)
    for a, b, what in ((qo, qo2, "q"), (kc, kc2, "k codes"), (ks, ks2, "k scales"),
                       (vc, vc2, "v codes"), (vs, vs2, "v scales")):
        assert_exact(a.numpy(), b.numpy(), what)
    # and against the oracle: rope within tolerance, codes of the GPU's rope'd k exact
    assert_close(qo.numpy(), oracle.rope(q, pos, theta), "q vs oracle")
    hq, hs = np.full((max_seq, nk, d), 5, np.int8), np.full((max_seq, nk), -2.0, np.float32)
    assert oracle.kv_append_int8(hq, hs, ko2.numpy(), pos0) == 0
    assert_exact(kc.numpy(), hq, "k codes vs oracle")
    assert_exact(ks.numpy(), hs, "k scales vs oracle")
    hq, hs = np.full((max_seq, nk, d), 5, np.int8), np.full((max_seq, nk), -2.0, np.float32)
    assert oracle.kv_append_int8(hq, hs, v, pos0) == 0
    assert_exact(vc.numpy(), hq, "v codes vs oracle")
    # the composed fallback must leave the flat argmax's scratch counter intact
    logits = sample(rng, (151936,), "bf16")
    i, m = empty((1,), L.DataType.I64), empty((1,), L.DataType.BF16)
    L.Ops.argmax(i, m, dev(logits, L.DataType.BF16))
    assert i.numpy()[0] == oracle.argmax(logits)[0]
    no_device_error()


# ---- INT8 boundary rows (division-free quotient, packed absmax) ----------------------------

def quant_edge_rows(dt, cols=256, seed=5):
    """Rows that reach every branch of the quantizer: zero, NaN (quiet, signalling, with
    low payload bits), +-inf, scales below / around the 2^-96 exact-division threshold,
    subnormals, exact half-integer ties on a power-of-two scale, signed zeros, the largest
    finite value, and random +-1 ulp near-ties."""
    rng = np.random.default_rng(seed)
    f32 = lambda u: np.array(u, np.uint32).view(np.float32)
    rows = []
    base = rng.standard_normal(cols).astype(np.float32)
    rows.append(np.zeros(cols, np.float32))
    r = base.copy(); r[[3, 100]] = np.nan; rows.append(r)
    r = base.copy(); r[5] = np.inf; rows.append(r)
    r = base.copy(); r[7] = -np.inf; r[9] = np.nan; rows.append(r)
    rows.append(base * np.float32(1e-30))                        # scale < 2^-96: IEEE path
    thr = np.float32(127.0) * np.float32(2.0 ** -96)
    for k in (-2, -1, 0, 1, 2):                                  # amax around the threshold
        r = base / np.abs(base).max() * thr
        r[0] = np.nextafter(thr, np.float32(np.inf if k > 0 else 0), dtype=np.float32) if k else thr
        if abs(k) == 2:
            r[0] = np.nextafter(r[0], np.float32(np.inf if k > 0 else 0), dtype=np.float32)
        rows.append(r.astype(np.float32))
    rows.append(base * np.float32(1e-39))                        # f32 subnormals
    s = np.float32(2.0 ** -3)
    ties = (np.arange(cols) % 254 - 127 + 0.5).astype(np.float32) * s
    ties[0] = 127 * s; rows.append(np.clip(ties, -127 * s, 127 * s))
    r = base.copy(); r[::2] = 0.0; r[1::4] = -0.0; rows.append(r)
    r = base.copy(); r[11] = np.finfo(np.float32).max; rows.append(r)
    amax = np.float32(3.0); sc = amax / np.float32(127.0)
    k = rng.integers(-126, 126, cols).astype(np.float32)
    near = ((k + np.float32(0.5)) * sc).astype(np.float32)
    near = np.where(rng.random(cols) < 0.5, np.nextafter(near, np.float32(0)), np.nextafter(near, np.float32(9)))
    near[0] = amax; rows.append(near.astype(np.float32))
    x = np.stack(rows).astype(np.float32)
    if dt == "f32":
        x[1, 50] = f32(0x7FC01234)   # quiet NaN with low payload bits
        x[1, 51] = f32(0xFF812345)   # signalling NaN, negative
        return x
    if dt == "bf16":
        b = f32_to_bf16(x)
        b[1, 50], b[1, 51], b[3, 52] = 0x7F81, 0xFFC1, 0x7F80  # sNaN, -qNaN, +inf
        b[-4, 11] = 0x7F7F                                     # largest finite bf16
        return b
    with np.errstate(over="ignore"):
        h = x.astype(np.float16)
    hv = h.view(np.uint16)
    hv[1, 50], hv[1, 51] = 0x7C01, 0xFE00                       # sNaN, -qNaN
    hv[-4, 11] = 0x7BFF                                         # largest finite f16
    return h


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
# one-wavefront lane groups (128, 200), lane-group plan, one wave per row (full / partial);
# rows of exactly 192 16-byte vectors (bf16 / f16 1536, f32 768) take the exact-fit form
@pytest.mark.parametrize("cols", [128, 200, 256, 768, 1536, 1000, 8960])
def test_quantize_boundary_rows(dt, cols):
    x = quant_edge_rows(dt, cols=cols)
    q, s = empty(x.shape, L.DataType.I8), empty(x.shape[:-1], L.DataType.F32)
    L.Ops.quantize_int8(q, s, dev(x, DTS[dt]))
    eq, es = oracle.quantize_int8(x)
    assert_exact(q.numpy(), eq, "codes")
    assert_exact(s.numpy(), es, "scales")
    # KV append (same kernel, pointed into a cache) and the dequantized read
    rows, cols = x.shape
    kv = x.reshape(rows, 1, cols)
    cq, cs = dev(np.zeros((rows + 3, 1, cols), np.int8)), dev(np.zeros((rows + 3, 1), np.float32))
    L.Ops.kv_append_int8(cq, cs, dev(kv, DTS[dt]), 2)
    assert_exact(cq.numpy()[2:2 + rows, 0], eq, "kv codes")
    assert_exact(cs.numpy()[2:2 + rows, 0], es, "kv scales")
    out = empty(x.shape, DTS[dt])
    L.Ops.dequantize_int8(out, q, s)
    assert_exact(out.numpy(), oracle.dequantize_int8(eq, es, x.dtype), "dequant")
    no_device_error()


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_dequantize_caller_scales_with_nan_payloads(dt):
    """Scales are caller data: NaN scales with payload bits (and infinities) must round
    like the reference's rule, which the hardware bf16 converter alone would not."""
    rng = np.random.default_rng(8)
    rows, cols = 64, 512
    q = rng.integers(-127, 128, (rows, cols)).astype(np.int8)
    s = (rng.random(rows).astype(np.float32) + np.float32(0.5)) * np.float32(0.01)
    bits = s.view(np.uint32)
    bits[3], bits[10], bits[11] = 0x7FC01234, 0xFF800001, 0x7F800000
    bits[12] = 0x7FFFFFFF
    out = empty((rows, cols), DTS[dt])
    L.Ops.dequantize_int8(out, dev(q), dev(s))
    assert_exact(out.numpy(), oracle.dequantize_int8(q, s, np.uint16 if dt == "bf16" else np.float16))


def test_rms_norm_nan_eps_matches_oracle_nan_pattern():
    rng = np.random.default_rng(9)
    x, w = sample(rng, (16, 1536), "bf16"), sample(rng, (1536,), "bf16", 0.1, 1.0)
    out = empty(x.shape, L.DataType.BF16)
    L.Ops.rms_norm(out, dev(x, L.DataType.BF16), dev(w, L.DataType.BF16), float("nan"))
    got = bf16_to_f32(out.numpy())
    ref = bf16_to_f32(oracle.rms_norm(x, w, float("nan")))
    assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.isnan(ref).all()


def test_rope_kv_append_far_positions():
    """The fused RoPE + INT8 KV append with positions up to 2^40 (the device library's sincos
    beside the reduced-argument routine) equals llaisysROPEQK followed by the pair append."""
    rng = np.random.default_rng(31)
    seq, nq, nk, d = 2048, 12, 2, 128
    q, k, v = (sample(rng, (seq, h, d), "bf16") for h in (nq, nk, nk))
    pos = rng.integers(0, 2 ** 40, size=seq).astype(np.int64)
    pos[::3] = np.arange(len(pos[::3]))
    T = L.DataType.BF16
    tq, tk, tv, tp = dev(q, T), dev(k, T), dev(v, T), dev(pos)
    def caches():
        return (dev(np.zeros((seq, nk, d), np.int8)), dev(np.zeros((seq, nk), np.float32)),
                dev(np.zeros((seq, nk, d), np.int8)), dev(np.zeros((seq, nk), np.float32)))
    kc, ks, vc, vs = caches()
    qo = empty(q.shape, T)
    L.Ops.rope_kv_append_int8(qo, tq, tk, tv, tp, 1e6, kc, ks, vc, vs, 0)
    kc2, ks2, vc2, vs2 = caches()
    qo2, ko2 = empty(q.shape, T), empty(k.shape, T)
    L.Ops.rope_qk(qo2, tq, ko2, tk, tp, 1e6)
    L.Ops.kv_append_int8(kc2, ks2, ko2, 0)
    L.Ops.kv_append_int8(vc2, vs2, tv, 0)
    for a, b, what in ((qo, qo2, "q"), (kc, kc2, "k codes"), (ks, ks2, "k scales"),
                       (vc, vc2, "v codes"), (vs, vs2, "v scales")):
        assert_exact(a.numpy(), b.numpy(), what)
    assert_close(qo.numpy(), oracle.rope(q, pos, 1e6), "q vs the oracle")


@pytest.mark.parametrize("dt", ["bf16", "f32", "f16"])
def test_rope_kv_append_boundary_rows(dt):
    """NaN / inf / tiny / zero k and v rows through the fused op equal the composition and
    the oracle's codes."""
    rows = quant_edge_rows(dt, cols=128)
    seq = rows.shape[0]
    rng = np.random.default_rng(10)
    T = DTS[dt]
    q = sample(rng, (seq, 12, 128), dt)
    k = np.stack([rows, rows[::-1]], axis=1)          # [seq, 2, 128]
    v = np.stack([rows[::-1], rows], axis=1)
    pos = np.arange(seq, dtype=np.int64) * 977
    tq, tk, tv, tp = dev(q, T), dev(k, T), dev(v, T), dev(pos)
    caches = lambda: (dev(np.zeros((seq, 2, 128), np.int8)), dev(np.zeros((seq, 2), np.float32)),
                      dev(np.zeros((seq, 2, 128), np.int8)), dev(np.zeros((seq, 2), np.float32)))
    kc, ks, vc, vs = caches()
    qo = empty(q.shape, T)
    L.Ops.rope_kv_append_int8(qo, tq, tk, tv, tp, 1e4, kc, ks, vc, vs, 0)
    kc2, ks2, vc2, vs2 = caches()
    qo2, ko2 = empty(q.shape, T), empty(k.shape, T)
    L.Ops.rope_qk(qo2, tq, ko2, tk, tp, 1e4)
    L.Ops.kv_append_int8(kc2, ks2, ko2, 0)
    L.Ops.kv_append_int8(vc2, vs2, tv, 0)
    for a, b, what in ((qo, qo2, "q"), (kc, kc2, "k codes"), (ks, ks2, "k scales"),
                       (vc, vc2, "v codes"), (vs, vs2, "v scales")):
        assert_exact(a.numpy(), b.numpy(), what)
    eq, es = oracle.quantize_int8(v.reshape(seq * 2, 128))
    assert_exact(vc.numpy().reshape(seq * 2, 128), eq, "v codes vs oracle")
    assert_exact(vs.numpy().reshape(seq * 2), es, "v scales vs oracle")
    eq, es = oracle.quantize_int8(ko2.numpy().reshape(seq * 2, 128))
    assert_exact(kc.numpy().reshape(seq * 2, 128), eq, "k codes vs oracle")
    no_device_error()
