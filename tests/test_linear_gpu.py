"""Linear layers on the GPU (llaisysLinear, llaisysLinearW8A16) against the oracle's
restatement of the reference kernel (linear_cpu.cpp:11-41) and of the W8A16 rule, which
tests/test_oracle.py pins to the compiled reference and to closed forms.  Tolerance:
numerics.assert_linear_close."""
import zlib

import numpy as np
import pytest

import llaisys_amd as L
import oracle
from llaisys_amd.hostfmt import f32_to_bf16
from numerics import assert_exact, assert_linear_close

pytestmark = pytest.mark.gpu

AMD = dict(device=L.DeviceType.AMD, device_id=0)
DTS = {"f32": L.DataType.F32, "bf16": L.DataType.BF16, "f16": L.DataType.F16}


def sample(rng, shape, dt, s=1.0):
    x = (s * rng.standard_normal(shape)).astype(np.float32)
    return {"f32": x, "bf16": f32_to_bf16(x), "f16": x.astype(np.float16)}[dt]


def dev(a, dt=None):
    return L.Tensor.from_numpy(a, dt, **AMD)


def linear(x, w, b, dt):
    out = L.Tensor((x.shape[0], w.shape[0]), DTS[dt], **AMD)
    L.Ops.linear(out, dev(x, DTS[dt]), dev(w, DTS[dt]), None if b is None else dev(b, DTS[dt]))
    return out.numpy()


def linear_w8a16(x, codes, scale, b, dt):
    out = L.Tensor((x.shape[0], codes.shape[0]), DTS[dt], **AMD)
    L.Ops.linear_w8a16(out, dev(x, DTS[dt]), dev(codes), dev(scale),
                       None if b is None else dev(b, DTS[dt]))
    return out.numpy()


def int8_weights(rng, out_f, in_f):
    codes = rng.integers(-127, 128, size=(out_f, in_f), dtype=np.int8)
    scale = (0.01 * (0.5 + rng.random(out_f))).astype(np.float32) / 127
    return codes, scale


SHAPES = [
    # rows, in_features, out_features -- reference test shape, decode rows of Qwen2-1.5B's
    # projections (q, kv, gate/up, down), a prefill block, ragged edges of the 128 x 128
    # block tile, in_features not a multiple of 8 (scalar path), one output
    (2, 4, 3), (1, 1536, 1536), (1, 1536, 256), (1, 1536, 8960), (1, 8960, 1536),
    (256, 1536, 1536), (129, 264, 200), (17, 40, 130), (3, 77, 9), (64, 1536, 1), (1, 8, 1),
    # few rows over few output tiles: K split across blocks (ragged last split, 16 rows)
    (16, 4096, 300), (2, 2056, 40),
    # one row with partly used chunk slots (1024 / 3000 inputs, odd channel counts) and a
    # row longer than 24 chunks per lane (16384 inputs, 16-bit weights: the streaming GEMV)
    (1, 1024, 33), (1, 3000, 77), (1, 16384, 3),
    # 192..255 tiles of 128 x 128: the 96 x 128 tile (full and ragged last channel tile)
    (2048, 64, 1536), (2048, 128, 1530),
    # 512+ tiles of 128 x 128: 4-wave blocks, two stages (ragged row and channel tiles)
    (1100, 64, 8200),
]


@pytest.mark.parametrize("bias", [True, False], ids=["bias", "nobias"])
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_linear_matches_oracle(shape, dt, bias):
    rows, in_f, out_f = shape
    rng = np.random.default_rng(zlib.crc32(repr((shape, dt, bias)).encode()))
    x, w = sample(rng, (rows, in_f), dt), sample(rng, (out_f, in_f), dt, 0.05)
    b = sample(rng, (out_f,), dt) if bias else None
    assert_linear_close(linear(x, w, b, dt), oracle.linear(x, w, b), x, w, f"{dt} {shape}")


def test_linear_golden_on_gpu(golden):
    n = 0
    for (op, dt, case), c in golden.items():
        if op == "linear":
            got = linear(c["x"], c["w"], c["bias"], dt)  # zero-element bias = no bias
            assert_linear_close(got, c["out"], c["x"], c["w"], f"golden {dt} {case}")
            n += 1
    assert n == 12


def test_linear_prefill_block_is_deterministic():
    rng = np.random.default_rng(3)
    x, w = sample(rng, (512, 1536, ), "bf16"), sample(rng, (2048, 1536), "bf16", 0.05)
    first = linear(x, w, None, "bf16")
    assert_exact(linear(x, w, None, "bf16"), first, "second run")


def test_linear_empty_rows():
    rng = np.random.default_rng(4)
    w = sample(rng, (16, 32), "bf16")
    assert linear(np.zeros((0, 32), np.uint16), w, None, "bf16").shape == (0, 16)


@pytest.mark.parametrize("bias", [True, False], ids=["bias", "nobias"])
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_linear_w8a16_matches_oracle(shape, dt, bias):
    rows, in_f, out_f = shape
    rng = np.random.default_rng(zlib.crc32(repr(("w8", shape, dt, bias)).encode()))
    x = sample(rng, (rows, in_f), dt)
    codes, scale = int8_weights(rng, out_f, in_f)
    b = sample(rng, (out_f,), dt) if bias else None
    assert_linear_close(linear_w8a16(x, codes, scale, b, dt), oracle.linear_w8a16(x, codes, scale, b),
                        x, codes, f"w8a16 {dt} {shape}", w_scale=scale)


@pytest.mark.parametrize("in_f, out_f", [(1536, 65541), (2048, 65600), (1024, 4100)])
def test_w8a16_one_row_over_many_channels(in_f, out_f):
    # INT8 rows of at most 2 chunks per lane over 65536+ channels take 4 channels per wave (the
    # lm_head form), with channels past the end clamped; 4100 channels read x from L1 / L2 in
    # one-channel waves.  Same per-channel sum either way, checked against the oracle.
    rng = np.random.default_rng(zlib.crc32(repr(("w8 rows", in_f, out_f)).encode()))
    x = sample(rng, (1, in_f), "bf16")
    codes, scale = int8_weights(rng, out_f, in_f)
    b = sample(rng, (out_f,), "bf16")
    assert_linear_close(linear_w8a16(x, codes, scale, b, "bf16"), oracle.linear_w8a16(x, codes, scale, b),
                        x, codes, f"w8a16 1 x {in_f} -> {out_f}", w_scale=scale)


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_w8a16_with_unit_scales_equals_dense_linear(dt):
    # codes are exact in bf16 / f16, and a scale of 1 multiplies exactly: the two entry
    # points must agree bit for bit on the same sums (in_features a multiple of 16, so both
    # take the MFMA path, which sums in the same order)
    rng = np.random.default_rng(6)
    x = sample(rng, (100, 528), dt, 0.1)
    codes = rng.integers(-127, 128, size=(300, 528), dtype=np.int8)
    w = {"bf16": f32_to_bf16(codes.astype(np.float32)), "f16": codes.astype(np.float16)}[dt]
    b = sample(rng, (300,), dt)
    got = linear_w8a16(x, codes, np.ones(300, np.float32), b, dt)
    assert_exact(got, linear(x, w, b, dt), dt)


def test_w8a16_of_quantized_weights_tracks_dense_linear():
    # weights quantized by the library's own llaisysQuantizeInt8 (one scale per output row)
    rng = np.random.default_rng(7)
    x, w = sample(rng, (32, 1536), "bf16"), sample(rng, (256, 1536), "bf16", 0.02)
    q, s = L.Tensor((256, 1536), L.DataType.I8, **AMD), L.Tensor((256,), L.DataType.F32, **AMD)
    L.Ops.quantize_int8(q, s, dev(w, L.DataType.BF16))
    codes, scale = q.numpy(), s.numpy()
    got = linear_w8a16(x, codes, scale, None, "bf16")
    assert_linear_close(got, oracle.linear_w8a16(x, codes, scale), x, codes, "quantized", w_scale=scale)
    dense = linear(x, w, None, "bf16")
    gf = (got.astype(np.uint32) << 16).view(np.float32)
    df = (dense.astype(np.uint32) << 16).view(np.float32)
    assert np.abs(gf - df).max() < 0.02 * np.abs(df).max()


def test_split_k_linear_repeats_and_interleaves_with_argmax():
    # the split-K few-row path keeps per-tile arrival counters in the library scratch next to
    # the flat argmax's counter; both must return to zero, so repeated and interleaved calls
    # give identical results
    rng = np.random.default_rng(8)
    x, w = sample(rng, (1, 8960), "bf16"), sample(rng, (1536, 8960), "bf16", 0.02)
    tx, tw = dev(x, DTS["bf16"]), dev(w, DTS["bf16"])
    logits = dev(sample(rng, (1, 151936), "bf16"), DTS["bf16"])
    outs = []
    for _ in range(3):
        out = L.Tensor((1, 1536), DTS["bf16"], **AMD)
        L.Ops.linear(out, tx, tw)
        i, v = L.Tensor((1,), L.DataType.I64, **AMD), L.Tensor((1,), DTS["bf16"], **AMD)
        L.Ops.argmax(i, v, logits)
        outs.append(out.numpy())
    for o in outs[1:]:
        assert_exact(o, outs[0], "repeat")
    assert_linear_close(outs[0], oracle.linear(x, w), x, w, "split-K decode")
