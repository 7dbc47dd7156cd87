"""Self-attention on the GPU (llaisysSelfAttention, llaisysSelfAttentionInt8KV) against the
oracle's restatement of the reference kernel (self_attention_cpu.cpp:13-115), which
tests/test_oracle.py pins to the compiled reference.  Tolerance: numerics.assert_attention_close.
The INT8 form must equal, bit for bit, dequantizing the caches and attending."""
import zlib

import numpy as np
import pytest

import llaisys_amd as L
import oracle
from llaisys_amd.hostfmt import f32_to_bf16
from numerics import assert_attention_close, assert_exact

pytestmark = pytest.mark.gpu

AMD = dict(device=L.DeviceType.AMD, device_id=0)
DTS = {"f32": L.DataType.F32, "bf16": L.DataType.BF16, "f16": L.DataType.F16}
NP = {"f32": np.float32, "bf16": np.uint16, "f16": np.float16}


def sample(rng, shape, dt):
    x = rng.standard_normal(shape, dtype=np.float32)
    return {"f32": x, "bf16": f32_to_bf16(x), "f16": x.astype(np.float16)}[dt]


def dev(a, dt=None):
    return L.Tensor.from_numpy(a, dt, **AMD)


def attend(q, k, v, scale, dt):
    out = L.Tensor(q.shape[:2] + (v.shape[2],), DTS[dt], **AMD)
    L.Ops.self_attention(out, dev(q, DTS[dt]), dev(k, DTS[dt]), dev(v, DTS[dt]), scale)
    return out.numpy()


SHAPES = [
    # seq, total, nh, nkvh, d  -- reference test shapes, Qwen2-1.5B decode (split keys) and
    # prefill, a prefix cache, seq > total (size_t wrap), head_dim 64, Llama GQA 4, group > 8
    (2, 2, 1, 1, 4), (5, 11, 4, 2, 8),
    (1, 37, 12, 2, 128), (1, 4097, 12, 2, 128),
    (256, 256, 12, 2, 128), (64, 300, 12, 2, 128),
    (3, 2, 2, 1, 128), (9, 40, 4, 2, 64),
    (1, 2048, 32, 8, 128), (5, 70, 16, 1, 128),
    # MFMA prefill path (bf16, >= 16 queries): ragged query count over a longer cache, GQA
    # groups of 8, 4 and 1, a single tile
    (200, 1000, 12, 2, 128), (33, 33, 16, 2, 128), (48, 48, 32, 8, 128), (17, 17, 4, 4, 128),
    (16, 16, 12, 2, 128),
    # more than 512 MFMA blocks: one wave per head (the key tiles of a block unsplit), with
    # groups of 6 and of 1
    (300, 300, 168, 28, 128), (600, 600, 16, 16, 128),
    # decode over 16K+ keys: 8-wave blocks of 256 keys each
    (2, 20000, 12, 2, 128),
]


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_self_attention_matches_oracle(dt, shape):
    seq, total, nh, nkvh, d = shape
    rng = np.random.default_rng(zlib.crc32(repr((dt, shape)).encode()))
    q, k, v = sample(rng, (seq, nh, d), dt), sample(rng, (total, nkvh, d), dt), sample(rng, (total, nkvh, d), dt)
    scale = 1.0 / np.sqrt(d)
    got = attend(q, k, v, scale, dt)
    assert_attention_close(got, oracle.self_attention(q, k, v, scale), v, f"{dt} {shape}")


def test_self_attention_golden_on_gpu(golden):
    n = 0
    for (op, dt, case), c in golden.items():
        if op == "self_attention":
            got = attend(c["q"], c["k"], c["v"], float(c["scale"]), dt)
            assert_attention_close(got, c["out"], c["v"], f"golden {dt} {case}")
            n += 1
    assert n == 18


@pytest.mark.parametrize("scale", [-0.2, 0.0, 3.0])
def test_self_attention_unusual_scales(scale):
    """Any scale the reference accepts (negative flips the softmax, 0 gives the mean of the
    visible values); prefill shape, so a positive one takes the MFMA kernel."""
    rng = np.random.default_rng(77)
    q, k, v = sample(rng, (40, 12, 128), "bf16"), sample(rng, (40, 2, 128), "bf16"), sample(rng, (40, 2, 128), "bf16")
    got = attend(q, k, v, scale, "bf16")
    assert_attention_close(got, oracle.self_attention(q, k, v, scale), v, f"scale {scale}")


def test_prefill_is_deterministic():
    """Repeated prefill launches, interleaved with other attention shapes (which reuse the
    library workspace), give bit-identical outputs."""
    rng = np.random.default_rng(8)
    q, k, v = sample(rng, (512, 12, 128), "bf16"), sample(rng, (512, 2, 128), "bf16"), sample(rng, (512, 2, 128), "bf16")
    tq, tk, tv = dev(q, L.DataType.BF16), dev(k, L.DataType.BF16), dev(v, L.DataType.BF16)
    outs = []
    for rep in range(4):
        out = L.Tensor((512, 12, 128), L.DataType.BF16, **AMD)
        L.Ops.self_attention(out, tq, tk, tv, 0.088)
        outs.append(out.numpy())
        attend(q[:64], k[:300], v[:300], 0.1, "bf16")  # another shape in between
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    assert_attention_close(outs[0], oracle.self_attention(q, k, v, 0.088), v, "prefill 512")


def test_self_attention_empty_cache_gives_zeros():
    q = f32_to_bf16(np.ones((2, 4, 128), np.float32))
    out = L.Tensor((2, 4, 128), L.DataType.BF16, **AMD)
    kz = L.Tensor((0, 2, 128), L.DataType.BF16, **AMD)
    L.Ops.self_attention(out, dev(q, L.DataType.BF16), kz, kz, 0.1)
    assert not out.numpy().any()


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("shape", [(1, 4097, 12, 2, 128), (128, 128, 12, 2, 128), (5, 11, 4, 2, 8), (7, 33, 4, 2, 64),
                                   # bf16 prefill over the INT8 cache on the MFMA kernel: a prefix
                                   # cache, GQA 4 with ragged tiles, unsplit (> 512 blocks)
                                   (200, 1000, 12, 2, 128), (48, 70, 32, 8, 128), (300, 300, 168, 28, 128),
                                   # a cache whose bf16 form exceeds the workspace of 16 x 2
                                   # query-heads: the INT8 MFMA kernel converts the codes itself
                                   (16, 20000, 2, 2, 128),
                                   # decode over 16K+ keys: 8-wave blocks
                                   (2, 20000, 12, 2, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_self_attention_int8kv(dt, shape):
    """INT8 cache (1% outliers x20, as config 3) against dequantize-then-attend on the GPU
    and against the oracle's composition.  A bf16 prefill (16+ queries, head_dim 128) over a
    cache whose bf16 form fits the workspace dequantizes the cache and runs the bf16 kernel,
    so it equals the composition bit for bit; the other forms convert codes in their own key
    tiling, within the attention tolerance."""
    seq, total, nh, nkvh, d = shape
    rng = np.random.default_rng(zlib.crc32(repr(("int8", dt, shape)).encode()))
    x = rng.standard_normal((2, total, nkvh, d), dtype=np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    kv = {"f32": x, "bf16": f32_to_bf16(x), "f16": x.astype(np.float16)}[dt]
    kq, ks = oracle.quantize_int8(kv[0])
    vq, vs = oracle.quantize_int8(kv[1])
    q = sample(rng, (seq, nh, d), dt)
    scale = 1.0 / np.sqrt(d)
    out = L.Tensor((seq, nh, d), DTS[dt], **AMD)
    tq = dev(q, DTS[dt])
    tkq, tks, tvq, tvs = dev(kq), dev(ks), dev(vq), dev(vs)
    L.Ops.self_attention_int8kv(out, tq, tkq, tks, tvq, tvs, scale)
    # the composition on the GPU: dequantize both caches, then attend
    kd, vd = L.Tensor((total, nkvh, d), DTS[dt], **AMD), L.Tensor((total, nkvh, d), DTS[dt], **AMD)
    L.Ops.dequantize_int8_pair(kd, tkq, tks, vd, tvq, tvs)
    ref = L.Tensor((seq, nh, d), DTS[dt], **AMD)
    L.Ops.self_attention(ref, tq, kd, vd, scale)
    vdq = oracle.dequantize_int8(vq, vs, NP[dt])
    assert_attention_close(out.numpy(), ref.numpy(), vdq, "int8 vs dequantize + attend")
    if dt == "bf16" and seq >= 16 and d == 128:
        assert_exact(out.numpy(), ref.numpy(), "int8 prefill vs dequantize + attend")
    exp = oracle.self_attention_int8kv(q, kq, ks, vq, vs, scale)
    assert_attention_close(out.numpy(), exp, vdq, f"int8 {dt} {shape}")


def test_split_decode_across_calls():
    """Split decode launches of different chunk counts, queries and GQA groups back to back:
    each call's partials (library scratch) must be merged into its own output only."""
    rng = np.random.default_rng(41)
    for total, nh, nkvh, seq in ((4097, 12, 2, 1), (300, 12, 2, 1), (9000, 32, 8, 2), (4097, 12, 2, 1),
                                 (2500, 16, 4, 3), (4097, 12, 2, 1)):
        q = sample(rng, (seq, nh, 128), "bf16")
        k, v = sample(rng, (total, nkvh, 128), "bf16"), sample(rng, (total, nkvh, 128), "bf16")
        scale = 1.0 / np.sqrt(128)
        got = attend(q, k, v, scale, "bf16")
        assert_attention_close(got, oracle.self_attention(q, k, v, scale), v, f"split decode {total} {nh}/{nkvh} x{seq}")


def test_split_decode_at_the_chunk_limit():
    """A group of 16 q heads over a cache long enough for the maximum of 1024 key chunks."""
    rng = np.random.default_rng(43)
    total = 1024 * 128 + 5
    q = sample(rng, (1, 16, 128), "bf16")
    k, v = sample(rng, (total, 1, 128), "bf16"), sample(rng, (total, 1, 128), "bf16")
    got = attend(q, k, v, 0.05, "bf16")
    assert_attention_close(got, oracle.self_attention(q, k, v, 0.05), v, "1024 chunks, group 16")
