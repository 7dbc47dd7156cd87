"""llaisysSelfAttentionInt8KVNoAlloc (the attention over the INT8 KV cache that allocates
nothing: its split partials, or a prefill's dequantized caches, live in a fixed device
scratch) against
llaisysSelfAttentionInt8KV, the allocating entry point it mirrors: the same launches with the
same chunking, so equal bit for bit.  Two calls in a row share the scratch; the second is
smaller, so a stale partial of the first call would show.  Both outputs are also checked
against the oracle's attention over the dequantized cache."""
import numpy as np
import pytest

import llaisys_amd as L
import oracle
from llaisys_amd.hostfmt import f32_to_bf16
from numerics import assert_attention_close, assert_exact

pytestmark = pytest.mark.gpu

AMD = dict(device=L.DeviceType.AMD, device_id=0)
BF, I8, F32 = L.DataType.BF16, L.DataType.I8, L.DataType.F32


def dev(a, dt=None):
    return L.Tensor.from_numpy(a, dt, **AMD)


def cache(rng, total, nkvh, d):
    """INT8 k / v caches written by the library's own append, plus their dequantized values."""
    k = f32_to_bf16(rng.standard_normal((total, nkvh, d), dtype=np.float32))
    v = f32_to_bf16(rng.standard_normal((total, nkvh, d), dtype=np.float32))
    kc, ks = L.Tensor((total, nkvh, d), I8, **AMD), L.Tensor((total, nkvh), F32, **AMD)
    vc, vs = L.Tensor((total, nkvh, d), I8, **AMD), L.Tensor((total, nkvh), F32, **AMD)
    L.Ops.kv_append_int8_pair(kc, ks, vc, vs, dev(k, BF), dev(v, BF), 0)
    deq = []
    for c, s in ((kc, ks), (vc, vs)):
        deq.append(oracle.dequantize_int8(c.numpy().reshape(-1, d), s.numpy().reshape(-1), np.uint16)
                   .reshape(total, nkvh, d))
    return (kc, ks, vc, vs), deq


@pytest.mark.parametrize("first,second", [
    # (seq, total, nh, nkvh, d): Qwen2-1.5B decode over 32K keys, then a shorter cache;
    # a speculative 3-token step (36 query-heads), then one token over 700 keys
    ((1, 32768, 12, 2, 128), (1, 5000, 12, 2, 128)),
    ((3, 4096, 12, 2, 128), (1, 700, 12, 2, 128)),
    # bf16 prefills on the MFMA kernel: caches dequantized into the scratch (2048 tokens of
    # Qwen2-1.5B, 2 MB), then a cache whose bf16 form exceeds the 24 MB scratch (the kernel
    # converts the codes itself)
    ((2048, 2048, 12, 2, 128), (16, 52000, 2, 2, 128)),
])
def test_no_alloc_attention_equals_allocating_entry(first, second):
    rng = np.random.default_rng(41)
    scale = 1.0 / np.sqrt(128)
    for seq, total, nh, nkvh, d in (first, second):
        q = f32_to_bf16(rng.standard_normal((seq, nh, d), dtype=np.float32))
        (kc, ks, vc, vs), (kd, vd) = cache(rng, total, nkvh, d)
        tq = dev(q, BF)
        ref, out = L.Tensor((seq, nh, d), BF, **AMD), L.Tensor((seq, nh, d), BF, **AMD)
        L.Ops.self_attention_int8kv(ref, tq, kc, ks, vc, vs, scale)
        L.Ops.self_attention_int8kv_noalloc(out, tq, kc, ks, vc, vs, scale)
        assert_exact(out.numpy(), ref.numpy(), f"{(seq, total)} vs the allocating entry point")
        exp = oracle.self_attention(q, kd, vd, scale)
        assert_attention_close(out.numpy(), exp, vd, f"{(seq, total)} vs the oracle")
    assert L.take_device_error() == 0

