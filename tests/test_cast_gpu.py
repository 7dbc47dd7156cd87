"""Device dtype conversion (llaisysCast) and the weight upload built on it
(llaisys_amd.weights) against the oracle's statement of the reference's cast<To>(From)
(oracle.cast, src/utils/types.hpp:116-139; pinned to the scalar rules in
tests/test_oracle.py).  Conversions are bit work: every output bit must match."""
import numpy as np
import pytest

import llaisys_amd as L
import oracle
from llaisys_amd import weights
from llaisys_amd.hostfmt import f32_to_bf16
from numerics import assert_exact

pytestmark = pytest.mark.gpu

AMD = dict(device=L.DeviceType.AMD, device_id=0)
CODE = {L.DataType.F32: oracle.F32, L.DataType.BF16: oracle.BF16, L.DataType.F16: oracle.F16}
NP = {L.DataType.F32: np.float32, L.DataType.BF16: np.uint16, L.DataType.F16: np.float16}


def values(rng, n):
    """Normal values over 16 decades plus the special cases of the rounding rules."""
    f = (rng.standard_normal(n) * 10.0 ** rng.integers(-8, 8, n)).astype(np.float32)
    raw = np.array([0x7FC00001, 0x7F800001, 0xFFC00000, 0x3F808000, 0x3F818000, 0x3F807FFF,
                    0x00000001, 0x80000000, 0x7F800000, 0x477FF000, 0x477FE000], np.uint32)
    k = min(n, raw.size)
    f[:k] = raw.view(np.float32)[:k]
    return f


def host(f, dt):
    return oracle.cast(f, CODE[dt])


@pytest.mark.parametrize("src", [L.DataType.F32, L.DataType.BF16, L.DataType.F16])
@pytest.mark.parametrize("dst", [L.DataType.F32, L.DataType.BF16, L.DataType.F16])
@pytest.mark.parametrize("shape", [(4096, 1536), (7, 13), (1,)])
def test_cast_matches_the_reference_rules(src, dst, shape):
    rng = np.random.default_rng(abs(hash((int(src), int(dst), shape))) % 2 ** 32)
    x = host(values(rng, int(np.prod(shape))).reshape(shape), src)
    out = L.Tensor(shape, dst, **AMD)
    L.Ops.cast(out, L.Tensor.from_numpy(x, src, **AMD))
    assert_exact(out.numpy(), oracle.cast(x, CODE[dst]), f"{src.name} -> {dst.name}")
    assert L.take_device_error() == 0


def test_cast_unaligned_slice_takes_the_scalar_kernel():
    rng = np.random.default_rng(3)
    x = values(rng, 1001)
    t = L.Tensor.from_numpy(x, L.DataType.F32, **AMD)
    part = t.slice(0, 3, 1000)            # 12-byte offset: not 16-byte aligned
    out = L.Tensor((997,), L.DataType.BF16, **AMD)
    L.Ops.cast(out, part)
    assert_exact(out.numpy(), f32_to_bf16(x[3:1000]))


def test_upload_keeps_weights_bf16_in_hbm():
    """The loader path: bf16 bits go up as they are; f32 / f16 host weights become the
    reference's bf16 of each value on the device; INT8 upload equals the oracle's
    quantization of the host weight."""
    rng = np.random.default_rng(9)
    w32 = (rng.standard_normal((1536, 1536)) * 0.02).astype(np.float32)
    wbf = f32_to_bf16(w32)
    t = weights.upload(wbf, L.DataType.BF16)
    assert t.dtype() == L.DataType.BF16 and t.device_type() == L.DeviceType.AMD
    assert_exact(t.numpy(), wbf)
    assert_exact(weights.upload(w32, L.DataType.BF16).numpy(), wbf)
    w16 = w32.astype(np.float16)
    assert_exact(weights.upload(w16, L.DataType.BF16).numpy(), oracle.cast(w16, oracle.BF16))
    assert_exact(weights.upload(wbf, L.DataType.F32).numpy(), oracle.cast(wbf, oracle.F32))
    codes, scales = weights.upload_int8(wbf)
    eq, es = oracle.quantize_int8(wbf)
    assert_exact(codes.numpy(), eq)
    assert_exact(scales.numpy(), es)
    assert L.take_device_error() == 0
