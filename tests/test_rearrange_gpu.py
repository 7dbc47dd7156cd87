"""Strided copy on the GPU (llaisysRearrange) and the tensor plumbing over it
(tensorContiguous, tensorReshape, tensorTo).

The reference's rearrange and Tensor::contiguous / reshape / to are stubs
(src/ops/rearrange/op.cpp:4-6, src/tensor/tensor.cpp:344-357); their meaning is an
element-by-element copy between layouts, so the expected result is numpy's copy of the same
strided view, bit for bit."""
import numpy as np
import pytest

import llaisys_amd as L
from llaisys_amd.hostfmt import f32_to_bf16
from numerics import assert_exact

pytestmark = pytest.mark.gpu

AMD = dict(device=L.DeviceType.AMD, device_id=0)
NP = {L.DataType.I8: np.int8, L.DataType.BF16: np.uint16, L.DataType.F32: np.float32,
      L.DataType.I64: np.int64}


def data(shape, dt, seed=0):
    rng = np.random.default_rng(seed)
    if dt == L.DataType.BF16:
        return f32_to_bf16(rng.standard_normal(shape).astype(np.float32))
    if dt in (L.DataType.I8, L.DataType.I64):
        return rng.integers(-100, 100, size=shape).astype(NP[dt])
    return rng.standard_normal(shape).astype(np.float32)


CASES = [
    # shape, permutation, dtype -- the kernel each reaches
    ((2048, 12, 128), (1, 0, 2), L.DataType.BF16),    # rows of 256 B (16-byte units)
    ((300, 517), (1, 0), L.DataType.F32),             # 2-D transpose, ragged tiles
    ((2, 3, 40, 33), (0, 2, 3, 1), L.DataType.BF16),  # transpose with outer dims on z
    ((5, 7, 9), (2, 1, 0), L.DataType.I8),            # 1-byte elements
    ((6, 4, 10), (1, 0, 2), L.DataType.I64),          # 8-byte elements, rows of 80 B
    ((1, 1, 64), (2, 0, 1), L.DataType.F32),          # size-1 dims collapse to a row copy
    ((8, 1, 3), (2, 1, 0), L.DataType.BF16),
    # 16-byte-vector transpose tiles: ragged edges of the 128 x 128 (2-byte), 64 x 64 (1-byte)
    # and 32 x 32 (4-byte) tiles, outer dims on z, and full multiples
    ((200, 72), (1, 0), L.DataType.BF16),
    ((3, 40, 136), (0, 2, 1), L.DataType.BF16),
    ((48, 80), (1, 0), L.DataType.I8),
    ((100, 36), (1, 0), L.DataType.F32),
    ((256, 512), (1, 0), L.DataType.BF16),
    ((1000, 264), (1, 0), L.DataType.BF16),           # 2-byte tiles ragged on both sides
    ((2, 3, 384, 136), (0, 1, 3, 2), L.DataType.BF16),  # two outer dims on z
    # vector-eligible in shape but one side's extent not a whole vector: element tiles
    ((200, 70), (1, 0), L.DataType.BF16),
]


@pytest.mark.parametrize("shape,perm,dt", CASES, ids=lambda v: str(v))
def test_rearrange_permuted_view_matches_numpy(shape, perm, dt):
    x = data(shape, dt)
    src = L.Tensor.from_numpy(x, dt, **AMD).permute(*perm)
    out = L.Tensor(src.shape(), dt, **AMD)
    L.Ops.rearrange(out, src)
    assert_exact(out.numpy(), np.ascontiguousarray(x.transpose(perm)), f"{shape} {perm}")


def test_rearrange_of_a_slice_and_into_a_strided_output():
    x = data((6, 8, 10), L.DataType.F32, 1)
    t = L.Tensor.from_numpy(x, L.DataType.F32, **AMD)
    s = t.slice(2, 1, 4)  # rows of 12 bytes (4-byte units)
    out = L.Tensor(s.shape(), L.DataType.F32, **AMD)
    L.Ops.rearrange(out, s)
    assert_exact(out.numpy(), np.ascontiguousarray(x[:, :, 1:4]), "slice")
    # into a permuted (non-contiguous) output: neither side's innermost dim matches
    base = L.Tensor((10, 6, 8), L.DataType.F32, **AMD)
    dst = base.permute(1, 2, 0)  # shape (6, 8, 10), strides (8, 1, 48)
    L.Ops.rearrange(dst, t)
    assert_exact(base.numpy(), np.ascontiguousarray(x.transpose(2, 0, 1)), "strided output")


def test_contiguous_reshape_to_on_the_gpu():
    x = data((4, 6, 32), L.DataType.BF16, 2)
    t = L.Tensor.from_numpy(x, L.DataType.BF16, **AMD)
    assert t.contiguous().data_ptr() == t.data_ptr()
    p = t.permute(2, 0, 1)
    c = p.contiguous()
    assert c.is_contiguous() and c.device_type() == L.DeviceType.AMD
    assert_exact(c.numpy(), np.ascontiguousarray(x.transpose(2, 0, 1)), "contiguous")
    r = p.reshape(32, 24)
    assert_exact(r.numpy(), np.ascontiguousarray(x.transpose(2, 0, 1).reshape(32, 24)), "reshape")
    h = p.to(L.DeviceType.CPU)  # non-contiguous device tensor to the host
    assert h.device_type() == L.DeviceType.CPU and h.is_contiguous()
    assert_exact(h.numpy(), np.ascontiguousarray(x.transpose(2, 0, 1)), "to cpu")
    back = L.Tensor.from_numpy(x, L.DataType.BF16, device=L.DeviceType.CPU).permute(1, 0, 2).to(L.DeviceType.AMD, 0)
    assert back.device_type() == L.DeviceType.AMD
    assert_exact(back.numpy(), np.ascontiguousarray(x.transpose(1, 0, 2)), "to amd")
    assert t.to(L.DeviceType.AMD).data_ptr() == t.data_ptr()


def test_rearrange_empty_and_one_element():
    e = L.Tensor((0, 5), L.DataType.F32, **AMD)
    L.Ops.rearrange(L.Tensor((0, 5), L.DataType.F32, **AMD), e)
    one = L.Tensor.from_numpy(np.array([[3.5]], np.float32), **AMD)
    out = L.Tensor((1, 1), L.DataType.F32, **AMD)
    L.Ops.rearrange(out, one.permute(1, 0))
    assert out.numpy()[0, 0] == np.float32(3.5)
