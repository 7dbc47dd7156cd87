"""C ABI and host-side logic of libllaisys.so (no GPU needed).

- every function declared in include/ is exported, and so is every name the
  reference's ctypes loader binds (python/llaisys/libllaisys/*.py);
- the runtime table and tensor metadata behave like the reference's test_runtime.py /
  test_tensor.py on the CPU device;
- argument errors print and end the process like the reference (checked in a
  subprocess, since the library throws through ctypes).
"""
import ctypes
import re
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest

import llaisys_amd as L
from llaisys_amd.libllaisys import LIB_PATH

ROOT = Path(__file__).resolve().parents[1]


def _declared_exports():
    names = set()
    for h in (ROOT / "include").rglob("*.h"):
        text = re.sub(r"/\*.*?\*/|//[^\n]*", "", h.read_text(), flags=re.S)
        text = "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))
        names |= set(re.findall(r"__export\s+[^;(]*?\b(\w+)\s*\(", text))
    return names


def _defined_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_every_declared_symbol_is_exported():
    declared = _declared_exports()
    assert len(declared) >= 35
    missing = declared - _defined_symbols()
    assert not missing, missing


def test_reference_loader_names_are_exported():
    # names bound by the reference's python/llaisys/libllaisys/{runtime,tensor,ops,qwen2}.py
    ref_names = {
        "llaisysGetRuntimeAPI", "llaisysSetContextRuntime",
        "tensorCreate", "tensorDestroy", "tensorGetData", "tensorGetNdim", "tensorGetShape",
        "tensorGetStrides", "tensorGetDataType", "tensorGetDeviceType", "tensorGetDeviceId",
        "tensorDebug", "tensorIsContiguous", "tensorLoad", "tensorView", "tensorPermute",
        "tensorSlice",
        "llaisysAdd", "llaisysArgmax", "llaisysEmbedding", "llaisysLinear", "llaisysRearrange",
        "llaisysRmsNorm", "llaisysROPE", "llaisysSelfAttention", "llaisysSwiGLU",
        "llaisysQwen2ModelCreate", "llaisysQwen2ModelDestroy", "llaisysQwen2ModelWeights",
        "llaisysQwen2ModelInfer",
    }
    assert not ref_names - _defined_symbols()


def test_enum_values_match_the_c_header():
    text = (ROOT / "include" / "llaisys.h").read_text()
    for name, val in (("LLAISYS_DEVICE_CPU", 0), ("LLAISYS_DEVICE_NVIDIA", 1), ("LLAISYS_DEVICE_AMD", 2),
                      ("LLAISYS_DTYPE_I8", 3), ("LLAISYS_DTYPE_I64", 6), ("LLAISYS_DTYPE_F16", 12),
                      ("LLAISYS_DTYPE_F32", 13), ("LLAISYS_DTYPE_BF16", 19)):
        assert re.search(rf"{name}\s*=\s*{val}\b", text), name
    assert L.DeviceType.AMD == 2 and L.DeviceType.COUNT == 3 and L.DataType.BF16 == 19


def test_runtime_table_cpu_roundtrip():
    api = L.RuntimeAPI(L.DeviceType.CPU)
    assert api.get_device_count() == 1
    n = 1 << 20
    a = np.zeros(n, np.uint8)
    b = np.ones(n, np.uint8)
    da, db = api.malloc_device(n), api.malloc_device(n)
    api.memcpy_sync(da, a.ctypes.data, n, L.MemcpyKind.H2D)
    api.memcpy_sync(db, da, n, L.MemcpyKind.D2D)
    api.memcpy_sync(b.ctypes.data, db, n, L.MemcpyKind.D2H)
    assert not b.any()
    api.free_device(da)
    api.free_device(db)


def test_nvidia_slot_reports_no_devices():
    assert L.RuntimeAPI(L.DeviceType.NVIDIA).get_device_count() == 0


def test_tensor_metadata_like_reference_test_tensor():
    data = np.arange(3 * 4 * 5, dtype=np.float32).reshape(3, 4, 5)
    t = L.Tensor.from_numpy(data, device=L.DeviceType.CPU)
    assert t.shape() == (3, 4, 5) and t.strides() == (20, 5, 1) and t.is_contiguous()
    assert t.dtype() == L.DataType.F32 and t.device_type() == L.DeviceType.CPU
    assert np.array_equal(t.numpy(), data)
    v = t.view(6, 10)
    assert v.shape() == (6, 10) and v.strides() == (10, 1)
    p = t.permute(2, 0, 1)
    assert p.shape() == (5, 3, 4) and p.strides() == (1, 20, 5) and not p.is_contiguous()
    s = t.slice(2, 1, 4)
    assert s.shape() == (3, 4, 3) and s.strides() == (20, 5, 1) and not s.is_contiguous()
    s0 = t.slice(0, 1, 3)
    assert s0.is_contiguous() and np.array_equal(s0.numpy(), data[1:3])
    # a view of a slice addresses the slice (the reference resets the offset to 0 here)
    assert np.array_equal(s0.view(40).numpy(), data[1:3].reshape(40))
    assert s0.data_ptr() == t.data_ptr() + 20 * 4


def test_tensor_contiguous_reshape_to_on_host_tensors():
    # host tensors: contiguous / reshape / to are data movement (reference tensor.hpp:55-57)
    data = np.arange(3 * 4 * 5, dtype=np.float32).reshape(3, 4, 5)
    t = L.Tensor.from_numpy(data, device=L.DeviceType.CPU)
    same = t.contiguous()
    assert same.data_ptr() == t.data_ptr()  # already contiguous: shared storage
    p = t.permute(2, 0, 1)
    c = p.contiguous()
    assert c.is_contiguous() and c.data_ptr() != t.data_ptr()
    assert np.array_equal(c.numpy(), np.ascontiguousarray(data.transpose(2, 0, 1)))
    s = t.slice(2, 1, 4)
    assert np.array_equal(s.contiguous().numpy(), data[:, :, 1:4])
    r = p.reshape(5, 12)
    assert r.shape() == (5, 12) and np.array_equal(r.numpy(), data.transpose(2, 0, 1).reshape(5, 12))
    assert t.reshape(60).data_ptr() == t.data_ptr()
    h = p.to(L.DeviceType.CPU)
    assert h.data_ptr() == p.data_ptr() and not h.is_contiguous()  # already there
    i8 = L.Tensor.from_numpy(np.arange(24, dtype=np.int8).reshape(2, 3, 4), device=L.DeviceType.CPU)
    assert np.array_equal(i8.permute(1, 2, 0).contiguous().numpy(),
                          np.arange(24, dtype=np.int8).reshape(2, 3, 4).transpose(1, 2, 0))


def test_tensor_load_and_bf16_roundtrip():
    from llaisys_amd.hostfmt import bf16_to_f32, f32_to_bf16
    x = np.random.default_rng(0).standard_normal((7, 9)).astype(np.float32)
    t = L.Tensor.from_numpy(f32_to_bf16(x), L.DataType.BF16, device=L.DeviceType.CPU)
    back = bf16_to_f32(t.numpy())
    assert np.abs(back - x).max() <= np.abs(x).max() * 2 ** -8


def _run(code):
    prog = textwrap.dedent(f"""
        import sys; sys.path.insert(0, {str(ROOT)!r})
        import numpy as np
        import llaisys_amd as L
        C = L.DeviceType.CPU
        def t(shape, dt=L.DataType.F32):
            return L.Tensor(shape, dt, C)
        {textwrap.indent(textwrap.dedent(code), '        ').strip()}
        print("RETURNED")
    """)
    return subprocess.run([sys.executable, "-c", prog], capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize("code,message", [
    ("x=t((4,8)); L.Ops.rms_norm(t((4,8)), x, t((8,)), 1e-5)", "Unsupported device"),
    ("L.Ops.rms_norm(t((4,8)), t((4,8)), t((7,)), 1e-5)", "RMSNorm weight shape mismatch"),
    ("L.Ops.rms_norm(t((4,8)), t((4,8)), t((8,), L.DataType.BF16), 1e-5)", "Datatypes mismatch"),
    ("L.Ops.swiglu(t((4,8)), t((4,8)), t((4,9)))", "Shapes mismatch"),
    ("L.Ops.rope(t((2,1,4)), t((2,1,4)), t((2,), L.DataType.I32), 1e4)", "token id data type must be INT64"),
    ("L.Ops.rope(t((2,1,3)), t((2,1,3)), t((2,), L.DataType.I64), 1e4)", "Head dimension must be even"),
    ("L.Ops.embedding(t((2,4)), t((2,), L.DataType.F32), t((8,4)))", "index data type must be INT32 or INT64"),
    ("L.Ops.argmax(t((1,), L.DataType.F32), t((1,)), t((8,)))", "max_idx must be INT32 or INT64"),
    ("L.Ops.rearrange(t((2,2)), t((2,2)))", "Unsupported device"),
    ("L.Ops.rearrange(t((2,3)), t((3,2)))", "Shapes mismatch"),
    ("L.Ops.random_sample(t((1,), L.DataType.I64), t((10,)), 0.8, 2000, 0.9, 1)", "top_k must be 1 or in [2, 1024]"),
    ("L.Ops.random_sample(t((2,), L.DataType.I64), t((3, 10)), 0.8, 20, 0.9, 1)", "one index per row"),
    ("L.Ops.linear(t((2,2)), t((2,2)), t((2,2)), t((3,)))", "Linear: bias shape mismatch"),
    ("L.Ops.linear(t((2,3)), t((2,2)), t((2,2)), t((2,)))", "Linear: output feature dim mismatch"),
    ("L.Ops.linear(t((2,2)), t((2,2)), t((2,2)))", "Unsupported device"),
    ("L.Ops.linear_w8a16(t((2,2)), t((2,2)), t((2,2)), t((2,)))", "weight codes must be INT8"),
    ("L.Ops.rms_norm_linear(t((1,4)), t((1,8)), t((8,)), 1e-6, t((4,8)))", "Unsupported device"),
    ("L.Ops.rms_norm_linear(t((1,3)), t((1,8)), t((8,)), 1e-6, t((7,8)), swiglu=True)", "swiglu needs an even number"),
    ("L.Ops.rms_norm_linear(t((1,4)), t((1,8)), t((8,)), 1e-6, t((8,8)), swiglu=False)", "Linear: output feature dim mismatch"),
    ("L.Ops.rms_norm_linear(t((1,4)), t((1,8)), t((8,)), 1e-6, t((4,8)), residual=t((1,8)))", "residual and residual_out come together"),
    ("x=t((1,8)); L.Ops.rms_norm_linear(t((1,4)), x, t((8,)), 1e-6, t((4,8)), residual=t((1,8)), residual_out=x)", "residual_out must not overlap"),
    ("x=t((1,8)); L.Ops.rms_norm_linear(x, x, t((8,)), 1e-6, t((8,8)))", "out must not overlap"),
    ("L.Ops.rms_norm_linear(t((1,4)), t((1,8)), t((8,)), 1e-6, t((4,8)), weight_scale=t((4,)))", "weight codes must be INT8"),
    ("L.Ops.kv_append_int8(t((4,2,8), L.DataType.I8), t((4,2)), t((3,2,8)), 2)", "append past the cache end"),
    ("L.Ops.quantize_int8(t((4,8), L.DataType.I8), t((3,)), t((4,8)))", "one scale per last-dim row"),
    ("L.Tensor((2,), L.DataType.F32, L.DeviceType.AMD, 0)", "invalid device id"),
    ("L.Ops.cast(t((2,2), L.DataType.BF16), t((2,2)))", "Unsupported device"),
    ("L.Ops.cast(t((2,3), L.DataType.BF16), t((2,2)))", "Shapes mismatch"),
    ("L.Ops.cast(t((2,2), L.DataType.I32), t((2,2)))", "Unsupported data type"),
    # 48 query-heads of head_dim 128 need 25.6 MB of partials: beyond the fixed 24 MiB scratch
    ("I8 = L.DataType.I8; L.Ops.self_attention_int8kv_noalloc(t((48,1,128)), t((48,1,128)), t((4,1,128), I8), "
     "t((4,1)), t((4,1,128), I8), t((4,1)), 0.1)", "more than the 25165824 it holds"),
    ("I8 = L.DataType.I8; L.Ops.self_attention_int8kv_noalloc(t((2,1,128)), t((2,1,128)), t((4,1,128), I8), "
     "t((4,1)), t((4,1,128), I8), t((4,1)), 0.1)", "Unsupported device"),
])
def test_errors_print_and_abort_like_the_reference(code, message):
    if "AMD" in code and L.RuntimeAPI(L.DeviceType.AMD).get_device_count() > 0:
        pytest.skip("a GPU is present")
    r = _run(code)
    assert r.returncode != 0 and "RETURNED" not in r.stdout
    assert message in r.stderr, r.stderr[-2000:]
    assert "[ERROR]" in r.stderr
