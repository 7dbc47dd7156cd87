"""numpy front end of the CPU oracle (oracle.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
always as the checker or the timed CPU baseline, never as a compute path of the product.
Arrays use the host formats of llaisys_amd.hostfmt: bf16 as uint16 bits, f16 as float16.

`reference_library()` loads oracle/_ref/libllaisys_ref.so, the reference's own CPU
library compiled from its sources by `make -C oracle ref` (present where /root/reference
was available at build time).
"""
import ctypes
from ctypes import c_float, c_int, c_size_t, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).parent
LIB_PATH = HERE / "_build" / "liboracle.so"
REF_PATH = HERE / "_ref" / "libllaisys_ref.so"

F16, F32, BF16, I32, I64 = 12, 13, 19, 5, 6
_CODE = {np.dtype(np.float32): F32, np.dtype(np.float16): F16, np.dtype(np.uint16): BF16}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise FileNotFoundError(f"{LIB_PATH} missing: run make -C oracle")
        L = ctypes.CDLL(str(LIB_PATH))
        P = c_void_p
        sig = {
            "orc_add": [P, P, P, c_size_t, c_int],
            "orc_rms_norm": [P, P, P, c_size_t, c_size_t, c_float, c_int],
            "orc_add_rms_norm": [P, P, P, P, P, c_size_t, c_size_t, c_float, c_int],
            "orc_rope": [P, P, P, c_size_t, c_size_t, c_size_t, c_float, c_int],
            "orc_swiglu": [P, P, P, c_size_t, c_int],
            "orc_embedding": [P, P, c_int, c_size_t, P, c_size_t, c_size_t, c_int],
            "orc_argmax": [P, c_int, P, P, c_size_t, c_int],
            "orc_argmax_rows": [P, c_int, P, P, c_size_t, c_size_t, c_int],
            "orc_quantize_int8": [P, P, P, c_size_t, c_size_t, c_int],
            "orc_dequantize_int8": [P, P, P, c_size_t, c_size_t, c_int],
            "orc_kv_append_int8": [P, P, c_size_t, P, c_size_t, c_size_t, c_size_t, c_size_t, c_int],
            "orc_self_attention": [P, P, P, P, c_size_t, c_size_t, c_size_t, c_size_t, c_size_t,
                                   c_size_t, c_float, c_int],
            "orc_linear": [P, P, P, P, c_size_t, c_size_t, c_size_t, c_int],
            "orc_linear_w8a16": [P, P, P, P, P, c_size_t, c_size_t, c_size_t, c_int],
            "orc_random_sample": [P, P, c_size_t, c_size_t, c_int, c_float, ctypes.c_int64, c_float,
                                  ctypes.c_uint64],
            "orc_cast": [P, c_int, P, c_int, c_size_t],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = c_int if name in ("orc_embedding", "orc_kv_append_int8", "orc_self_attention",
                                           "orc_random_sample") else None
        L.orc_sample_exp2.argtypes = [c_float]
        L.orc_sample_exp2.restype = c_float
        L.orc_splitmix64.argtypes = [ctypes.c_uint64]
        L.orc_splitmix64.restype = ctypes.c_uint64
        for name in ("orc_f32_to_bf16", "orc_f32_to_f16"):
            getattr(L, name).argtypes = [c_float]
            getattr(L, name).restype = ctypes.c_uint16
        for name in ("orc_bf16_to_f32", "orc_f16_to_f32"):
            getattr(L, name).argtypes = [ctypes.c_uint16]
            getattr(L, name).restype = c_float
        _lib = L
    return _lib


def reference_library():
    """ctypes handle of the compiled reference CPU library, or None if it was not built."""
    if not REF_PATH.is_file():
        return None
    return ctypes.CDLL(str(REF_PATH))


def _p(a):
    return a.ctypes.data_as(c_void_p)


def _code(a):
    return _CODE[np.dtype(a.dtype)]


def _c(a):
    return np.ascontiguousarray(a)


_NP_OF = {F32: np.float32, F16: np.float16, BF16: np.uint16}


def cast(x, out_code):
    """The reference's cast<To>(From) (types.hpp:116-139) of every element of x (host
    formats: bf16 as uint16 bits) into out_code (F32 / F16 / BF16)."""
    x = _c(x)
    out = np.empty(x.shape, dtype=_NP_OF[out_code])
    lib().orc_cast(_p(out), out_code, _p(x), _code(x), x.size)
    return out


def add(a, b):
    a, b = _c(a), _c(b)
    c = np.empty_like(a)
    lib().orc_add(_p(c), _p(a), _p(b), a.size, _code(a))
    return c


def rms_norm(x, w, eps):
    x, w = _c(x), _c(w)
    y = np.empty_like(x)
    cols = x.shape[-1]
    lib().orc_rms_norm(_p(y), _p(x), _p(w), x.size // cols, cols, eps, _code(x))
    return y


def add_rms_norm(x, r, w, eps):
    x, r, w = _c(x), _c(r), _c(w)
    y, h = np.empty_like(x), np.empty_like(x)
    cols = x.shape[-1]
    lib().orc_add_rms_norm(_p(y), _p(h), _p(x), _p(r), _p(w), x.size // cols, cols, eps, _code(x))
    return y, h


def rope(x, pos, theta):
    x, pos = _c(x), np.ascontiguousarray(pos, dtype=np.int64)
    y = np.empty_like(x)
    s, h, d = x.shape
    lib().orc_rope(_p(y), _p(x), _p(pos), s, h, d, theta, _code(x))
    return y


def swiglu(g, u):
    g, u = _c(g), _c(u)
    y = np.empty_like(g)
    lib().orc_swiglu(_p(y), _p(g), _p(u), g.size, _code(g))
    return y


def embedding(idx, w):
    """Returns (out, status); status -1 means an id was out of range."""
    idx, w = _c(idx), _c(w)
    out = np.zeros((idx.size, w.shape[1]), dtype=w.dtype)
    st = lib().orc_embedding(_p(out), _p(idx), I64 if idx.dtype == np.int64 else I32, idx.size,
                             _p(w), w.shape[0], w.shape[1], _code(w))
    return out, st


def argmax(vals, idx_dtype=np.int64):
    vals = _c(vals)
    i = np.zeros(1, dtype=idx_dtype)
    v = np.zeros(1, dtype=vals.dtype)
    lib().orc_argmax(_p(i), I64 if i.dtype == np.int64 else I32, _p(v), _p(vals), vals.size,
                     _code(vals))
    return i[0], v[0]


def argmax_rows(vals, idx_dtype=np.int64):
    vals = _c(vals)
    rows, cols = vals.shape
    i = np.zeros(rows, dtype=idx_dtype)
    v = np.zeros(rows, dtype=vals.dtype)
    lib().orc_argmax_rows(_p(i), I64 if i.dtype == np.int64 else I32, _p(v), _p(vals), rows,
                          cols, _code(vals))
    return i, v


def quantize_int8(x):
    x = _c(x)
    cols = x.shape[-1]
    q = np.empty(x.shape, dtype=np.int8)
    s = np.empty(x.shape[:-1], dtype=np.float32)
    lib().orc_quantize_int8(_p(q), _p(s), _p(x), x.size // cols, cols, _code(x))
    return q, s


def dequantize_int8(q, scale, dtype):
    q, scale = _c(q), np.ascontiguousarray(scale, dtype=np.float32)
    out = np.empty(q.shape, dtype=dtype)
    cols = q.shape[-1]
    lib().orc_dequantize_int8(_p(out), _p(q), _p(scale), q.size // cols, cols, _code(out))
    return out


def kv_append_int8(cache_q, cache_scale, kv, pos):
    """Appends in place into (cache_q, cache_scale); returns the status (0 or -1)."""
    kv = _c(kv)
    max_seq, nkvh, d = cache_q.shape
    return lib().orc_kv_append_int8(_p(cache_q), _p(cache_scale), max_seq, _p(kv), kv.shape[0],
                                    nkvh, d, pos, _code(kv))


def self_attention(q, k, v, scale):
    """Reference self_attention (self_attention_cpu.cpp:13-115): q [seq, nh, d],
    k [total, nkvh, d], v [total, nkvh, dv] of one dtype; returns [seq, nh, dv]."""
    q, k, v = _c(q), _c(k), _c(v)
    assert q.dtype == k.dtype == v.dtype
    seq, nh, d = q.shape
    total, nkvh, dv = v.shape
    assert k.shape == (total, nkvh, d)
    out = np.empty((seq, nh, dv), dtype=q.dtype)
    rc = lib().orc_self_attention(_p(out), _p(q), _p(k), _p(v), seq, total, nh, nkvh, d, dv,
                                  float(scale), _code(q))
    assert rc == 0, "invalid head split"
    return out


def self_attention_int8kv(q, k_codes, k_scale, v_codes, v_scale, scale):
    """Attention over an INT8 cache: self_attention of q with k and v dequantized into
    q's element type (the composition llaisysDequantizeInt8 then llaisysSelfAttention)."""
    k = dequantize_int8(k_codes, k_scale, q.dtype)
    v = dequantize_int8(v_codes, v_scale, q.dtype)
    return self_attention(q, k, v, scale)


def linear(x, w, bias=None):
    """Reference linear (linear_cpu.cpp:11-41): x [rows, in], w [out, in], bias [out]."""
    x, w = _c(x), _c(w)
    rows, in_f = x.shape
    out_f = w.shape[0]
    assert w.shape == (out_f, in_f) and x.dtype == w.dtype
    b = None if bias is None else _c(bias)
    out = np.empty((rows, out_f), dtype=x.dtype)
    lib().orc_linear(_p(out), _p(x), _p(w), None if b is None else _p(b), rows, in_f, out_f, _code(x))
    return out


def linear_w8a16(x, codes, scale, bias=None):
    """W8A16 rule: T(scale[n] * sum_k x[m, k] * codes[n, k] + bias[n])."""
    x, codes = _c(x), np.ascontiguousarray(codes, dtype=np.int8)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    rows, in_f = x.shape
    out_f = codes.shape[0]
    b = None if bias is None else _c(bias)
    out = np.empty((rows, out_f), dtype=x.dtype)
    lib().orc_linear_w8a16(_p(out), _p(x), _p(codes), _p(scale), None if b is None else _p(b), rows,
                           in_f, out_f, _code(x))
    return out


def random_sample(logits, temperature, top_k, top_p, seed):
    """Sampling rule of oracle.h orc_random_sample: logits [V] or [rows, V] -> int64 [rows]."""
    x = _c(logits)
    rows, V = (1, x.shape[0]) if x.ndim == 1 else x.shape
    out = np.empty(rows, dtype=np.int64)
    rc = lib().orc_random_sample(_p(out), _p(x), rows, V, _code(x), float(temperature), int(top_k),
                                 float(top_p), int(seed) & (2 ** 64 - 1))
    if rc != 0:
        raise ValueError("top_k must be 1 or in [2, 1024] when sampling")
    return out


def sample_exp2(t):
    return float(lib().orc_sample_exp2(float(t)))


def splitmix64(x):
    return int(lib().orc_splitmix64(int(x) & (2 ** 64 - 1)))
