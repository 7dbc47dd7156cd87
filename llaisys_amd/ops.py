"""Ops: the LLAISYS operators as static methods.

The nine reference methods match python/llaisys/ops.py:6-55 (rearrange is implemented here:
a strided copy between two layouts of one shape, where the reference's C++ rearrange is a
stub); the rest wrap the additive entry points of include/llaisys/ops.h.
"""
from ctypes import c_float, c_int64, c_size_t, c_uint8, c_uint64

from .libllaisys import LIB_LLAISYS
from .tensor import Tensor


class Ops:
    @staticmethod
    def add(c: Tensor, a: Tensor, b: Tensor):
        LIB_LLAISYS.llaisysAdd(c.lib_tensor(), a.lib_tensor(), b.lib_tensor())

    @staticmethod
    def argmax(max_idx: Tensor, max_val: Tensor, vals: Tensor):
        LIB_LLAISYS.llaisysArgmax(max_idx.lib_tensor(), max_val.lib_tensor(), vals.lib_tensor())

    @staticmethod
    def embedding(out: Tensor, index: Tensor, weight: Tensor):
        LIB_LLAISYS.llaisysEmbedding(out.lib_tensor(), index.lib_tensor(), weight.lib_tensor())

    @staticmethod
    def linear(out: Tensor, inp: Tensor, weight: Tensor, bias: Tensor = None):
        LIB_LLAISYS.llaisysLinear(out.lib_tensor(), inp.lib_tensor(), weight.lib_tensor(),
                                  None if bias is None else bias.lib_tensor())

    @staticmethod
    def rearrange(out: Tensor, inp: Tensor):
        LIB_LLAISYS.llaisysRearrange(out.lib_tensor(), inp.lib_tensor())

    @staticmethod
    def rms_norm(out: Tensor, inp: Tensor, weight: Tensor, eps: float):
        LIB_LLAISYS.llaisysRmsNorm(out.lib_tensor(), inp.lib_tensor(), weight.lib_tensor(),
                                   c_float(eps))

    @staticmethod
    def rope(out: Tensor, inp: Tensor, pos_ids: Tensor, theta: float):
        LIB_LLAISYS.llaisysROPE(out.lib_tensor(), inp.lib_tensor(), pos_ids.lib_tensor(),
                                c_float(theta))

    @staticmethod
    def self_attention(attn_val: Tensor, q: Tensor, k: Tensor, v: Tensor, scale: float):
        LIB_LLAISYS.llaisysSelfAttention(attn_val.lib_tensor(), q.lib_tensor(), k.lib_tensor(),
                                         v.lib_tensor(), c_float(scale))

    @staticmethod
    def swiglu(out: Tensor, gate: Tensor, up: Tensor):
        LIB_LLAISYS.llaisysSwiGLU(out.lib_tensor(), gate.lib_tensor(), up.lib_tensor())

    # ---- additive ops -----------------------------------------------------------------
    @staticmethod
    def add_rms_norm(out: Tensor, residual_out: Tensor, inp: Tensor, residual: Tensor,
                     weight: Tensor, eps: float):
        LIB_LLAISYS.llaisysAddRmsNorm(out.lib_tensor(), residual_out.lib_tensor(),
                                      inp.lib_tensor(), residual.lib_tensor(),
                                      weight.lib_tensor(), c_float(eps))

    @staticmethod
    def rope_qk(q_out: Tensor, q_in: Tensor, k_out: Tensor, k_in: Tensor, pos_ids: Tensor,
                theta: float):
        LIB_LLAISYS.llaisysROPEQK(q_out.lib_tensor(), q_in.lib_tensor(), k_out.lib_tensor(),
                                  k_in.lib_tensor(), pos_ids.lib_tensor(), c_float(theta))

    @staticmethod
    def rope_kv_append_int8(q_out: Tensor, q_in: Tensor, k_in: Tensor, v_in: Tensor,
                            pos_ids: Tensor, theta: float, k_cache: Tensor, k_scale: Tensor,
                            v_cache: Tensor, v_scale: Tensor, pos: int):
        LIB_LLAISYS.llaisysROPEKVAppendInt8(
            q_out.lib_tensor(), q_in.lib_tensor(), k_in.lib_tensor(), v_in.lib_tensor(),
            pos_ids.lib_tensor(), c_float(theta), k_cache.lib_tensor(), k_scale.lib_tensor(),
            v_cache.lib_tensor(), v_scale.lib_tensor(), c_size_t(pos))

    @staticmethod
    def argmax_rows(max_idx: Tensor, max_val: Tensor, vals: Tensor):
        LIB_LLAISYS.llaisysArgmaxRows(max_idx.lib_tensor(), max_val.lib_tensor(),
                                      vals.lib_tensor())

    @staticmethod
    def quantize_int8(q: Tensor, scale: Tensor, inp: Tensor):
        LIB_LLAISYS.llaisysQuantizeInt8(q.lib_tensor(), scale.lib_tensor(), inp.lib_tensor())

    @staticmethod
    def dequantize_int8(out: Tensor, q: Tensor, scale: Tensor):
        LIB_LLAISYS.llaisysDequantizeInt8(out.lib_tensor(), q.lib_tensor(), scale.lib_tensor())

    @staticmethod
    def kv_append_int8(cache_q: Tensor, cache_scale: Tensor, kv: Tensor, pos: int):
        LIB_LLAISYS.llaisysKVAppendInt8(cache_q.lib_tensor(), cache_scale.lib_tensor(),
                                        kv.lib_tensor(), c_size_t(pos))

    @staticmethod
    def kv_append_int8_pair(k_cache: Tensor, k_scale: Tensor, v_cache: Tensor, v_scale: Tensor,
                            k: Tensor, v: Tensor, pos: int):
        LIB_LLAISYS.llaisysKVAppendInt8Pair(k_cache.lib_tensor(), k_scale.lib_tensor(),
                                            v_cache.lib_tensor(), v_scale.lib_tensor(),
                                            k.lib_tensor(), v.lib_tensor(), c_size_t(pos))

    @staticmethod
    def self_attention_int8kv(attn_val: Tensor, q: Tensor, k_codes: Tensor, k_scale: Tensor,
                              v_codes: Tensor, v_scale: Tensor, scale: float):
        LIB_LLAISYS.llaisysSelfAttentionInt8KV(attn_val.lib_tensor(), q.lib_tensor(),
                                               k_codes.lib_tensor(), k_scale.lib_tensor(),
                                               v_codes.lib_tensor(), v_scale.lib_tensor(),
                                               c_float(scale))

    @staticmethod
    def self_attention_int8kv_noalloc(attn_val: Tensor, q: Tensor, k_codes: Tensor, k_scale: Tensor,
                                      v_codes: Tensor, v_scale: Tensor, scale: float):
        """self_attention_int8kv without allocating: partials in the library's fixed device
        scratch (llaisysSelfAttentionInt8KVNoAlloc)."""
        LIB_LLAISYS.llaisysSelfAttentionInt8KVNoAlloc(attn_val.lib_tensor(), q.lib_tensor(),
                                                      k_codes.lib_tensor(), k_scale.lib_tensor(),
                                                      v_codes.lib_tensor(), v_scale.lib_tensor(),
                                                      c_float(scale))

    @staticmethod
    def cast(out: Tensor, inp: Tensor):
        """out = cast(inp) on the device with the reference's conversion rules (llaisysCast)."""
        LIB_LLAISYS.llaisysCast(out.lib_tensor(), inp.lib_tensor())

    @staticmethod
    def dequantize_int8_pair(out0: Tensor, q0: Tensor, scale0: Tensor, out1: Tensor, q1: Tensor,
                             scale1: Tensor):
        LIB_LLAISYS.llaisysDequantizeInt8Pair(out0.lib_tensor(), q0.lib_tensor(),
                                              scale0.lib_tensor(), out1.lib_tensor(),
                                              q1.lib_tensor(), scale1.lib_tensor())

    @staticmethod
    def linear_w8a16(out: Tensor, inp: Tensor, w_codes: Tensor, w_scale: Tensor,
                     bias: Tensor = None):
        LIB_LLAISYS.llaisysLinearW8A16(out.lib_tensor(), inp.lib_tensor(), w_codes.lib_tensor(),
                                       w_scale.lib_tensor(),
                                       None if bias is None else bias.lib_tensor())

    @staticmethod
    def rms_norm_linear(out: Tensor, inp: Tensor, norm_weight: Tensor, eps: float, weight: Tensor,
                        weight_scale: Tensor = None, bias: Tensor = None, residual: Tensor = None,
                        residual_out: Tensor = None, swiglu: bool = False):
        """out = linear(rms_norm(inp [+ residual])) [then swiglu over the weight's two halves];
        residual_out receives inp + residual."""
        opt = lambda t: None if t is None else t.lib_tensor()
        LIB_LLAISYS.llaisysRmsNormLinear(out.lib_tensor(), opt(residual_out), inp.lib_tensor(),
                                         opt(residual), norm_weight.lib_tensor(), c_float(eps),
                                         weight.lib_tensor(), opt(weight_scale), opt(bias),
                                         c_uint8(1 if swiglu else 0))

    @staticmethod
    def random_sample(out_idx: Tensor, logits: Tensor, temperature: float, top_k: int, top_p: float,
                      seed: int):
        LIB_LLAISYS.llaisysRandomSample(out_idx.lib_tensor(), logits.lib_tensor(), c_float(temperature),
                                        c_int64(top_k), c_float(top_p), c_uint64(seed & (2 ** 64 - 1)))
