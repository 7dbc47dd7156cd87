"""Comparison rules of the parity tests.

Tolerances: integer work bit-exact; f32 within 1e-5 relative;
bf16 within 2 bf16 ulps; f16 within 2 f16 ulps.  All against the f32-accumulating CPU
oracle / reference outputs.  Non-finite values must match exactly.
"""
import numpy as np

from llaisys_amd.hostfmt import bf16_ulp_distance

F32_RTOL = 1e-5
HALF_ULPS = 2


def _f16_ulps(a, b):
    def key(u):
        u = np.asarray(u).view(np.uint16).astype(np.int32)
        return np.where(u & 0x8000, 0x8000 - u, u)
    return np.abs(key(a) - key(b))


def assert_close(got, exp, what=""):
    got, exp = np.asarray(got), np.asarray(exp)
    assert got.shape == exp.shape and got.dtype == exp.dtype, (what, got.shape, exp.shape)
    if got.size == 0:
        return
    if exp.dtype == np.float32:
        fin = np.isfinite(exp)
        assert np.array_equal(np.isnan(got), np.isnan(exp)), f"{what}: NaN pattern differs"
        assert np.array_equal(got[~fin & ~np.isnan(exp)], exp[~fin & ~np.isnan(exp)]), f"{what}: inf differs"
        err = np.abs(got[fin].astype(np.float64) - exp[fin]) / np.maximum(np.abs(exp[fin]), 1e-38)
        bad = err > F32_RTOL
        assert not bad.any(), f"{what}: {bad.sum()} f32 values beyond 1e-5 rel (max {err.max():.3g})"
    elif exp.dtype == np.uint16:  # bf16 bits
        gf = (got.astype(np.uint32) << 16).view(np.float32)
        ef = (exp.astype(np.uint32) << 16).view(np.float32)
        fin = np.isfinite(ef)
        assert np.array_equal(got[~fin], exp[~fin]), f"{what}: non-finite bf16 differ"
        d = bf16_ulp_distance(got[fin], exp[fin])
        assert d.max(initial=0) <= HALF_ULPS, f"{what}: bf16 off by {d.max()} ulps ({(d > HALF_ULPS).sum()} values)"
    elif exp.dtype == np.float16:
        fin = np.isfinite(exp)
        assert np.array_equal(got[~fin].view(np.uint16), exp[~fin].view(np.uint16)), f"{what}: non-finite f16 differ"
        d = _f16_ulps(got[fin], exp[fin])
        assert d.max(initial=0) <= HALF_ULPS, f"{what}: f16 off by {d.max()} ulps"
    else:
        assert np.array_equal(got, exp), f"{what}: integer results differ"


def assert_exact(got, exp, what=""):
    got, exp = np.asarray(got), np.asarray(exp)
    assert got.shape == exp.shape and got.dtype == exp.dtype, (what, got.shape, exp.shape)
    assert np.array_equal(got.view(np.uint8), exp.view(np.uint8)), f"{what}: not bit-identical"
