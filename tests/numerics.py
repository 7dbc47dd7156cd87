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


def _as_f32(a):
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def assert_attention_close(got, exp, v, what=""):
    """Attention outputs against the oracle.  Each output is a softmax-weighted sum over up
    to `total` keys; the reference accumulates it left to right in f32, so its own rounding
    error is of the order of 2^-24 * sqrt(total) * max|v|, and an output that cancels to
    near 0 cannot be matched to a few ulps by any other summation order.  Bound: within the
    op's usual tolerance (2 ulps for bf16 / f16, 1e-5 relative for f32) OR within an
    absolute floor of max(2^-16, 8 * sqrt(total) * 2^-24) * max|v| (total = v.shape[0], the
    keys: the second term, a few standard deviations of the random-walk error of two f32
    summation orders, exceeds the first from about 16K keys on)."""
    got, exp = np.asarray(got), np.asarray(exp)
    assert got.shape == exp.shape and got.dtype == exp.dtype, (what, got.shape, exp.shape)
    g, e = _as_f32(got).astype(np.float64), _as_f32(exp).astype(np.float64)
    assert np.array_equal(np.isnan(g), np.isnan(e)), f"{what}: NaN pattern differs"
    fin = np.isfinite(e)
    total = np.asarray(v).shape[0] if np.asarray(v).ndim == 3 else 1
    floor = max(2.0 ** -16, 8.0 * np.sqrt(total) * 2.0 ** -24) * float(np.abs(_as_f32(v)).max(initial=0.0))
    absd = np.abs(g[fin] - e[fin])
    if exp.dtype == np.float32:
        ok = absd <= F32_RTOL * np.abs(e[fin])
    elif exp.dtype == np.uint16:
        ok = bf16_ulp_distance(got[fin], exp[fin]) <= HALF_ULPS
    else:
        ok = _f16_ulps(got[fin], exp[fin]) <= HALF_ULPS
    ok |= absd <= floor
    assert ok.all(), (f"{what}: {(~ok).sum()} of {ok.size} outputs beyond tolerance "
                      f"(max abs diff {absd.max():.3g}, floor {floor:.3g})")


def assert_linear_close(got, exp, x, w, what="", w_scale=None):
    """Linear outputs against the oracle.  Each output is a K-term dot product that the
    reference sums left to right in f32; the GPU sums the same exact products in another
    order, so the two f32 sums differ by at most about K * 2^-24 * sum_k |x_k w_k| (much less
    in practice).  Bound: the op's usual tolerance (2 ulps bf16 / f16, 1e-5 relative f32) OR
    an absolute floor of 2^-16 * sum_k |x_k w_k| (times w_scale[n] for INT8 weights), which
    covers outputs that cancel to near 0."""
    got, exp = np.asarray(got), np.asarray(exp)
    assert got.shape == exp.shape and got.dtype == exp.dtype, (what, got.shape, exp.shape)
    g, e = _as_f32(got).astype(np.float64), _as_f32(exp).astype(np.float64)
    assert np.array_equal(np.isnan(g), np.isnan(e)), f"{what}: NaN pattern differs"
    wf = w.astype(np.float64) if w.dtype == np.int8 else _as_f32(w).astype(np.float64)
    mag = np.abs(_as_f32(x).astype(np.float64)) @ np.abs(wf).T
    if w_scale is not None:
        mag = mag * np.abs(np.asarray(w_scale, dtype=np.float64))[None, :]
    floor = 2.0 ** -16 * mag
    fin = np.isfinite(e)
    absd = np.abs(g - e)
    if exp.dtype == np.float32:
        ok = absd <= F32_RTOL * np.abs(e)
    elif exp.dtype == np.uint16:
        ok = bf16_ulp_distance(got, exp) <= HALF_ULPS
    else:
        ok = _f16_ulps(got, exp) <= HALF_ULPS
    ok = (ok | (absd <= floor))[fin]
    assert np.array_equal(got[~fin], exp[~fin]), f"{what}: non-finite outputs differ"
    assert ok.all(), (f"{what}: {(~ok).sum()} of {ok.size} outputs beyond tolerance "
                      f"(max abs diff {absd[fin].max():.3g})")
