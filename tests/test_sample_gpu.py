"""Random sampling on the GPU (llaisysRandomSample) against the oracle's statement of the rule
(oracle/oracle.h orc_random_sample), which tests/test_oracle.py pins by closed forms (greedy
cases are argmax), an independent integer restatement and its sampled distribution.  The
rule is integer work plus IEEE single multiplies / adds in a fixed order, so the indices
must be equal bit for bit."""
import numpy as np
import pytest

import llaisys_amd as L
import oracle
from llaisys_amd.hostfmt import f32_to_bf16

pytestmark = pytest.mark.gpu

AMD = dict(device=L.DeviceType.AMD, device_id=0)
DTS = {"f32": L.DataType.F32, "bf16": L.DataType.BF16, "f16": L.DataType.F16}


def conv(x, dt):
    return {"f32": x.astype(np.float32), "bf16": f32_to_bf16(x.astype(np.float32)), "f16": x.astype(np.float16)}[dt]


def gpu_sample(x, dt, T, k, p, seed, i64=True):
    rows = 1 if x.ndim == 1 else x.shape[0]
    out = L.Tensor((rows,), L.DataType.I64 if i64 else L.DataType.I32, **AMD)
    L.Ops.random_sample(out, L.Tensor.from_numpy(x, DTS[dt], **AMD), T, k, p, seed)
    return out.numpy().astype(np.int64)


CASES = [
    # rows, V, scale, temperature, top_k, top_p
    (1, 151936, 3.0, 0.8, 50, 0.8),     # Qwen2 vocabulary, the reference generate() defaults + top_k
    (1, 151936, 3.0, 1.0, 1024, 0.95),
    (1, 151936, 3.0, 0.7, 40, 1.0),     # top-k only
    (4, 32000, 1.0, 1.3, 200, 0.9),
    (2, 20000, 1.0, 1.0, 300, 0.9),     # k > 256: the 512-thread finish, a 512-item sort
    (20, 5000, 2.0, 0.9, 64, 0.7),      # more than 16 rows: two launches
    (3, 100, 1.0, 1.0, 500, 0.9),       # k > V
    (2, 4097, 5.0, 0.5, 2, 0.0),        # top_p <= 0: the top token
    (1, 151936, 3.0, 0.0, 50, 0.8),     # temperature 0: argmax
    (5, 3000, 1.0, 0.8, 1, 0.8),        # top_k 1: argmax
]


@pytest.mark.parametrize("dt", ["bf16", "f32", "f16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_random_sample_matches_oracle(case, dt):
    rows, V, scale, T, k, p = case
    rng = np.random.default_rng(hash((case, dt)) % 2 ** 32)
    x = conv(rng.standard_normal((rows, V)) * scale, dt)
    for seed in (0, 12345, 2 ** 63 + 7):
        exp = oracle.random_sample(x, T, k, p, seed)
        got = gpu_sample(x, dt, T, k, p, seed)
        assert np.array_equal(got, exp), (case, dt, seed, got, exp)


def test_random_sample_ties_and_tie_overflow():
    rng = np.random.default_rng(4)
    # many exact ties around the k-th key (rounded logits) and more ties than the list holds
    x1 = np.round(rng.standard_normal((3, 20000)) * 2).astype(np.float32)
    x2 = np.zeros((2, 10000), np.float32)
    x2[1, 9999] = 1.0
    for x in (x1, x2):
        for seed in (1, 99):
            for k, p in ((1024, 0.9), (37, 1.0), (5, 0.5)):
                exp = oracle.random_sample(x, 1.0, k, p, seed)
                assert np.array_equal(gpu_sample(x, "f32", 1.0, k, p, seed), exp), (x.shape, k, p, seed)


def test_random_sample_bucket_overflow_with_distinct_keys():
    # more than 4096 logits share the top 22 bits of the k-th key (1 + j ulp, 1024 distinct
    # values, about five copies each, scattered): the finish resolves the last 10 bits in a
    # scan of the row, then takes the members above that key and the ties at it by index
    rng = np.random.default_rng(8)
    x = np.full((2, 20000), -1.0, np.float32)
    for r in range(2):
        pos = rng.choice(20000, 5000, replace=False)
        x[r, pos] = (np.float32(1.0) + (np.arange(5000) % 1024).astype(np.float32) * np.float32(2.0 ** -23))
    x[1, 123] = 2.0  # one key above the bucket
    for seed in (3, 77):
        for k, p in ((100, 0.9), (1024, 1.0), (9, 0.5)):
            exp = oracle.random_sample(x, 1.0, k, p, seed)
            assert np.array_equal(gpu_sample(x, "f32", 1.0, k, p, seed), exp), (k, p, seed)


def test_random_sample_repeats_and_int32_output():
    rng = np.random.default_rng(5)
    x = conv(rng.standard_normal((2, 151936)) * 3, "bf16")
    first = gpu_sample(x, "bf16", 0.8, 100, 0.9, 42)
    for _ in range(3):  # the sampler's scratch state returns to zero after every launch
        assert np.array_equal(gpu_sample(x, "bf16", 0.8, 100, 0.9, 42), first)
    assert np.array_equal(gpu_sample(x, "bf16", 0.8, 100, 0.9, 42, i64=False), first)


def test_random_sample_distribution_on_gpu():
    x = np.array([2.0, 1.0, 0.5, 0.0, -1.0, 3.0, 0.2, -0.3], np.float32)
    T, k, p, n = 1.0, 6, 0.9, 3000
    z = x.astype(np.float64) / T
    order = np.argsort(-z, kind="stable")[:k]
    pr = np.exp(z[order] - z[order].max())
    pr /= pr.sum()
    keep = int(np.searchsorted(np.cumsum(pr), p - 1e-12) + 1)
    probs = np.zeros(len(x))
    probs[order[:keep]] = pr[:keep] / pr[:keep].sum()
    rows = np.tile(x, (n, 1))  # one launch: row r draws with splitmix64(seed + r)
    got = gpu_sample(rows, "f32", T, k, p, 1000)
    assert np.array_equal(got, oracle.random_sample(rows, T, k, p, 1000))
    counts = np.bincount(got, minlength=len(x))
    exp = probs * n
    assert counts[probs == 0].sum() == 0
    m = exp > 0
    chi2 = float((((counts[m] - exp[m]) ** 2) / exp[m]).sum())
    assert chi2 < 30, (counts, exp)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_random_sample_nan_and_infinite_logits(dt):
    """NaN logits order as -inf, infinite maxima share the mass, an all -inf / NaN row
    draws among its lowest indices: the GPU equals the oracle's rule on every row."""
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((4, 151936)) * 3).astype(np.float32)
    x[0, rng.choice(151936, 500, replace=False)] = np.nan
    x[0, 7] = -np.nan
    x[1, [100, 90000]] = np.inf
    x[1, [5, 6]] = np.nan
    x[2, :] = -np.inf
    x[2, [3, 77]] = np.nan
    x[3, :] = np.nan
    x[3, 1234] = 1.0
    xd = conv(x, dt)
    for seed in (0, 5, 2 ** 40 + 3):
        for k, p in ((50, 0.8), (1024, 1.0), (3, 0.5)):
            exp = oracle.random_sample(xd, 1.0, k, p, seed)
            got = gpu_sample(xd, dt, 1.0, k, p, seed)
            assert np.array_equal(got, exp), (dt, seed, k, p, got, exp)
            assert not np.isnan(x[0, got[0]])
            assert x[1, got[1]] == np.inf and got[3] == 1234
