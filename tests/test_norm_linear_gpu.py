"""llaisysRmsNormLinear on the GPU: rms_norm (after an optional residual add) fused ahead of a
linear, optionally with swiglu after it.

The fused kernel is specified as the composition of the library's own ops: for one row it
must equal rms_norm / add_rms_norm -> linear (the one-row GEMV) -> swiglu launched
separately, bit for bit; other row counts run that composition.  Each op of the
composition is checked against the oracle in its own test file; here the fused output is
also checked against the oracle directly: the stored residual bit for bit (oracle add), and
the projection against the oracle's linear of the normalised row (numerics tolerance)."""
import numpy as np
import pytest

import llaisys_amd as L
import oracle
from llaisys_amd.hostfmt import bf16_to_f32, f32_to_bf16
from numerics import assert_exact, assert_linear_close

pytestmark = pytest.mark.gpu

AMD = dict(device=L.DeviceType.AMD, device_id=0)
DTS = {"bf16": L.DataType.BF16, "f16": L.DataType.F16, "f32": L.DataType.F32}
EPS = 1e-6


def sample(rng, shape, dt, s=1.0, mean=0.0):
    x = (mean + s * rng.standard_normal(shape)).astype(np.float32)
    return {"f32": x, "bf16": f32_to_bf16(x), "f16": x.astype(np.float16)}[dt]


def to_f32(a, dt):
    return bf16_to_f32(a) if dt == "bf16" else a.astype(np.float32)


def dev(a, dt=None):
    return L.Tensor.from_numpy(a, dt, **AMD)


def empty(shape, dt):
    return L.Tensor(shape, DTS[dt], **AMD)


class Case:
    def __init__(self, rows, K, N, dt, int8, swiglu, bias, res, seed=0):
        rng = np.random.default_rng(seed + 7919 * K + N)
        self.rows, self.K, self.N, self.dt, self.int8, self.swiglu = rows, K, N, dt, int8, swiglu
        Nw = 2 * N if swiglu else N
        self.x = sample(rng, (rows, K), dt)
        self.r = sample(rng, (rows, K), dt) if res else None
        self.nw = sample(rng, (K,), dt, 0.1, 1.0)
        if int8:
            self.w = rng.integers(-127, 128, size=(Nw, K), dtype=np.int8)
            self.sc = ((0.5 + rng.random(Nw)) / 127 / np.sqrt(K)).astype(np.float32)
        else:
            self.w = sample(rng, (Nw, K), dt, 1.0 / np.sqrt(K))
            self.sc = None
        self.b = sample(rng, (Nw,), dt, 0.1) if bias else None
        self.t = {k: (None if v is None else dev(v, None if k in ("w", "sc") and int8 else DTS[dt]))
                  for k, v in dict(x=self.x, r=self.r, nw=self.nw, w=self.w, sc=self.sc, b=self.b).items()}

    def fused(self):
        out = empty((self.rows, self.N), self.dt)
        h = empty((self.rows, self.K), self.dt) if self.r is not None else None
        t = self.t
        L.Ops.rms_norm_linear(out, t["x"], t["nw"], EPS, t["w"], t["sc"], t["b"], residual=t["r"],
                              residual_out=h, swiglu=self.swiglu)
        return out.numpy(), None if h is None else h.numpy()

    def _lin(self, out, xn, w, sc, b):
        if sc is None:
            L.Ops.linear(out, xn, w, b)
        else:
            L.Ops.linear_w8a16(out, xn, w, sc, b)

    def composed(self):
        """The library's separate ops: (add_)rms_norm, linear per weight half, swiglu."""
        t, rows, K, N, dt = self.t, self.rows, self.K, self.N, self.dt
        xn = empty((rows, K), dt)
        h = None
        if self.r is not None:
            h = empty((rows, K), dt)
            L.Ops.add_rms_norm(xn, h, t["x"], t["r"], t["nw"], EPS)
        else:
            L.Ops.rms_norm(xn, t["x"], t["nw"], EPS)
        out = empty((rows, N), dt)
        if not self.swiglu:
            self._lin(out, xn, t["w"], t["sc"], t["b"])
        else:
            halves = []
            for i in range(2):
                w = t["w"].slice(0, i * N, (i + 1) * N)
                sc = None if t["sc"] is None else t["sc"].slice(0, i * N, (i + 1) * N)
                b = None if t["b"] is None else t["b"].slice(0, i * N, (i + 1) * N)
                y = empty((rows, N), dt)
                self._lin(y, xn, w, sc, b)
                halves.append(y)
            L.Ops.swiglu(out, halves[0], halves[1])
        return out.numpy(), xn.numpy(), None if h is None else h.numpy()


# (K, norm lanes / vectors the fused kernel takes): 1536 -> one wave x 3 vectors, 2048 ->
# one wave x 4, 3584 -> 256 lanes x 2, 12288 -> 256 lanes x 6 (8-vector registers);
# 512 (a 32-lane norm group) runs the composition.
FUSED_K = [1536, 2048, 3584, 12288, 512]


@pytest.mark.parametrize("swiglu", [False, True], ids=["plain", "swiglu"])
@pytest.mark.parametrize("int8", [False, True], ids=["dense", "int8"])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("K", FUSED_K)
def test_one_row_equals_separate_ops_bit_for_bit(K, dt, int8, swiglu):
    # N below 4096 keeps the separate INT8 linear on the one-row GEMV (same sum order)
    c = Case(1, K, 1000 if swiglu else 2056, dt, int8, swiglu, bias=True, res=True)
    got, h = c.fused()
    want, _, h_want = c.composed()
    assert_exact(h, h_want, f"residual K={K}")
    assert_exact(got, want, f"K={K} {dt} int8={int8} swiglu={swiglu}")


@pytest.mark.parametrize("swiglu", [False, True], ids=["plain", "swiglu"])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_int8_many_channels_equal_separate_ops_bit_for_bit(dt, swiglu):
    """INT8 weights over 4096+ channels: the separate linear takes the skinny MFMA kernel
    and so does the fused one (same K split, same order of the partials)."""
    c = Case(1, 1536, 4100 if not swiglu else 4104, dt, True, swiglu, bias=True, res=True, seed=11)
    got, h = c.fused()
    want, _, h_want = c.composed()
    assert_exact(h, h_want, "residual")
    assert_exact(got, want, f"INT8 N={c.N} {dt} swiglu={swiglu}")


@pytest.mark.parametrize("res", [False, True], ids=["norm", "add_norm"])
@pytest.mark.parametrize("bias", [False, True], ids=["nobias", "bias"])
def test_qwen2_decode_projections_against_oracle(res, bias):
    """Qwen2-1.5B's q/k/v ([2048, 1536], bias) and gate/up ([2 x 8960, 1536]) projections."""
    for N, swiglu, int8 in ((2048, False, False), (2048, False, True), (8960, True, False), (8960, True, True)):
        c = Case(1, 1536, N, "bf16", int8, swiglu, bias=bias, res=res, seed=3)
        got, h = c.fused()
        want, xn, h_want = c.composed()
        if res:
            hx = oracle.add(c.x, c.r)
            assert_exact(h, hx, "residual vs oracle add")
            assert_exact(h_want, hx, "composed residual vs oracle add")
        if not swiglu:
            if int8:
                ref = oracle.linear_w8a16(xn, c.w, c.sc, c.b)
                assert_linear_close(got, ref, xn, c.w, f"N={N} int8", w_scale=c.sc)
            else:
                assert_linear_close(got, oracle.linear(xn, c.w, c.b), xn, c.w, f"N={N}")
            assert_exact(got, want, f"N={N} int8={int8} vs separate ops")
        else:
            # gate / up from the oracle's linear of the normalised row, then oracle swiglu.  A
            # projection may round to a neighbouring bf16 value when the GPU's sum order
            # differs, so the bound is 2 ulps of the result plus one ulp (2^-7 relative) of
            # gate and of up carried through swiglu's partial derivatives (|d/dg| <= 1.1 |u|,
            # |d/du| = |silu(g)|)
            if int8:
                y = oracle.linear_w8a16(xn, c.w, c.sc, c.b)
            else:
                y = oracle.linear(xn, c.w, c.b)
            ref = to_f32(oracle.swiglu(y[:, :N], y[:, N:]), "bf16").astype(np.float64)
            gf, uf = (to_f32(y[:, :N], "bf16").astype(np.float64), to_f32(y[:, N:], "bf16").astype(np.float64))
            silu = gf / (1.0 + np.exp(-gf))
            tol = (2 * 2.0 ** -8 * np.abs(ref) + 1.1 * np.abs(uf) * 2.0 ** -7 * np.abs(gf)
                   + np.abs(silu) * 2.0 ** -7 * np.abs(uf))
            err = np.abs(to_f32(got, "bf16").astype(np.float64) - ref)
            assert np.all(err <= tol), f"N={N} int8={int8}: max err {err.max()}"
            assert_exact(got, want, f"N={N} int8={int8} swiglu vs separate ops")


@pytest.mark.parametrize("rows", [2, 5])
@pytest.mark.parametrize("swiglu", [False, True], ids=["plain", "swiglu"])
def test_several_rows_run_the_composition(rows, swiglu):
    c = Case(rows, 1536, 300, "bf16", False, swiglu, bias=True, res=True, seed=5)
    got, h = c.fused()
    want, _, h_want = c.composed()
    assert_exact(h, h_want, "residual")
    assert_exact(got, want, f"rows={rows}")


def test_f32_runs_the_composition():
    c = Case(1, 256, 40, "f32", False, True, bias=True, res=False, seed=8)
    got, _ = c.fused()
    want, _, _ = c.composed()
    assert_exact(got, want, "f32")


def test_ragged_channel_count_and_repeat():
    """N not a multiple of the 4 channels per block; two calls give the same bits."""
    c = Case(1, 1536, 1001, "bf16", True, False, bias=False, res=True, seed=9)
    a, _ = c.fused()
    b, _ = c.fused()
    want, _, _ = c.composed()
    assert_exact(a, b, "repeat")
    assert_exact(a, want, "ragged")


def test_graph_replays_of_the_decode_projections_match_eager():
    """The two fused decode projections (q/k/v with bias and add+norm; gate/up with swiglu,
    INT8, the skinny form) and the separate attention-output GEMV captured in one HIP graph
    and replayed three times, with eager work between replays: every replay equals the eager
    results (outputs cleared before each replay)."""
    api = L.RuntimeAPI(L.DeviceType.AMD)
    qkv = Case(1, 1536, 2048, "bf16", True, False, bias=True, res=True, seed=21)
    gu = Case(1, 1536, 8960, "bf16", True, True, bias=False, res=True, seed=22)
    outs = {"qkv": empty((1, 2048), "bf16"), "h1": empty((1, 1536), "bf16"),
            "act": empty((1, 8960), "bf16"), "h2": empty((1, 1536), "bf16")}

    def step():
        t = qkv.t
        L.Ops.rms_norm_linear(outs["qkv"], t["x"], t["nw"], EPS, t["w"], t["sc"], t["b"], residual=t["r"],
                              residual_out=outs["h1"])
        t = gu.t
        L.Ops.rms_norm_linear(outs["act"], outs["h1"], t["nw"], EPS, t["w"], t["sc"], residual=t["r"],
                              residual_out=outs["h2"], swiglu=True)

    step()
    eager = {k: v.numpy() for k, v in outs.items()}
    graph = L.Graph.capture()
    step()
    graph.end()
    for _ in range(3):
        for tt in outs.values():
            z = np.zeros(tt.shape(), dtype=np.uint16)
            api.memcpy_sync(tt.data_ptr(), z.ctypes.data, z.nbytes, L.MemcpyKind.H2D)
        gu.fused()  # unrelated eager work between replays
        graph.launch()
        api.device_synchronize()
        for k, v in outs.items():
            assert_exact(v.numpy(), eager[k], f"replay {k}")
