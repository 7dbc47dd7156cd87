"""The division-free INT8 code of the quantize / KV-append kernels, checked on the host.

quantize.hpp computes q = rint(x / s) without a division: q0 = x * RN(1/s), one fma for
the residual, one for the correction (Markstein's final division step), and rint through
an add of 1.5 * 2^23.  This checks that arithmetic identity against IEEE division,
exhaustively for bf16 and f16 data and on random / near-tie f32 pairs; the GPU tests then
compare the kernels' codes with the oracle bit for bit.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_division_free_code_equals_ieee_code(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "quant_quotient_check"
    subprocess.run([gcc, "-O2", "-std=c11", "-ffp-contract=off", "-fopenmp",
                    os.path.join(ROOT, "tests", "quant_quotient_check.c"), "-o", str(exe), "-lm"],
                   check=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([str(exe), "20000000"], check=True, capture_output=True, text=True,
                         env=env, timeout=600)
    pairs, bad = map(int, out.stdout.split())
    assert pairs > 2_000_000_000 + 10_000_000
    assert bad == 0, out.stdout
