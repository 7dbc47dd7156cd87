"""The RoPE kernels' double-precision sincos, checked on the host against glibc.

sincos.hpp is plain C++ (fma, rint) and compiles for the host unchanged, so its results
here are the ones the GPU computes (IEEE double fma and rounding are the same on both).
glibc's sin/cos are what the reference rope calls (src/ops/rope/cpu/rope_cpu.cpp:33-34).
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNELS = os.path.join(ROOT, "llaisys_amd", "csrc", "kernels")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("sincos") / "sincos_check"
    subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-I", KERNELS,
                    os.path.join(ROOT, "tests", "sincos_check.cc"), "-o", str(exe)], check=True)
    return exe


def test_sincos_within_one_ulp_of_glibc(checker):
    out = subprocess.run([str(checker), "16384"], check=True, capture_output=True, text=True)
    angles, differ, max_ulp, f32_differ = map(int, out.stdout.split())
    assert angles == 3 * 64 * 16384 + 200000
    assert max_ulp <= 1, out.stdout
    # an ulp in cos / sin never moved a rotated pair's float result in this sample
    assert f32_differ == 0, out.stdout
    # the comparison is live: a fraction of the angles differ by that ulp
    assert 0 < differ < angles // 2
