"""Host checks of the backend's own device math (technograd_amd/csrc/tg_devmath.h),
built with g++ from the same header the kernels include."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("stride", [97])
def test_log1p_unit_correctly_rounded(tmp_path, stride):
    """softplus's log1pf: every 97th f32 in [0, 1] (11 M values) equals the
    correctly rounded log1p (the f32 rounding of the C library's f64 log1p),
    and is within 1 ulp of the reference's glibc log1pf. NaN stays NaN,
    log1p(0) = +0, log1p(1) = ln 2 rounded. (Run over all 1.07 G values, the
    routine differs from the correctly rounded value once, at a rounding
    boundary.)"""
    exe = tmp_path / "l1p"
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-I", os.path.join(ROOT, "technograd_amd", "csrc"), "-o", str(exe),
                    os.path.join(ROOT, "tests", "cpp", "log1p_unit_check.cpp")], check=True)
    out = subprocess.run([str(exe), str(stride)], check=True, capture_output=True, text=True).stdout.split()
    n, off_cr, off_lib, worst, nan_ok, zero_ok, l2_ok = (int(v) for v in out)
    assert n > 10_000_000
    assert off_cr == 0
    assert worst <= 1
    assert off_lib < n // 100  # glibc 2.35's log1pf is within 1 ulp, not correctly rounded
    assert nan_ok and zero_ok and l2_ok
