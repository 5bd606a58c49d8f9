"""The block-sparse kernels' LUT arithmetic (csrc/h3a_lut.h), compiled for the host and
checked against int64 math: the key block of a stage (t / sub, with sub = 3 as a
multiply-high) and a stage's first key, including LUT entries far outside the key
range (2^24 + 5, 2^31 - 1, negative), which must map to Skv (load nothing) instead
of wrapping a 32-bit multiply.  No GPU needed."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import PKG, ROOT


def test_lut_arithmetic_on_host(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.fail("g++ not found")
    exe = tmp_path / "lut_check"
    subprocess.run([cxx, "-std=c++17", "-O2", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    f"-I{os.path.join(PKG, 'csrc')}", os.path.join(ROOT, "tests", "lut_arith_check.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "OK", r.stdout + r.stderr
