"""The attention kernels' stale-max refresh predicate (csrc/h3a_stale.h), compiled for the
host with the library's own -fno-honor-nans (clang) and with gcc's -ffinite-math-only:
a stage sum above 2^16, +inf or NaN must ask for a refresh under both, finite sums up
to 2^16 must not.  No GPU needed."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import PKG, ROOT

COMPILERS = [("clang", "/opt/rocm/llvm/bin/clang++", ["-fno-honor-nans"]),
             ("gcc", shutil.which("g++") or "g++", ["-ffinite-math-only"])]


@pytest.mark.parametrize("name,cxx,flags", COMPILERS, ids=[c[0] for c in COMPILERS])
def test_stale_sum_predicate_on_host(tmp_path, name, cxx, flags):
    if not os.path.exists(cxx) and shutil.which(cxx) is None:
        pytest.fail(f"{cxx} not found")
    exe = tmp_path / f"stale_{name}"
    subprocess.run([cxx, "-std=c++20", "-O3", *flags, "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    f"-I{os.path.join(PKG, 'csrc')}", os.path.join(ROOT, "tests", "stale_sum_check.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "OK", r.stdout + r.stderr
