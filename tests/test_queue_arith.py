"""The ping-pong kernels' work distribution (csrc/h3a_queue.h), compiled for the host:
xcd_remap is a bijection whose per-XCD ranges are exactly the per-XCD queue shares,
every work item sits in exactly one queue (whole tiles before split pieces), a
workgroup drains its own XCD's queue before it steals, and concurrent takers (threads
over relaxed atomic counters) hand out every item exactly once and return -1 only
after all are claimed.  No GPU needed."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import PKG, ROOT


def test_queue_arithmetic_on_host(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.fail("g++ not found")
    exe = tmp_path / "queue_check"
    subprocess.run([cxx, "-std=c++17", "-O2", "-pthread", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    f"-I{os.path.join(PKG, 'csrc')}", os.path.join(ROOT, "tests", "queue_check.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip() == "OK", r.stdout + r.stderr
