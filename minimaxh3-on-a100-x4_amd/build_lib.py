"""Build libh3attn.so (gfx950) in-tree from csrc/*.hip with hipcc.

Usage: python build_lib.py [--verbose] [--profile] [-DKNOB=VALUE ...] [--out=PATH]
  --profile builds the phase-profile library h3attn/libh3attn_prof.so as well.

The library lands next to the Python package (h3attn/libh3attn.so) so it
travels with the source tree.  Every call rebuilds: compile each translation
unit in parallel, then link.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT_DIR = os.path.join(HERE, "h3attn")
LIB_NAME = "libh3attn.so"
# The phase-profile build (H3A_PROFILE=1) of the same sources.
PROF_LIB_OUT = os.path.join(OUT_DIR, "libh3attn_prof.so")
BUILD_DIR = os.path.join(HERE, "_build")

ARCH = "gfx950"
# Packed-FP32 VALU ops are disabled for all device code.
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # No kernel relies on NaN semantics; without this, every fmaxf is preceded
    # by a NaN-canonicalising v_max_f32 in IEEE mode.
    "-fno-honor-nans",
    "-Wall", "-Wno-unused-function", f"-I{INCLUDE}", f"-I{CSRC}",
]


def _hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found; ROCm is required to build libh3attn")
    return p


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    noise = [ln for ln in r.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln
             and "is not a recognized feature" not in ln and not ln.startswith("1 warning")]
    if verbose and noise:
        print("\n".join(noise), flush=True)
    return r


def build(verbose: bool = False, defines=(), out: str | None = None) -> str:
    """Compile and link; `defines` are extra -D tuning knobs, `out` an alternative .so path."""
    hipcc = _hipcc()
    tag = "_".join(d.replace("=", "") for d in defines)
    bdir = os.path.join(BUILD_DIR, tag) if tag else BUILD_DIR
    os.makedirs(bdir, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = []
    cmds = []
    for s in srcs:
        obj = os.path.join(bdir, s[:-4] + ".o")
        objs.append(obj)
        cmds.append([hipcc, *CFLAGS, *[f"-D{d}" for d in defines], "-c", os.path.join(CSRC, s), "-o", obj])
    workers = min(len(cmds), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    final = out or os.path.join(OUT_DIR, LIB_NAME)
    tmp = final + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, final)
    return final


if __name__ == "__main__":
    args = sys.argv[1:]
    defs = [a[2:] for a in args if a.startswith("-D")]
    outp = next((a.split("=", 1)[1] for a in args if a.startswith("--out=")), None)
    print(build(verbose="--verbose" in args, defines=defs, out=outp))
    if "--profile" in args:
        print(build(verbose="--verbose" in args, defines=defs + ["H3A_PROFILE=1"], out=PROF_LIB_OUT))
