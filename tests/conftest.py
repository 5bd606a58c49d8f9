"""Shared pytest setup: import paths, the `gpu` marker, seeded inputs, tolerances.

GPU tests are marked @pytest.mark.gpu and run only on an MI355X box
(`pytest -m gpu`); everything else runs on the CPU (`pytest -m "not gpu"`).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "minimaxh3-on-a100-x4_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE):
    if p not in sys.path:
        sys.path.insert(0, p)

# Tolerance for floating-point attention outputs, relative to the
# reference's absolute maximum: max |o - ref| <= 1e-2 * absmax(ref) and
# mean |o - ref| <= 1e-3 * absmax(ref).
MAX_REL = 1e-2
MEAN_REL = 1e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct MI355X (gfx950) GPU")


def assert_close_absmax(out, ref, max_rel=MAX_REL, mean_rel=MEAN_REL, what=""):
    """Attention tolerance check on float arrays/tensors; returns (max_err, mean_err, absmax)."""
    o = np.asarray(out, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    assert o.shape == r.shape, f"{what}: shape {o.shape} vs {r.shape}"
    assert np.isfinite(o).all(), f"{what}: non-finite output"
    err = np.abs(o - r)
    amax = float(np.abs(r).max()) if r.size else 0.0
    mx, mean = float(err.max()) if err.size else 0.0, float(err.mean()) if err.size else 0.0
    scale = max(amax, 1e-30)
    assert mx <= max_rel * scale, f"{what}: max_abs_err {mx:.3e} > {max_rel}*absmax ({amax:.3e})"
    assert mean <= mean_rel * scale, f"{what}: mean_abs_err {mean:.3e} > {mean_rel}*absmax ({amax:.3e})"
    return mx, mean, amax


def assert_prologue_close(got_bits, ref_bits, what, min_exact=0.99):
    """Prologue output (kernel, fp32 math) vs the oracle (fp64 math), both rounded once to bf16.

    Allowed per value: one bf16 ulp of the result (<= 2^-7 |r|) plus the fp32
    error of the rotation before rounding, ~1e-6 * (|y_i| + |y_{i+rot/2}|)
    with |y| <= ~8 here, taken as an absolute 1e-5.  The second term only
    matters where the rotation cancels to a value near zero.  At least
    `min_exact` of the values must be bit-identical.
    """
    import oracle
    g = oracle.bf16_to_f32(got_bits).reshape(got_bits.shape).astype(np.float64)
    r = oracle.bf16_to_f32(ref_bits).reshape(ref_bits.shape).astype(np.float64)
    exact = np.mean(got_bits == ref_bits)
    tol = np.abs(r) * 2.0 ** -7 + 1e-5
    bad = np.abs(g - r) > tol
    if bad.any():
        i = np.unravel_index(np.argmax(np.abs(g - r) - tol), r.shape)
        raise AssertionError(f"{what}: {int(bad.sum())} values off by more than 1 ulp + 1e-5; "
                             f"worst at {i}: got {g[i]!r} want {r[i]!r}")
    assert exact >= min_exact, f"{what}: only {exact:.4f} bit-exact"


def bf16_bits(x_f32: np.ndarray) -> np.ndarray:
    import oracle
    return oracle.f32_to_bf16(x_f32)


def randn_bf16(rng: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    """Seeded N(0, scale^2) values rounded to bf16, as uint16 bit patterns."""
    return bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))


def ramp_case(rng: np.random.Generator, S: int, slope: float, q0: float, H: int = 2):
    """Scores that move steadily along the keys: dim 0 of key j is slope*j and dim 0
    of the queries is +q0 (even rows: scores rise along the keys) or -q0 (odd rows:
    they fall), the other dims small noise.  Returns q, k, v as bf16 bits."""
    q = rng.standard_normal((1, H, S, 128)).astype(np.float32) * 0.1
    k = rng.standard_normal((1, H, S, 128)).astype(np.float32) * 0.1
    v = rng.standard_normal((1, H, S, 128)).astype(np.float32)
    q[..., 0] = np.where(np.arange(S) % 2 == 0, q0, -q0)
    k[..., 0] = slope * np.arange(S)
    return tuple(bf16_bits(x) for x in (q, k, v))


@pytest.fixture(scope="session")
def gpu():
    """The MI355X device; fails loudly when absent (GPU tests must not silently skip)."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch.device("cuda:0")


def to_dev_bf16(bits: np.ndarray, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)
    return t.to(device)


def from_dev_bf16(t) -> np.ndarray:
    import torch
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
