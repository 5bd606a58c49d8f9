"""The phase profiler (counterpart of the reference's -DPROFILE build, get_prof and
reset_prof, attn_sm80/fa3_sm80_h3.cu:96-105, 213-239, 572-582).

One launch that fits a single round of workgroups (B=1, H=2, S=32768: 256 query tiles
of 256 rows, one per CU) through the profile build.  Workgroup 0's per-wave phase
ticks must be non-zero, tile its stage loop exactly and count its stages; its loop
time in the constant 100 MHz clock must fit inside the HIP-event time of the whole
launch (with 2 % for the clocks' skew).  How much of the launch the loop fills and the
implied shader clock vary by box under the power limit, so they are printed only.  The
profile build's output must equal the product build's bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import attn_sm80
import h3attn
from h3attn import ops

pytestmark = pytest.mark.gpu


def test_product_build_records_nothing(gpu):
    assert not ops.prof_enabled(profile=False)
    ext = attn_sm80._build()
    assert torch.equal(ext.get_prof(), torch.zeros(5, dtype=torch.float64))


def test_profile_build_phases_add_up(gpu):
    assert ops.prof_enabled(profile=True)
    B, H, S = 1, 2, 32768
    g = torch.Generator(device=gpu).manual_seed(4)
    q, k, v = (torch.randn(B, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    ext = attn_sm80._build(profile=True)
    O = torch.empty_like(q)
    ext.fa3(q, k, v, O)  # warm-up
    ext.reset_prof()
    assert all(x == 0 for row in ops.prof_read() for x in row)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    ext.fa3(q, k, v, O)
    e1.record()
    torch.cuda.synchronize()
    launch_ms = e0.elapsed_time(e1)
    rows = np.array(ops.prof_read(), dtype=np.int64)
    stages = -(-S // 64)
    for w, r in enumerate(rows):
        assert r[6] == stages, f"wave {w}: {r[6]} stages"
        assert (r[:6] > 0).all(), f"wave {w}: a phase is empty: {r[:6]}"
        assert r[:6].sum() == r[7], f"wave {w}: phases do not tile the loop"
        assert r[9] > 0 and r[10] > 0
        # A wave's loop runs inside the launch (2 % for the two clocks' skew).  How much of
        # the launch it fills, and the shader clock, depend on the box: printed, not checked.
        loop_ms = r[8] / 1e5  # 100 MHz ticks
        assert 0 < loop_ms <= 1.02 * launch_ms, (w, loop_ms, launch_ms)
        # the matrix cluster is 32 MFMAs of >= 32 cycles each per stage
        mfma_phase = r[1] if w < 4 else r[3]
        assert mfma_phase >= 0.8 * 1024 * stages, (w, mfma_phase)
    prof = ext.get_prof()
    w0 = rows[0]
    assert prof.tolist() == [float(w0[0] + w0[2] + w0[4] + w0[5]), float(w0[1]), float(w0[3]), 0.0,
                             float(w0[9])]
    print(f"[profile] launch {launch_ms:.3f} ms, wave 0 loop {w0[8] / 1e5:.3f} ms, "
          f"{w0[7] / (w0[8] * 10.0):.2f} GHz; per stage (ticks): "
          + ", ".join(f"{x / stages:.0f}" for x in w0[:6]))
    # same arithmetic as the product build
    want = h3attn.attn_fwd(q, k, v, split_tail=False)
    torch.cuda.synchronize()
    assert torch.equal(O, want)
