"""The split-tail dense path (h3a_attn_fwd_ws): the query tiles of the last,
partly filled round of workgroups are cut into key ranges whose partial
results (unnormalised O, reference max, row sum) are merged by a second
kernel.  Results must match the oracle, and the unsplit kernel
(h3a_attn_fwd), at the attention tolerance.  The merge is exact algebra of
the online softmax; only P's bf16 rounding sees a different reference max.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import h3attn
import oracle
from conftest import assert_close_absmax, from_dev_bf16, randn_bf16, to_dev_bf16
from h3attn import ops

pytestmark = pytest.mark.gpu


def _cus():
    return torch.cuda.get_device_properties(0).multi_processor_count


@pytest.mark.parametrize("B,H,Sq,Skv", [(1, 2, 1000, 1000), (1, 3, 4104, 4104), (2, 1, 500, 3000),
                                        (1, 1, 64, 2000), (1, 4, 2048, 2048)])
def test_split_matches_oracle_and_unsplit(gpu, B, H, Sq, Skv):
    rng = np.random.default_rng(Sq + Skv + H)
    q = randn_bf16(rng, (B, H, Sq, 128))
    k, v = randn_bf16(rng, (B, H, Skv, 128)), randn_bf16(rng, (B, H, Skv, 128))
    assert ops.attn_workspace_bytes(B, H, Sq, Skv) > 0, "this shape is meant to exercise the split"
    qd, kd, vd = (to_dev_bf16(x, gpu) for x in (q, k, v))
    o_split = ops.attn_fwd(qd, kd, vd)
    o_whole = ops.attn_fwd(qd, kd, vd, split_tail=False)
    got = oracle.bf16_to_f32(from_dev_bf16(o_split)).reshape(o_split.shape)
    assert_close_absmax(got, oracle.attn_fwd(q, k, v), what=f"split {B}x{H}x{Sq}x{Skv} vs oracle")
    whole = oracle.bf16_to_f32(from_dev_bf16(o_whole)).reshape(o_whole.shape)
    # up to rounding: P's bf16 rounding sees each piece's own reference max
    assert_close_absmax(got, whole, what="split vs unsplit")


def test_no_split_when_rounds_are_full(gpu):
    """A problem whose tiles fill every round exactly needs no workspace."""
    H = _cus()  # one 256-row tile per head, one round
    assert ops.attn_workspace_bytes(1, H, 256, 4096) == 0
    assert ops.attn_workspace_bytes(1, 1, 300, 200) == 0  # 4 stages: too short to split


def test_workspace_too_small_is_an_error(gpu):
    q = torch.randn(1, 2, 1000, 128, device=gpu, dtype=torch.bfloat16)
    need = ops.attn_workspace_bytes(1, 2, 1000, 1000)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    o = torch.empty_like(q)
    L = h3attn._lib.lib()
    S3 = h3attn._lib.strides3
    st = S3(*q.stride()[:3])
    args = (q.data_ptr(), q.data_ptr(), q.data_ptr(), o.data_ptr(), 1, 2, 1000, 1000, 128, st, st, st, st, 0.088)
    assert L.h3a_attn_fwd_ws(*args, ws.data_ptr(), need - 1, None) == h3attn._lib.H3A_ERR_INVALID_ARG
    assert b"workspace" in L.h3a_last_error()
    assert L.h3a_attn_fwd_ws(*args, None, 0, None) == h3attn._lib.H3A_ERR_INVALID_ARG
    assert L.h3a_attn_fwd_ws(*args, ws.data_ptr(), need, None) == 0
    torch.cuda.synchronize()


def test_split_full_h3_shape_matches_unsplit(gpu):
    """H=56, S=42120: the tiles of the last round are split; every output row
    must match the unsplit kernel up to rounding."""
    S, H = 42120, 56
    g = torch.Generator(device=gpu).manual_seed(11)
    q, k = (torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(2))
    v = torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) * 4
    assert ops.attn_workspace_bytes(1, H, S, S) > 0
    o_split = ops.attn_fwd(q, k, v)
    o_whole = ops.attn_fwd(q, k, v, split_tail=False)
    torch.cuda.synchronize()
    d = (o_split.float() - o_whole.float()).abs()
    ref = o_whole.float().abs().max().item()
    assert d.max().item() <= 1e-2 * ref and d.mean().item() <= 1e-4 * ref
    # the split tiles are the last ones of the last head: they must be the only ones that differ
    assert torch.equal(o_split[0, :H - 1], o_whole[0, :H - 1])


def _ws_call(q, k, v, o, ws):
    L = h3attn._lib.lib()
    S3 = h3attn._lib.strides3
    B, H, Sq, D = q.shape
    st = [S3(*t.stride()[:3]) for t in (q, k, v, o)]
    stream = h3attn.ops._stream(q)
    rc = L.h3a_attn_fwd_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq, k.shape[2], D,
                           *st, 1.0 / np.sqrt(D), ws.data_ptr(), ws.numel(), stream)
    h3attn._lib.check("h3a_attn_fwd_ws", rc)


def test_queued_dispatch_matches_one_tile_per_workgroup(gpu):
    """Four rounds of tiles and more run on a persistent grid that takes tiles from per-XCD
    queues (1 KiB of counters in the workspace).  Each tile's arithmetic is that of the
    one-workgroup-per-tile launch, so without a split tail the outputs are equal bit for
    bit, also when the workspace starts out holding garbage (the call clears the counters),
    and on a second call over the first call's counters."""
    cus = _cus()
    B, H, Sq, Skv = 4, max(cus // 4, 1), 1024, 640  # 4 tiles per head: 4 * CUs tiles, no remainder
    assert ops.attn_workspace_bytes(B, H, Sq, Skv) == 1024
    g = torch.Generator(device=gpu).manual_seed(5)
    q, k, v = (torch.randn(B, H, n, 128, generator=g, device=gpu, dtype=torch.bfloat16)
               for n in (Sq, Skv, Skv))
    want = ops.attn_fwd(q, k, v, split_tail=False)  # h3a_attn_fwd: one workgroup per tile
    ws = torch.full((1024,), 0x7F, dtype=torch.uint8, device=gpu)
    for call in range(2):
        got = torch.full_like(q, float("nan"))
        _ws_call(q, k, v, got, ws)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {call}: queued dispatch differs from one tile per workgroup"


def test_queued_dispatch_with_split_tail(gpu):
    """Queues and a split tail together: the whole tiles match the unsplit kernel bit for
    bit, the split ones (the last two heads) match it and the oracle at the attention
    tolerance."""
    cus = _cus()
    H, Sq, Skv = cus // 4 + 2, 4000, 1024  # 16 tiles per head: 4 * CUs + 32 tiles
    nbytes = ops.attn_workspace_bytes(1, H, Sq, Skv)
    assert nbytes > 1024, "meant to split and queue"
    rng = np.random.default_rng(17)
    q = randn_bf16(rng, (1, H, Sq, 128))
    k, v = randn_bf16(rng, (1, H, Skv, 128)), randn_bf16(rng, (1, H, Skv, 128))
    qd, kd, vd = (to_dev_bf16(x, gpu) for x in (q, k, v))
    o_split = ops.attn_fwd(qd, kd, vd)
    o_whole = ops.attn_fwd(qd, kd, vd, split_tail=False)
    torch.cuda.synchronize()
    assert torch.equal(o_split[0, :H - 2], o_whole[0, :H - 2])
    got = oracle.bf16_to_f32(from_dev_bf16(o_split[:, H - 2:].contiguous())).reshape(1, 2, Sq, 128)
    assert_close_absmax(got, oracle.attn_fwd(q[:, H - 2:], k[:, H - 2:], v[:, H - 2:]),
                        what="queued split heads vs oracle")
    whole = oracle.bf16_to_f32(from_dev_bf16(o_whole[:, H - 2:].contiguous())).reshape(1, 2, Sq, 128)
    assert_close_absmax(got, whole, what="queued split vs unsplit")
