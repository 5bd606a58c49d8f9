"""The allocation-free dense entry point h3a_attn_fwd_noalloc (no counterpart in the
reference; for callers that cannot allocate), called through the C ABI and checked
against h3a_attn_fwd_ws (the same kernels and split plan, with a workspace from torch's
allocator): equal bit for bit on two calls in a row, the second with a smaller input,
both with a split tail, so the second call runs over the first call's scratch contents,
and a third call at the first size again.  The smaller case is also checked against the
oracle at the attention tolerance.  The first call on a device sets the array up (the
runtime maps the library's device globals then); no later call may change the device's
free memory."""
from __future__ import annotations

import ctypes
import math

import pytest
import torch

import h3attn
import oracle
from conftest import assert_close_absmax, from_dev_bf16
from h3attn import _lib, ops

pytestmark = pytest.mark.gpu


def _bhs(t):
    return _lib.strides3(*(0 if t.shape[d] == 1 else t.stride(d) for d in range(3)))


def _noalloc(q, k, v, o):
    L = _lib.lib()
    B, H, Sq, D = q.shape
    stream = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
    rc = L.h3a_attn_fwd_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), B, H, Sq, k.shape[2], D,
                                _bhs(q), _bhs(k), _bhs(v), _bhs(o), 1.0 / math.sqrt(D), stream)
    _lib.check("h3a_attn_fwd_noalloc", rc)


def test_noalloc_first_call_under_graph_capture(gpu):
    """The process's first h3a_attn_fwd_noalloc call (no other test calls it before this one)
    is made inside a HIP graph capture, where it sets up the device's scratch address.  Every
    replay equals h3a_attn_fwd_ws bit for bit, with eager no-alloc calls on other inputs, which
    overwrite the scratch, between the replays.  One captured case has a split tail, the other
    queued dispatch."""
    ins, want = [], []
    for H, S, seed in ((4, 2048, 11), (56, 8192, 12)):
        print(f"[noalloc graph] H={H} S={S}", flush=True)
        g = torch.Generator(device=gpu).manual_seed(seed)
        q, k, v = (torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
        ins.append((q, k, v))
        want.append(h3attn.attn_fwd(q, k, v, split_tail=True))  # h3a_attn_fwd_ws
    outs = [torch.full_like(q, float("nan")) for q, _, _ in ins]
    g = torch.Generator(device=gpu).manual_seed(13)
    other = [torch.randn(1, 8, 3000, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3)]
    other_out = torch.empty_like(other[0])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for (q, k, v), o in zip(ins, outs):
            _noalloc(q, k, v, o)
    torch.cuda.synchronize()
    for r in range(3):
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for o, w, (q, _, _) in zip(outs, want, ins):
            assert torch.equal(o, w), f"replay {r}, H={q.shape[1]}: differs from h3a_attn_fwd_ws"
        _noalloc(*other, other_out)
        torch.cuda.synchronize()
    assert torch.equal(other_out, h3attn.attn_fwd(*other, split_tail=True))


def test_noalloc_matches_workspace_entry_point(gpu):
    for i, (H, S, seed) in enumerate(((56, 42120, 1), (4, 2048, 2), (56, 42120, 3))):
        print(f"[noalloc] H={H} S={S}", flush=True)
        g = torch.Generator(device=gpu).manual_seed(seed)
        q, k, v = (torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
        nbytes = ops.attn_workspace_bytes(1, H, S, S)
        assert 0 < nbytes <= 34079744, nbytes  # the split tail runs, within the static array
        want = h3attn.attn_fwd(q, k, v, split_tail=True)  # h3a_attn_fwd_ws
        got = torch.full_like(q, float("nan"))
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info(gpu)[0]
        _noalloc(q, k, v, got)
        torch.cuda.synchronize()
        if i > 0:
            assert torch.cuda.mem_get_info(gpu)[0] == free0, "the call changed the device's free memory"
        assert torch.equal(got, want), f"H={H} S={S}: differs from h3a_attn_fwd_ws"
        if H == 4:
            ref = oracle.attn_fwd(from_dev_bf16(q), from_dev_bf16(k), from_dev_bf16(v))
            assert_close_absmax(got.float().cpu().numpy(), ref, what="noalloc vs oracle")


def test_noalloc_rejects_bad_arguments(gpu):
    L = _lib.lib()
    z = _lib.strides3(0, 0, 0)
    assert L.h3a_attn_fwd_noalloc(None, 16, 16, 16, 1, 1, 4, 4, 128, z, z, z, z, 0.1, None) == _lib.H3A_ERR_INVALID_ARG
    assert L.h3a_attn_fwd_noalloc(16, 16, 16, 16, 1, 1, 4, 4, 64, z, z, z, z, 0.1, None) == _lib.H3A_ERR_UNSUPPORTED
