"""HIP-graph capture of attention layers and per-component timing on the GPU.

A graph of several DiT attention layers (in-place prologue on the fused QKV
output, then dense or block-sparse attention writing [S, H*D]) is replayed
several times, with eager work in between, and every replay must equal the
eager run bit for bit: the captured kernels are the same kernels on the same
inputs.  (benchmark_log.md:100-104 motivates the capture; the timing names
follow custom_nodes/h3_profiler/__init__.py:98-115.)
"""
from __future__ import annotations

import pytest
import torch

import h3attn
import standin_dit
from h3attn import graphs, hooks, ops, profiling

pytestmark = pytest.mark.gpu


def _layers(gpu, S=700, H=4, n=3, seed=31):
    g = torch.Generator(device=gpu).manual_seed(seed)
    rope = h3attn.rope_freqs(S, 128, device=gpu)
    layers, pristine = [], []
    for i in range(n):
        qkv = torch.randn(S, 3 * H * 128, generator=g, device=gpu).to(torch.bfloat16)
        qw = (1 + 0.05 * torch.randn(128, generator=g, device=gpu)).to(torch.bfloat16)
        kw = (1 + 0.05 * torch.randn(128, generator=g, device=gpu)).to(torch.bfloat16)
        L = {"qkv": qkv, "rope": rope, "qw": qw, "kw": kw}
        if i == n - 1:
            L.update(keep=0.5, blk=128)  # one block-sparse layer
        layers.append(L)
        pristine.append(qkv.clone())
    return layers, pristine


def _restore(layers, pristine):
    for L, p in zip(layers, pristine):
        L["qkv"].copy_(p)


def test_graph_replay_matches_eager(gpu):
    layers, pristine = _layers(gpu)
    seq = graphs.LayerSequence(layers, heads=4)
    want = [o.clone() for o in seq.run()]
    _restore(layers, pristine)
    outs = seq.capture(warmup=1)
    other = torch.randn(1, 2, 300, 128, device=gpu, dtype=torch.bfloat16)
    for r in range(3):
        _restore(layers, pristine)  # the prologue works in place: fresh inputs per replay
        h3attn.attn_fwd(other, other, other)  # unrelated eager work between replays
        torch.cuda.synchronize()
        seq.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o, w), f"replay {r}, layer {i} differs from the eager run"


@pytest.mark.parametrize("nk", [700, 1300, 2000])
def test_graph_capture_of_wide_block_select(gpu, nk):
    """Block select over long rows: 700 key blocks (44 score tiles per row, 14 query blocks
    per 4-wave workgroup, keys counted in 12 registers per lane), 1300 (8-wave workgroups
    over static LDS, 15 query blocks each, 2 rows per wave in 24 registers) and 2000 (the
    16-wave workgroup, 16 query blocks, 48 registers per lane): captured into a graph,
    every replay equals the eager call."""
    g = torch.Generator(device=gpu).manual_seed(41)
    pq = torch.randn(1, 2, 20, 128, generator=g, device=gpu)
    pk = torch.randn(1, 2, nk, 128, generator=g, device=gpu)
    keep = nk // 4
    want = [t.clone() for t in ops.block_select(pq, pk, keep, 64, 64)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.block_select(pq, pk, keep, 64, 64)  # warm-up off the default stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = ops.block_select(pq, pk, keep, 64, 64)
    other = torch.randn(1, 2, 300, 128, device=gpu, dtype=torch.bfloat16)
    for r in range(3):
        h3attn.attn_fwd(other, other, other)  # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, o, w in zip(("map", "lut", "counts"), outs, want):
            assert torch.equal(o, w), f"replay {r}: {name} differs from the eager call"


def test_graph_replay_of_queued_launches(gpu):
    """Launches of at least four rounds of work items run on the persistent grid fed by
    the per-XCD queues, whose counters a kernel zeroes before each launch, and here also
    split their last round (H=9, S=32768: 1152 tiles, and 1152 pairs of 128-row blocks).
    Dense and block-sparse attention captured in one graph: every replay, with eager
    work and cleared outputs in between, equals the eager calls bit for bit."""
    g = torch.Generator(device=gpu).manual_seed(43)
    B, H, S = 1, 9, 32768
    q, k, v = (torch.randn(B, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    nq = S // 128
    bmap = torch.rand(B, H, nq, nq, generator=g, device=gpu) < 0.25
    diag = torch.arange(nq, device=gpu)
    bmap[..., diag, diag] = True
    lut, cnt = h3attn.block_map_to_lut(bmap.to(torch.uint8))
    partials = 128 * 2 * 256 * 130 * 4  # 128 last-round items, two key ranges each
    assert ops.attn_workspace_bytes(B, H, S, S) >= partials + 1024
    assert ops.sparse_workspace_bytes(B, H, S, S, 128, 128, lut.shape[3]) >= partials + 1024

    def fn():
        return h3attn.attn_fwd(q, k, v), h3attn.attn_fwd_blocksparse(q, k, v, lut, cnt, 128, 128)

    want = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    graph, outs = graphs.capture(fn, warmup=1)
    other = torch.randn(1, 2, 300, 128, device=gpu, dtype=torch.bfloat16)
    for r in range(3):
        h3attn.attn_fwd(other, other, other)  # unrelated eager work between replays
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, o, w in zip(("dense", "sparse"), outs, want):
            assert torch.equal(o, w), f"replay {r}: {name} differs from the eager call"


def test_graph_replay_of_key_split_and_tile_launches(gpu):
    """The 64-row key-split pairs (64x64 blocks) and the tile path (96x96 blocks over 64x64
    tiles) at H=9, S=32768, both through the queued entry points (a kernel zeroes the
    counters before each launch): captured in one graph, every replay, with eager work and
    cleared outputs in between, equals the eager calls bit for bit."""
    g = torch.Generator(device=gpu).manual_seed(44)
    B, H, S = 1, 9, 32768
    q, k, v = (torch.randn(B, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    maps = {}
    for blk in (64, 96):
        nb = -(-S // blk)
        m = torch.rand(B, H, nb, nb, generator=g, device=gpu) < 0.25
        d = torch.arange(nb, device=gpu)
        m[..., d, d] = True
        maps[blk] = m.to(torch.uint8)
    lut, cnt = h3attn.block_map_to_lut(maps[64])
    tl, tc = ops.block_map_to_tile_lut(maps[96], 96, 96, S, S)
    assert ops.sparse_workspace_bytes(B, H, S, S, 64, 64, lut.shape[3]) > 0  # queued
    assert ops.tiles_workspace_bytes(B, H, S, S, tl.shape[3]) > 8 * B * H * (S // 64 // 2)  # map + queues

    def fn():
        return (h3attn.attn_fwd_blocksparse(q, k, v, lut, cnt, 64, 64),
                ops.attn_fwd_blocksparse_tiles(q, k, v, tl, tc, queues=True))

    want = [t.clone() for t in fn()]
    torch.cuda.synchronize()
    graph, outs = graphs.capture(fn, warmup=1)
    other = torch.randn(1, 2, 300, 128, device=gpu, dtype=torch.bfloat16)
    for r in range(3):
        h3attn.attn_fwd(other, other, other)  # unrelated eager work between replays
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, o, w in zip(("64x64 key-split", "96x96 tiles"), outs, want):
            assert torch.equal(o, w), f"replay {r}: {name} differs from the eager call"


def test_graph_capture_requires_capture_before_replay(gpu):
    layers, _ = _layers(gpu, n=1)
    with pytest.raises(RuntimeError):
        graphs.LayerSequence(layers, heads=4).replay()


def test_timer_on_patched_forward(gpu):
    class A(standin_dit.Attention):
        pass

    torch.manual_seed(0)
    m = A(512, 4, dtype=torch.bfloat16, device=gpu)
    with torch.no_grad():
        m.qkv_proj.weight.normal_(0, 512 ** -0.5)
        m.out_proj.weight.normal_(0, 512 ** -0.5)
    x = torch.randn(800, 512, device=gpu, dtype=torch.bfloat16)
    rope = h3attn.rope_freqs(800, 128, device=gpu)
    timer = profiling.OpTimer()
    with torch.no_grad():
        assert hooks.install(A, timer=timer)
        try:
            timer.arm()
            for _ in range(2):
                m(x, rope_freqs=rope)
            timer.disarm()
        finally:
            hooks.uninstall(A)
    rep = timer.report()
    assert rep["calls"] == {c: 2 for c in profiling.COMPONENTS}
    assert all(v > 0 for v in rep["components_ms"].values())
