"""HIP-graph capture of a sequence of attention calls.

Launch overhead was a measured cost in the reference's block loop
(benchmark_log.md:100-104): every layer enqueues the prologue and the attention
kernel from Python.  `capture` records everything a callable enqueues on the
current stream into one HIP graph (torch.cuda.CUDAGraph is the HIP graph API
on ROCm), which `replay()` then submits with a single launch.

The libh3attn entry points are capture-safe: they enqueue kernels on the
caller's stream and nothing else (no allocation, no memset, no
synchronisation).  Outputs and any block-map buffers are allocated by torch
inside the capture, from the graph's private memory pool, and stay valid for
every replay.  The prologue works in place: a graph that contains it must be
given fresh q/k contents before each replay, exactly as a new layer input
would be.
"""
from __future__ import annotations

from typing import Callable


def capture(fn: Callable[[], object], warmup: int = 1, pool=None):
    """Run `fn` `warmup` times on a side stream, then capture one call of it.

    Returns (graph, result): `graph.replay()` re-runs the captured work;
    `result` is what the captured call returned (its tensors are the graph's
    static outputs, rewritten by every replay).
    """
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, pool=pool):
        result = fn()
    return graph, result


class LayerSequence:
    """N attention layers of the DiT on static buffers, replayable as one graph.

    Each layer is a dict with the fused QKV output `qkv` ([S, 3*H*D] bf16), the
    RoPE table `rope`, the norm weights `qw`, `kw`, and optionally `keep`
    (block-sparse keep ratio, with `blk`).  A layer runs the in-place prologue
    on the q/k views, then dense or block-sparse attention, and writes its O
    as [S, H*D].  `run()` does this eagerly; `capture()` records it once and
    `replay()` re-submits it.
    """

    def __init__(self, layers, heads: int, head_dim: int = 128, eps: float = 1e-6):
        self.layers = list(layers)
        self.H, self.D, self.eps = heads, head_dim, eps
        self.graph = None
        self.outputs = None

    def _layer(self, L):
        import torch

        from . import ops, sla

        qkv = L["qkv"]
        S = qkv.shape[0]
        H, D = self.H, self.D
        q = qkv[:, :H * D].view(1, S, H, D)
        k = qkv[:, H * D:2 * H * D].view(1, S, H, D)
        v = qkv[:, 2 * H * D:].view(1, S, H, D)
        rot = L["rope"].shape[-3] * 2
        ops.rms_rope_split_half_(q, k, L["rope"], L["qw"], L["kw"], epsilon=self.eps, rot_dim=rot)
        qh, kh, vh = (t.transpose(1, 2) for t in (q, k, v))
        keep = L.get("keep")
        if keep is None or keep >= 1.0:
            o = torch.empty(1, S, H, D, dtype=torch.bfloat16, device=qkv.device)
            ops.attn_fwd(qh, kh, vh, out=o.transpose(1, 2))
            return o.view(S, H * D)
        o = sla.sparse_attention(qh, kh, vh, keep, L.get("blk", 128), force_diag=L.get("force_diag", True))
        return o.transpose(1, 2).reshape(S, H * D)

    def run(self):
        """Eager execution of every layer; returns the list of [S, H*D] outputs."""
        return [self._layer(L) for L in self.layers]

    def capture(self, warmup: int = 1):
        self.graph, self.outputs = capture(self.run, warmup=warmup)
        return self.outputs

    def replay(self):
        if self.graph is None:
            raise RuntimeError("LayerSequence.replay() before capture()")
        self.graph.replay()
        return self.outputs
