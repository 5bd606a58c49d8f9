"""The drop-in hooks on the GPU: the patched Attention.forward (HIP prologue in
place on the fused QKV output + HIP attention writing [S,H*D]) and the patched
optimized_attention must reproduce the stock forward (custom_nodes/h3_profiler/
__init__.py:92-111, restated in tests/standin_dit.py) on the same module."""
from __future__ import annotations

import pytest
import torch

import h3attn
import standin_dit
from conftest import assert_close_absmax
from h3attn import hooks

pytestmark = pytest.mark.gpu


def _module(cls, gpu, dim=512, heads=4, seed=0):
    torch.manual_seed(seed)
    m = cls(dim, heads, dtype=torch.bfloat16, device=gpu)
    with torch.no_grad():
        m.qkv_proj.weight.normal_(0, dim ** -0.5)
        m.out_proj.weight.normal_(0, (heads * 128) ** -0.5)
        m.q_norm.weight.copy_(1 + 0.05 * torch.randn(128, device=gpu))
        m.k_norm.weight.copy_(1 + 0.05 * torch.randn(128, device=gpu))
    return m


def test_patched_forward_matches_stock(gpu):
    class A(standin_dit.Attention):
        pass

    m = _module(A, gpu)
    S = 1000
    x = torch.randn(S, 512, device=gpu, dtype=torch.bfloat16)
    rope = h3attn.rope_freqs(S, 128, device=gpu)
    with torch.no_grad():
        want = m(x, rope_freqs=rope).float()
        assert hooks.install(A)
        got = m(x, rope_freqs=rope).float()
        no_rope = m(x).float()  # falls through to the stock path
        hooks.uninstall(A)
        want_no_rope = m(x).float()
    assert_close_absmax(got.cpu().numpy(), want.cpu().numpy(), what="patched forward")
    assert torch.equal(no_rope, want_no_rope)


def test_patched_optimized_attention(gpu):
    q, k, v = (torch.randn(1, 4, 300, 128, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    want = standin_dit.optimized_attention(q, k, v, 4, skip_reshape=True).float()
    orig = standin_dit.optimized_attention
    try:
        assert hooks.install_optimized_attention(standin_dit)
        assert not hooks.install_optimized_attention(standin_dit)
        got = standin_dit.optimized_attention(q, k, v, 4, skip_reshape=True).float()
        flat = standin_dit.optimized_attention(*(t.transpose(1, 2).reshape(1, 300, 512) for t in (q, k, v)), 4)
        masked = standin_dit.optimized_attention(q, k, v, 4, mask=torch.ones(300, 300, dtype=torch.bool, device=gpu),
                                                 skip_reshape=True)  # defers to the original
    finally:
        standin_dit.optimized_attention = orig
    assert_close_absmax(got.cpu().numpy(), want.cpu().numpy(), what="optimized_attention")
    assert torch.equal(flat.float(), got)
    assert_close_absmax(masked.float().cpu().numpy(), want.cpu().numpy(), what="masked fallback")


def test_sparse_override_in_dit_scope(gpu):
    """h3_sla-style override: keep < 1 runs the block-sparse kernel, keep = 1 runs dense."""
    class A(standin_dit.Attention):
        pass

    hooks.install_scope_patch(A)
    m = _module(A, gpu)
    m._h3sla_layer = 0
    S = 600
    x = torch.randn(S, 512, device=gpu, dtype=torch.bfloat16)
    rope = h3attn.rope_freqs(S, 128, device=gpu)
    dense_sched = hooks.Schedule("custom", [1.0] * 50, blk=64)
    sparse_sched = hooks.Schedule("custom", [0.5] * 50, blk=64)
    with torch.no_grad():
        stock = m(x, rope_freqs=rope).float()
        d = m(x, rope_freqs=rope, transformer_options={
            "optimized_attention_override": hooks.make_sla_override(schedule=dense_sched)}).float()
        logs = []
        s = m(x, rope_freqs=rope, transformer_options={
            "optimized_attention_override": hooks.make_sla_override(schedule=sparse_sched, log=logs.append)})
    assert torch.equal(d, stock)
    assert logs == [] and torch.isfinite(s.float()).all()
    assert not torch.equal(s.float(), stock)  # half the key blocks were skipped
