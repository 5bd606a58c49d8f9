"""The drop-in hooks on the GPU: the patched Attention.forward (HIP prologue in
place on the fused QKV output + HIP attention writing [S,H*D]) and the patched
optimized_attention must reproduce the stock forward (custom_nodes/h3_profiler/
__init__.py:92-111, restated in tests/standin_dit.py) on the same module."""
from __future__ import annotations

import pytest
import torch

import h3attn
import standin_dit
import oracle
from conftest import assert_close_absmax, from_dev_bf16
from h3attn import hooks, ops, sla

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


@pytest.mark.parametrize("S,heads,rot", [(1, 4, 128), (2, 1, 64), (63, 3, 128), (65, 2, 32), (777, 5, 128),
                                         (2048, 8, 96)])
def test_patched_forward_matches_stock_shapes(gpu, S, heads, rot):
    """The patched forward against the stock one over sequence lengths (one token
    included, where the kernels see a length-1 sequence), head counts and rot dims."""
    class A(standin_dit.Attention):
        pass

    dim = 128 * heads
    m = _module(A, gpu, dim=dim, heads=heads, seed=S)
    x = torch.randn(S, dim, device=gpu, dtype=torch.bfloat16)
    rope = h3attn.rope_freqs(S, rot, device=gpu)
    with torch.no_grad():
        want = m(x, rope_freqs=rope).float()
        assert hooks.install(A)
        try:
            got = m(x, rope_freqs=rope).float()
        finally:
            hooks.uninstall(A)
    assert_close_absmax(got.cpu().numpy(), want.cpu().numpy(), what=f"patched forward S={S} H={heads}")


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


def _capture_sparse(monkeypatch, layers):
    """Wrap sla.sparse_attention to keep (q, k, v, keep, kwargs, output) of the given layers."""
    real = sla.sparse_attention
    got = {}

    def spy(q, k, v, keep, blk, **kw):
        o = real(q, k, v, keep, blk, **kw)
        layer = hooks._state.layer
        if layer in layers:
            got[layer] = tuple(from_dev_bf16(t) for t in (q, k, v)) + (keep, blk, kw, from_dev_bf16(o))
        return o

    monkeypatch.setattr(sla, "sparse_attention", spy)
    return got


def _check_against_masked_oracle(captured, keep):
    """The captured layer output equals the oracle's attention masked by the oracle's block map at
    `keep` (top floor(keep * nk) key blocks by mean-pooled score, no forced diagonal)."""
    q, k, v, used_keep, blk, kw, o = captured
    assert used_keep == keep and not kw.get("force_diag", False)
    nk = -(-q.shape[2] // blk)
    bmap = oracle.block_map(q, k, blk, blk, keep=sla.keep_count(keep, nk), force_diag=False)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk, blk_k=blk)
    got = oracle.bf16_to_f32(o).reshape(o.shape)
    assert_close_absmax(got, ref, what=f"sparse layer at keep {keep}")
    return got, bmap


def test_sparse_override_in_dit_scope(gpu, monkeypatch):
    """h3_sla-style override: keep < 1 runs the block-sparse kernel on the layer's q/k/v (checked
    against the masked oracle), keep = 1 runs dense."""
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
    captured = _capture_sparse(monkeypatch, {0})
    with torch.no_grad():
        stock = m(x, rope_freqs=rope).float()
        d = m(x, rope_freqs=rope, transformer_options={
            "optimized_attention_override": hooks.make_sla_override(schedule=dense_sched)}).float()
        assert captured == {}
        logs = []
        m(x, rope_freqs=rope, transformer_options={
            "optimized_attention_override": hooks.make_sla_override(schedule=sparse_sched, log=logs.append)})
    assert torch.equal(d, stock)
    assert logs == []
    _check_against_masked_oracle(captured[0], 0.5)


def test_patched_model_runs_scheduled_keeps_against_masked_oracle(gpu, monkeypatch):
    """hooks.patch_model with the "balanced" preset on a 50-block stand-in DiT with the HIP forward
    installed: layer 30 (SLA15) and layer 31 (SLA25) each match the masked oracle at their own
    keep, and not at the other's (custom_nodes/h3_sla/__init__.py:44-49, 296-305, 328-346)."""
    class A(standin_dit.Attention):
        pass

    torch.manual_seed(0)
    dm = standin_dit.MiniMaxH3Model(512, 4, depth=50, attention_cls=A, dtype=torch.bfloat16, device=gpu)
    with torch.no_grad():
        for blk in dm.blocks:
            a = blk.attn
            a.qkv_proj.weight.normal_(0, 512 ** -0.5)
            a.out_proj.weight.normal_(0, 0.1 * 512 ** -0.5)
            a.q_norm.weight.copy_(1 + 0.05 * torch.randn(128, device=gpu))
            a.k_norm.weight.copy_(1 + 0.05 * torch.randn(128, device=gpu))
    mp = standin_dit.ModelPatcher(dm)
    try:
        assert hooks.install(A)
        logs = []
        pm = hooks.patch_model(mp, topk=0.35, blk=64, preset="balanced", log=logs.append)
        keeps = hooks.get_schedule(pm.model_options["transformer_options"]).keeps
        assert (keeps[30], keeps[31]) == (0.15, 0.25)
        captured = _capture_sparse(monkeypatch, {30, 31})
        S = 1000  # 16 key blocks: keep 0.15 -> 2 blocks, 0.25 -> 4
        x = torch.randn(S, 512, device=gpu, dtype=torch.bfloat16)
        rope = h3attn.rope_freqs(S, 128, device=gpu)
        with torch.no_grad():
            out = pm(x, rope)
        torch.cuda.synchronize()
    finally:
        hooks.uninstall(A)
    assert torch.isfinite(out.float()).all()
    for layer, keep, other in ((30, 0.15, 0.25), (31, 0.25, 0.15)):
        got, bmap = _check_against_masked_oracle(captured[layer], keep)
        assert int(bmap[0, 0, 0].sum()) == sla.keep_count(keep, 16)
        q, k, v = captured[layer][:3]
        wrong = oracle.attn_fwd(q, k, v, block_map=oracle.block_map(q, k, 64, 64, keep=sla.keep_count(other, 16),
                                                                     force_diag=False), blk_q=64, blk_k=64)
        with pytest.raises(AssertionError):
            assert_close_absmax(got, wrong, what="the other layer's keep")


def test_sparse_layers_take_block_means_from_the_prologue(gpu, monkeypatch):
    """With the HIP forward installed and an h3attn sparse override, a sparse layer's prologue pools
    q and k (h3a_qk_rmsnorm_rope_pool) and the override uses those means instead of pooling again;
    dense layers (keep 1) do not pool.  The model output equals that of the same run with the
    pooling left to the block map (the means are equal bit for bit, so is the selection)."""
    class A(standin_dit.Attention):
        pass

    torch.manual_seed(3)
    dm = standin_dit.MiniMaxH3Model(512, 4, depth=4, attention_cls=A, dtype=torch.bfloat16, device=gpu)
    with torch.no_grad():
        for blk in dm.blocks:
            blk.attn.qkv_proj.weight.normal_(0, 512 ** -0.5)
            blk.attn.out_proj.weight.normal_(0, 0.1 * 512 ** -0.5)
    mp = standin_dit.ModelPatcher(dm)
    S = 900
    x = torch.randn(S, 512, device=gpu, dtype=torch.bfloat16)
    rope = h3attn.rope_freqs(S, 128, device=gpu)
    real = sla.sparse_attention
    seen = []

    def spy(q, k, v, keep, blk, pooled=None, **kw):
        seen.append((hooks._state.layer, pooled is not None))
        return real(q, k, v, keep, blk, pooled=pooled, **kw)

    monkeypatch.setattr(sla, "sparse_attention", spy)
    pools = []
    real_rope = ops.qk_rmsnorm_rope_
    monkeypatch.setattr(ops, "qk_rmsnorm_rope_",
                        lambda *a, **kw: pools.append(kw.get("pool_blk")) or real_rope(*a, **kw))
    try:
        assert hooks.install(A)
        pm = hooks.patch_model(mp, topk=0.3, blk=64, preset="custom", layer_keep="100:2", log=lambda s: None)
        with torch.no_grad():
            fused = pm(x, rope)
            torch.cuda.synchronize()
            assert seen == [(0, True), (1, True), (3, True)] and pools == [64, 64, None, 64]
            seen.clear()
            monkeypatch.setattr(hooks, "_pool_blk_for", lambda opts: None)
            plain = pm(x, rope)
            torch.cuda.synchronize()
    finally:
        hooks.uninstall(A)
    assert seen == [(0, False), (1, False), (3, False)]
    assert torch.equal(fused, plain)
