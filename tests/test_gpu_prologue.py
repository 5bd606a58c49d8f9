"""Parity of the fused qk-RMSNorm + split-half RoPE kernel (h3a_qk_rmsnorm_rope) with the oracle.

Call contract: comfy.quant_ops.ck.rms_rope_split_half_(q, k, rope_freqs, qw, kw,
epsilon, rot_dim) on [1,S,H,D] strided views (harness/sp_runtime.py:93-99,
custom_nodes/h3_profiler/__init__.py:99-106).  Outputs are bf16: the kernel
(fp32 math) and the oracle (fp64 math) must agree to within one bf16 ulp,
with at least 99% of values bit-identical.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import h3attn
import oracle
from conftest import assert_prologue_close, from_dev_bf16, to_dev_bf16

pytestmark = pytest.mark.gpu


def _inputs(rng, S, H, spread=True):
    x = rng.standard_normal((2, S, H, 128)).astype(np.float32)
    if spread:  # per-token dynamic range U(0.5, 4), as in the S=8192 prologue workload
        x *= rng.uniform(0.5, 4.0, size=(2, S, 1, 1)).astype(np.float32)
    w = (1.0 + 0.05 * rng.standard_normal((2, 128))).astype(np.float32)
    return oracle.f32_to_bf16(x), oracle.f32_to_bf16(w)


def _run_gpu(xq, xk, w, rope, rot, device, fused_layout):
    S, H = xq.shape[0], xq.shape[1]
    if fused_layout:
        qkv = torch.zeros(S, 3 * H * 128, dtype=torch.bfloat16, device=device)
        q = qkv[:, :H * 128].view(1, S, H, 128)
        k = qkv[:, H * 128:2 * H * 128].view(1, S, H, 128)
        vpart = qkv[:, 2 * H * 128:]
        vpart.copy_(torch.full_like(vpart, 0.5))
        q.copy_(to_dev_bf16(xq, device).view(1, S, H, 128))
        k.copy_(to_dev_bf16(xk, device).view(1, S, H, 128))
    else:
        q = to_dev_bf16(xq, device).view(1, S, H, 128).clone()
        k = to_dev_bf16(xk, device).view(1, S, H, 128).clone()
        vpart = None
    rope_t = None if rope is None else torch.from_numpy(rope).view(1, S, 1, rot // 2, 2, 2).to(device)
    h3attn.rms_rope_split_half_(q, k, rope_t, to_dev_bf16(w[0], device), to_dev_bf16(w[1], device),
                                epsilon=1e-6, rot_dim=rot)
    torch.cuda.synchronize()
    if vpart is not None:
        assert torch.all(vpart == 0.5), "kernel wrote outside q/k"
    return from_dev_bf16(q)[0], from_dev_bf16(k)[0]


@pytest.mark.parametrize("S,H,rot,fused", [
    (37, 3, 128, False), (37, 3, 64, True), (5, 1, 0, False), (200, 7, 128, True), (64, 56, 32, True),
    (33, 28, 128, True), (17, 84, 64, False),  # 28 heads per wave: one chunk, three chunks
])
def test_prologue_small(gpu, S, H, rot, fused):
    rng = np.random.default_rng(S * 100 + rot)
    x, w = _inputs(rng, S, H)
    rope = oracle.rope_table(S, rot) if rot else None
    gq, gk = _run_gpu(x[0], x[1], w, rope, rot, gpu, fused)
    rq, rk = oracle.qk_rmsnorm_rope(x[0][None], x[1][None], rope, w[0], w[1], eps=1e-6, rot_dim=rot)
    assert_prologue_close(gq, rq[0], "q")
    assert_prologue_close(gk, rk[0], "k")


def test_prologue_s8192_h56_fused_views(gpu):
    """S=8192, H=56 strided views of the fused QKV output, theta 10000, rot 128."""
    S, H = 8192, 56
    rng = np.random.default_rng(8192)
    x, w = _inputs(rng, S, H)
    rope = oracle.rope_table(S, 128)
    gq, gk = _run_gpu(x[0], x[1], w, rope, 128, gpu, True)
    rq, rk = oracle.qk_rmsnorm_rope(x[0][None], x[1][None], rope, w[0], w[1], eps=1e-6, rot_dim=128)
    assert_prologue_close(gq, rq[0], "q")
    assert_prologue_close(gk, rk[0], "k")


def test_prologue_rejects_bad_layout(gpu):
    q = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16, device=gpu)
    k = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16, device=gpu)
    w = torch.ones(128, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        h3attn.qk_rmsnorm_rope_(q[..., ::2], k[..., ::2], None, w[:64], w[:64], rot_dim=0)
    with pytest.raises(ValueError):
        h3attn.qk_rmsnorm_rope_(q, k, None, w, w, rot_dim=24)


@pytest.mark.parametrize("B,S,H,rot,pool", [(1, 1, 1, 128, None), (2, 1, 3, 64, 16), (1, 1, 56, 128, 64),
                                           (2, 5, 1, 0, 48), (1, 300, 1, 128, 256)])
def test_size_one_dimensions(gpu, B, S, H, rot, pool):
    """One token and/or one head: a size-1 dimension's stride reaches the library as 0.  q/k
    within one bf16 ulp of the oracle; the pooled means equal block_pool's."""
    from h3attn import ops
    rng = np.random.default_rng(B * 1000 + S * 10 + H)
    x = rng.standard_normal((2, B, S, H, 128)).astype(np.float32)
    w = (1.0 + 0.05 * rng.standard_normal((2, 128))).astype(np.float32)
    xb, wb = oracle.f32_to_bf16(x), oracle.f32_to_bf16(w)
    q, k = to_dev_bf16(xb[0], gpu).clone(), to_dev_bf16(xb[1], gpu).clone()
    rope = oracle.rope_table(S, rot) if rot else None
    rope_t = None if rope is None else torch.from_numpy(rope).view(1, S, 1, rot // 2, 2, 2).to(gpu)
    qw, kw = to_dev_bf16(wb[0], gpu), to_dev_bf16(wb[1], gpu)
    if pool:
        pq, pk = ops.qk_rmsnorm_rope_(q, k, rope_t, qw, kw, eps=1e-6, rot_dim=rot, pool_blk=pool)
    else:
        h3attn.rms_rope_split_half_(q, k, rope_t, qw, kw, epsilon=1e-6, rot_dim=rot)
    torch.cuda.synchronize()
    rq, rk = oracle.qk_rmsnorm_rope(xb[0], xb[1], rope, wb[0], wb[1], eps=1e-6, rot_dim=rot)
    assert_prologue_close(from_dev_bf16(q).reshape(rq.shape), rq, "q")
    assert_prologue_close(from_dev_bf16(k).reshape(rk.shape), rk, "k")
    if pool:
        assert torch.equal(pq, ops.block_pool(q.transpose(1, 2), pool))
        assert torch.equal(pk, ops.block_pool(k.transpose(1, 2), pool))


@pytest.mark.parametrize("S,H,blk,rot", [(8192, 56, 64, 128), (1000, 5, 16, 64), (777, 56, 200, 128),
                                         (300, 12, 128, 0), (3, 2, 64, 128), (4100, 9, 48, 128)])
def test_pooled_prologue_equals_prologue_then_block_pool(gpu, S, H, blk, rot):
    """h3a_qk_rmsnorm_rope_pool on fused-QKV views: q and k equal h3a_qk_rmsnorm_rope's bit for bit,
    the v part is untouched, and the block means equal block_pool of the result bit for bit (the
    same sums in the same order), including a partial last block, blocks of fewer than 4 tokens
    and head counts that leave a partial head chunk."""
    from h3attn import ops
    g = torch.Generator(device=gpu).manual_seed(S + H + blk)
    qkv = torch.randn(S, 3 * H * 128, generator=g, device=gpu, dtype=torch.float32)
    qkv[:, :2 * H * 128] *= torch.empty(S, 1, device=gpu).uniform_(0.5, 4.0, generator=g)
    qkv = qkv.to(torch.bfloat16)
    qw = (1 + 0.05 * torch.randn(128, generator=g, device=gpu)).to(torch.bfloat16)
    kw = (1 + 0.05 * torch.randn(128, generator=g, device=gpu)).to(torch.bfloat16)
    rope = h3attn.rope_freqs(S, rot, device=gpu) if rot else None

    def views(t):
        return t[:, :H * 128].view(1, S, H, 128), t[:, H * 128:2 * H * 128].view(1, S, H, 128)

    a, b = qkv.clone(), qkv.clone()
    h3attn.qk_rmsnorm_rope_(*views(a), rope, qw, kw, rot_dim=rot)
    pq, pk = h3attn.qk_rmsnorm_rope_(*views(b), rope, qw, kw, rot_dim=rot, pool_blk=blk)
    torch.cuda.synchronize()
    assert torch.equal(a, b), "pooled prologue changed q/k differently (or touched v)"
    assert torch.equal(b[:, 2 * H * 128:], qkv[:, 2 * H * 128:])
    qh, kh = (t.transpose(1, 2) for t in views(b))
    assert tuple(pq.shape) == (1, H, -(-S // blk), 128)
    assert torch.equal(pq, ops.block_pool(qh, blk)), "q means differ from block_pool"
    assert torch.equal(pk, ops.block_pool(kh, blk)), "k means differ from block_pool"
