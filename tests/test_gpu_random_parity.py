"""Randomized parity over the attention paths: dense, native block-sparse (blocks 64/128/192/256,
square or mixed), the tile-LUT path (every other multiple of 16) and the SLA route
(sla.sparse_attention with its own block map), each against the oracle at the attention
tolerance (max error <= 1e-2 * absmax, mean error <= 1e-3 * absmax).  Also the prologue
(qk-RMSNorm + RoPE, plain and with the block pooling; within one bf16 ulp of the oracle,
>= 99 % bit-identical, means equal to block_pool's) and the GPU block map (equal to the
oracle's fp64 selection except at near-ties; LUT and counts consistent with the map), and
shapes large enough for the work queues and split tails, against fp32 attention on the GPU.

Shapes are drawn per case from a fixed seed: B 1-2, H 1-3, Sq and Skv 1-1399 (equal or not),
q, k, v and O each contiguous, sequence-major, with padded rows or with padded batches,
block maps of random density with empty rows.  Such a sweep found that a length-1 query sequence (its stride 0, as for any
size-1 dimension) sent the kernels' padding rows onto row 0.

Reference: custom_nodes/h3_sla/__init__.py:226-235 (block map + sparse attention);
attn_sm80/fa3_sm80_h3.cu:355-457 (the dense kernel's masking, softmax and store).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import h3attn
import oracle
from conftest import assert_close_absmax, assert_prologue_close, from_dev_bf16, randn_bf16, to_dev_bf16
from h3attn import ops, sla

pytestmark = pytest.mark.gpu

NATIVE = (64, 128, 192, 256)
MODES = ("dense", "native", "tiles", "sla")


LAYOUTS = ("bhsd", "bshd", "padrow", "padbatch")


def _device(bits, gpu, layout):
    """The values of [B,H,S,D] `bits` on the GPU in one of four memory layouts: contiguous,
    sequence-major ([B,S,H,D] buffer), rows padded to 192 elements, or batches padded apart."""
    t = to_dev_bf16(bits, gpu)
    B, H, S, D = bits.shape
    if layout == "bshd":
        buf = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=gpu)
        buf.copy_(t.transpose(1, 2))
        return buf.transpose(1, 2)
    if layout == "padrow":
        buf = torch.full((B, H, S, D + 64), 7.0, dtype=torch.bfloat16, device=gpu)
        buf[..., :D] = t
        return buf[..., :D]
    if layout == "padbatch":
        buf = torch.full((B, H + 1, S, D), 7.0, dtype=torch.bfloat16, device=gpu)
        buf[:, :H] = t
        return buf[:, :H]
    return t


def _out_like(q, gpu, layout):
    """None (the library allocates O) or a preallocated O in a sequence-major or padded layout."""
    B, H, Sq, D = q.shape
    if layout == "bshd":
        return torch.empty(B, Sq, H, D, dtype=torch.bfloat16, device=gpu).transpose(1, 2)
    if layout == "padrow":
        return torch.empty(B, H, Sq, D + 64, dtype=torch.bfloat16, device=gpu)[..., :D]
    return None


def _case(seed):
    rng = np.random.default_rng(seed)
    mode = MODES[seed % 4]
    B = 1 if mode == "sla" else int(rng.integers(1, 3))
    H = int(rng.integers(1, 4))
    Sq = int(rng.integers(1, 1400))
    Skv = Sq if mode == "sla" or rng.random() < 0.6 else int(rng.integers(1, 1400))
    strided = bool(rng.random() < 0.4)
    if mode == "native":
        bq, bk = int(rng.choice(NATIVE)), int(rng.choice(NATIVE))
    elif mode in ("tiles", "sla"):
        while True:
            bq = 16 * int(rng.integers(1, 17))
            bk = bq if mode == "sla" or rng.random() < 0.5 else 16 * int(rng.integers(1, 17))
            if mode == "sla" or not (bq in NATIVE and bk in NATIVE):
                break
    else:
        bq = bk = 0
    return rng, mode, B, H, Sq, Skv, strided, bq, bk


@pytest.mark.parametrize("seed", list(range(7000, 7120)) + [50297])
def test_random_case_against_oracle(gpu, seed):
    rng, mode, B, H, Sq, Skv, strided, bq, bk = _case(seed)
    q = randn_bf16(rng, (B, H, Sq, 128))
    k = randn_bf16(rng, (B, H, Skv, 128))
    v = randn_bf16(rng, (B, H, Skv, 128), scale=4.0)
    lay = [("bshd" if strided else "bhsd") if rng.random() < 0.5 else LAYOUTS[int(rng.integers(0, 4))]
           for _ in range(3)]
    out_lay = LAYOUTS[int(rng.integers(0, 4))]
    what = f"seed {seed}: {mode} B={B} H={H} Sq={Sq} Skv={Skv} layouts={lay} out={out_lay} blk=({bq},{bk})"
    qd, kd, vd = (_device(x, gpu, lt) for x, lt in zip((q, k, v), lay))
    out = _out_like(qd, gpu, out_lay)
    if mode == "dense":
        o = h3attn.attn_fwd(qd, kd, vd, out=out)
        ref = oracle.attn_fwd(q, k, v)
    elif mode == "sla":
        keep, diag = float(rng.uniform(0.05, 0.9)), bool(rng.random() < 0.5)
        bmap, _, _ = sla.get_block_map(qd, kd, keep, bq, bq, force_diag=diag, want_map=True)
        o = sla.sparse_attention(qd, kd, vd, keep, bq, force_diag=diag)
        ref = oracle.attn_fwd(q, k, v, block_map=bmap.cpu().numpy(), blk_q=bq, blk_k=bq)
    else:
        nq, nk = -(-Sq // bq), -(-Skv // bk)
        bmap = (rng.random((B, H, nq, nk)) < rng.uniform(0.0, 0.7)).astype(np.uint8)
        if nq > 1 and rng.random() < 0.5:
            bmap[0, 0, int(rng.integers(0, nq))] = 0  # an empty row
        bt = torch.from_numpy(bmap).to(gpu)
        if mode == "native":
            lut, cnt = h3attn.block_map_to_lut(bt)
            o = h3attn.attn_fwd_blocksparse(qd, kd, vd, lut, cnt, bq, bk, out=out)
        else:
            lut, cnt = ops.block_map_to_tile_lut(bt, bq, bk, Sq, Skv)
            o = ops.attn_fwd_blocksparse_tiles(qd, kd, vd, lut, cnt, out=out, queues=bool(rng.random() < 0.5))
        ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=bq, blk_k=bk)
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(from_dev_bf16(o.contiguous())).reshape(o.shape)
    assert_close_absmax(got, ref, what=what)


@pytest.mark.parametrize("seed", range(3000, 3030))
def test_random_prologue_case(gpu, seed):
    """Reference: harness/sp_runtime.py:93-99 (rms_rope_split_half_ on fused-QKV views)."""
    rng = np.random.default_rng(seed)
    S, H, rot = int(rng.integers(1, 700)), int(rng.integers(1, 90)), 16 * int(rng.integers(0, 9))
    fused = bool(rng.random() < 0.5)
    B = 1 if fused else int(rng.integers(1, 3))
    pool = int(16 * rng.integers(1, 17)) if rng.random() < 0.5 else None
    what = f"seed {seed}: B={B} S={S} H={H} rot={rot} fused={fused} pool={pool}"
    x = rng.standard_normal((2, B, S, H, 128)).astype(np.float32)
    x *= rng.uniform(0.5, 4.0, size=(2, B, S, 1, 1)).astype(np.float32)
    w = (1.0 + 0.05 * rng.standard_normal((2, 128))).astype(np.float32)
    xb, wb = oracle.f32_to_bf16(x), oracle.f32_to_bf16(w)
    if fused:
        qkv = torch.zeros(S, 3 * H * 128, dtype=torch.bfloat16, device=gpu)
        q = qkv[:, :H * 128].view(1, S, H, 128)
        k = qkv[:, H * 128:2 * H * 128].view(1, S, H, 128)
        q.copy_(to_dev_bf16(xb[0], gpu))
        k.copy_(to_dev_bf16(xb[1], gpu))
    else:
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
    assert_prologue_close(from_dev_bf16(q).reshape(rq.shape), rq, what + " q")
    assert_prologue_close(from_dev_bf16(k).reshape(rk.shape), rk, what + " k")
    if pool:
        assert torch.equal(pq, ops.block_pool(q.transpose(1, 2), pool)), what + ": q means"
        assert torch.equal(pk, ops.block_pool(k.transpose(1, 2), pool)), what + ": k means"


@pytest.mark.parametrize("seed", range(5000, 5030))
def test_random_block_map_case(gpu, seed):
    """Reference: custom_nodes/h3_sla/__init__.py:232 (SLA get_block_map at the node's sizes)."""
    rng = np.random.default_rng(seed)
    B, H, S = int(rng.integers(1, 3)), int(rng.integers(1, 4)), int(rng.integers(1, 3000))
    bq = 16 * int(rng.integers(1, 17))
    bk = bq if rng.random() < 0.6 else 16 * int(rng.integers(1, 17))
    ratio, diag = float(rng.uniform(0.01, 1.0)), bool(rng.random() < 0.5)
    what = f"seed {seed}: B={B} H={H} S={S} blk=({bq},{bk}) ratio={ratio:.3f} diag={diag}"
    q, k = randn_bf16(rng, (B, H, S, 128)), randn_bf16(rng, (B, H, S, 128))
    keep = sla.keep_count(ratio, -(-S // bk))
    ref, scores = oracle.block_map(q, k, bq, bk, keep=keep, force_diag=diag, return_scores=True)
    bmap, lut, cnt = sla.get_block_map(to_dev_bf16(q, gpu), to_dev_bf16(k, gpu), ratio, bq, bk,
                                       force_diag=diag, want_map=True)
    got = bmap.cpu().numpy()
    for b, h, i, j in np.argwhere(got != ref):  # only fp32-vs-fp64 near-ties may differ
        thr = np.sort(scores[b, h, i])[::-1][keep - 1]
        assert abs(scores[b, h, i, j] - thr) <= 1e-4 * max(1.0, abs(thr)), what
    cn, ln = cnt.cpu().numpy(), lut.cpu().numpy()
    assert np.array_equal(cn, np.minimum(got.sum(-1), ln.shape[-1])), what + ": counts"
    for idx in np.ndindex(*got.shape[:3]):
        nz = np.flatnonzero(got[idx])[:ln.shape[-1]]
        assert np.array_equal(ln[idx][:len(nz)], nz) and np.all(ln[idx][len(nz):] == -1), what


def _ref_head(q, k, v, mask=None):
    """fp32 attention of one head from contiguous operands (plain matmuls, no batched bf16 products)."""
    s = (q.float() @ k.float().t().contiguous()) / 128 ** 0.5
    if mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, -1), nan=0.0)
    return p @ v.float()


@pytest.mark.parametrize("seed", [8000, 8001, 8002, 8003, 8005, 8006])
def test_random_large_case(gpu, seed):
    """Shapes large enough for the persistent grid with per-XCD work queues and split last
    rounds (H 4-24, Sq and Skv 2048-16384): dense, and native block-sparse at a random block
    size, against fp32 attention per head on the GPU."""
    rng = np.random.default_rng(seed)
    mode = ("dense", "sparse")[seed % 2]
    H, Sq = int(rng.integers(4, 25)), int(rng.integers(2048, 16385))
    Skv = Sq if rng.random() < 0.7 else int(rng.integers(2048, 16385))
    blk = int(rng.choice(NATIVE))
    g = torch.Generator(device=gpu).manual_seed(seed)
    q = torch.randn(1, H, Sq, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    k = torch.randn(1, H, Skv, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    v = torch.randn(1, H, Skv, 128, generator=g, device=gpu, dtype=torch.bfloat16) * 4
    bm = None
    if mode == "dense":
        o = h3attn.attn_fwd(q, k, v)
    else:
        nq, nk = -(-Sq // blk), -(-Skv // blk)
        bm = (torch.rand(1, H, nq, nk, generator=g, device=gpu) < float(rng.uniform(0.05, 0.5))).to(torch.uint8)
        lut, cnt = h3attn.block_map_to_lut(bm)
        o = h3attn.attn_fwd_blocksparse(q, k, v, lut, cnt, blk, blk)
    torch.cuda.synchronize()
    for h in range(H):
        mask = None
        if bm is not None:
            mask = bm[0, h].bool().repeat_interleave(blk, 0)[:Sq].repeat_interleave(blk, 1)[:, :Skv]
        ref = _ref_head(q[0, h], k[0, h], v[0, h], mask)
        assert_close_absmax(o[0, h].float().cpu().numpy(), ref.cpu().numpy(),
                            what=f"seed {seed}: {mode} H={H} Sq={Sq} Skv={Skv} blk={blk} head {h}")
