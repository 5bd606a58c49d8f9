"""Randomized parity over the attention paths: dense, native block-sparse (blocks 64/128/192/256,
square or mixed), the tile-LUT path (every other multiple of 16) and the SLA route
(sla.sparse_attention with its own block map), each against the oracle at the attention
tolerance (max error <= 1e-2 * absmax, mean error <= 1e-3 * absmax).

Shapes are drawn per case from a fixed seed: B 1-2, H 1-3, Sq and Skv 1-1399 (equal or not),
inputs contiguous or read through [B,S,H,D] buffers, block maps of random density with
empty rows.  Such a sweep found that a length-1 query sequence (its stride 0, as for any
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
from conftest import assert_close_absmax, from_dev_bf16, randn_bf16, to_dev_bf16
from h3attn import ops, sla

pytestmark = pytest.mark.gpu

NATIVE = (64, 128, 192, 256)
MODES = ("dense", "native", "tiles", "sla")


def _device(bits, gpu, strided):
    t = to_dev_bf16(bits, gpu)  # [B,H,S,D] contiguous
    if strided:  # the same values read through a [B,S,H,D] buffer
        B, H, S, D = bits.shape
        buf = torch.empty(B, S, H, D, dtype=torch.bfloat16, device=gpu)
        buf.copy_(t.transpose(1, 2))
        t = buf.transpose(1, 2)
    return t


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
    what = f"seed {seed}: {mode} B={B} H={H} Sq={Sq} Skv={Skv} strided={strided} blk=({bq},{bk})"
    q = randn_bf16(rng, (B, H, Sq, 128))
    k = randn_bf16(rng, (B, H, Skv, 128))
    v = randn_bf16(rng, (B, H, Skv, 128), scale=4.0)
    qd, kd, vd = (_device(x, gpu, strided) for x in (q, k, v))
    if mode == "dense":
        o = h3attn.attn_fwd(qd, kd, vd)
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
            o = h3attn.attn_fwd_blocksparse(qd, kd, vd, lut, cnt, bq, bk)
        else:
            lut, cnt = ops.block_map_to_tile_lut(bt, bq, bk, Sq, Skv)
            o = ops.attn_fwd_blocksparse_tiles(qd, kd, vd, lut, cnt, queues=bool(rng.random() < 0.5))
        ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=bq, blk_k=bk)
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(from_dev_bf16(o.contiguous())).reshape(o.shape)
    assert_close_absmax(got, ref, what=what)
