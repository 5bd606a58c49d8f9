"""Parity of the block-sparse kernel (h3a_attn_fwd_blocksparse) and the LUT builder.

Reference: custom_nodes/h3_sla/__init__.py:226-235 (block map + sparse attention;
skipped key blocks contribute nothing).  The sparse output is compared with dense
attention masked to the same block map (the oracle), at the attention tolerance
(max error <= 1e-2 * absmax, mean error <= 1e-3 * absmax).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import h3attn
import oracle
from conftest import assert_close_absmax, from_dev_bf16, ramp_case, randn_bf16, to_dev_bf16
from h3attn import _lib, ops, sla

pytestmark = pytest.mark.gpu


def _lut_np(bmap, max_k):
    B, H, nq, nk = bmap.shape
    lut = np.full((B, H, nq, max_k), -1, np.int32)
    cnt = np.zeros((B, H, nq), np.int32)
    for idx in np.ndindex(B, H, nq):
        nz = np.flatnonzero(bmap[idx])
        cnt[idx] = len(nz)
        lut[idx][:len(nz)] = nz
    return lut, cnt


def test_block_map_to_lut(gpu):
    rng = np.random.default_rng(3)
    bmap = (rng.random((2, 3, 17, 29)) < 0.3).astype(np.uint8)
    bmap[0, 0, 0] = 0  # an empty row
    max_k = int(bmap.sum(-1).max())
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu), max_k)
    rl, rc = _lut_np(bmap, max_k)
    assert np.array_equal(cnt.cpu().numpy(), rc)
    assert np.array_equal(lut.cpu().numpy(), rl)


@pytest.mark.parametrize("blk,S,H", [(128, 1000, 2), (64, 1000, 2), (128, 1160, 1), (64, 777, 3),
                                     (192, 1000, 2), (256, 1000, 2), (192, 1537, 1), (256, 1300, 3)])
def test_sparse_vs_masked_oracle(gpu, blk, S, H):
    rng = np.random.default_rng(blk + S)
    q, k, v = (randn_bf16(rng, (1, H, S, 128)) for _ in range(3))
    nk = -(-S // blk)
    bmap = oracle.block_map(q, k, blk, blk, keep=max(1, nk // 4), force_diag=True)
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    o = h3attn.attn_fwd_blocksparse(*(to_dev_bf16(x, gpu) for x in (q, k, v)), lut, cnt, blk, blk)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk, blk_k=blk)
    assert_close_absmax(got, ref, what=f"sparse blk={blk}")


@pytest.mark.parametrize("blk_q,blk_k,S", [(256, 64, 1000), (64, 256, 1000), (192, 128, 1111),
                                           (128, 192, 1111), (256, 192, 777), (192, 256, 1500)])
@pytest.mark.parametrize("split", [True, False])
def test_sparse_mixed_block_sizes(gpu, blk_q, blk_k, S, split):
    """Query and key blocks of different sizes from {64, 128, 192, 256}: a LUT row serves
    blk_q / 64 or blk_q / 128 query sub-blocks, a key block is blk_k / 64 stages."""
    rng = np.random.default_rng(blk_q * 7 + blk_k + S)
    H = 2
    q, k, v = (randn_bf16(rng, (1, H, S, 128)) for _ in range(3))
    nk = -(-S // blk_k)
    bmap = oracle.block_map(q, k, blk_q, blk_k, keep=max(1, nk // 3), force_diag=True)
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    o = h3attn.attn_fwd_blocksparse(*(to_dev_bf16(x, gpu) for x in (q, k, v)), lut, cnt, blk_q, blk_k,
                                    split_tail=split)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk_q, blk_k=blk_k)
    assert_close_absmax(got, ref, what=f"sparse blk_q={blk_q} blk_k={blk_k}")


@pytest.mark.parametrize("blk_q,blk_k,Sq,Skv,split", [(128, 128, 700, 1100, True), (64, 64, 1100, 700, False),
                                                       (192, 128, 900, 1300, True), (256, 64, 1000, 600, False)])
def test_sparse_batched_cross_lengths_strided_side_stream(gpu, blk_q, blk_k, Sq, Skv, split):
    """B=2 with Sq != Skv (either way round), q read from a [B,Sq,H,D] buffer and k/v from
    one fused [B,Skv,2*H*D] buffer through strided [B,H,S,D] views, O written into a
    strided view, on a side stream: the masked oracle on the same block map."""
    rng = np.random.default_rng(blk_q * 31 + blk_k + Sq + Skv)
    B, H, D = 2, 3, 128
    q, k, v = randn_bf16(rng, (B, H, Sq, D)), randn_bf16(rng, (B, H, Skv, D)), randn_bf16(rng, (B, H, Skv, D))
    nk = -(-Skv // blk_k)
    bmap = oracle.block_map(q, k, blk_q, blk_k, keep=max(1, nk // 3), force_diag=True)
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    qbuf = to_dev_bf16(np.ascontiguousarray(q.transpose(0, 2, 1, 3)), gpu)          # [B,Sq,H,D]
    kv = np.concatenate([k.transpose(0, 2, 1, 3).reshape(B, Skv, H * D),
                         v.transpose(0, 2, 1, 3).reshape(B, Skv, H * D)], axis=2)    # [B,Skv,2HD]
    kvbuf = to_dev_bf16(np.ascontiguousarray(kv), gpu)
    qd = qbuf.transpose(1, 2)
    kd = kvbuf[:, :, :H * D].view(B, Skv, H, D).transpose(1, 2)
    vd = kvbuf[:, :, H * D:].view(B, Skv, H, D).transpose(1, 2)
    obuf = torch.full((B, Sq, H, D), 7.0, dtype=torch.bfloat16, device=gpu)
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        h3attn.attn_fwd_blocksparse(qd, kd, vd, lut, cnt, blk_q, blk_k, out=obuf.transpose(1, 2),
                                    split_tail=split)
    side.synchronize()
    got = oracle.bf16_to_f32(from_dev_bf16(obuf.transpose(1, 2))).reshape(B, H, Sq, D)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk_q, blk_k=blk_k)
    assert_close_absmax(got, ref, what=f"sparse B=2 Sq={Sq} Skv={Skv} blk_q={blk_q} blk_k={blk_k}")


def test_sparse_unsupported_block_sizes_raise(gpu):
    """Block sizes that are not multiples of 16 raise ValueError before any launch; the native
    entry point h3a_attn_fwd_blocksparse refuses sizes outside {64, 128, 192, 256} with
    H3A_ERR_UNSUPPORTED (the Python op runs those through the tile LUT entry points)."""
    q = torch.zeros(1, 1, 256, 128, dtype=torch.bfloat16, device=gpu)
    lut = torch.zeros(1, 1, 8, 1, dtype=torch.int32, device=gpu)
    cnt = torch.ones(1, 1, 8, dtype=torch.int32, device=gpu)
    for bq, bk in ((40, 64), (64, 24), (8, 8), (-64, 64)):
        nqb = -(-256 // abs(bq))
        with pytest.raises(ValueError, match="unsupported"):
            h3attn.attn_fwd_blocksparse(q, q, q, lut[:, :, :1].expand(1, 1, nqb, 1).contiguous(),
                                        cnt[:, :, :1].expand(1, 1, nqb).contiguous(), bq, bk)
    L = _lib.lib()
    st = _lib.strides3(256 * 128, 256 * 128, 128)
    for bq, bk in ((32, 64), (64, 96), (48, 48), (320, 64)):
        rc = L.h3a_attn_fwd_blocksparse(q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(), 1, 1, 256, 256, 128,
                                        st, st, st, st, lut.data_ptr(), cnt.data_ptr(), bq, bk, 1, 0.1, None)
        assert rc == _lib.H3A_ERR_UNSUPPORTED, (bq, bk, rc)


@pytest.mark.parametrize("S,blk_k,blk_q", [(640, 128, 128), (1300, 64, 128), (131, 128, 128),
                                           (640, 64, 64), (1300, 128, 64), (131, 64, 64), (700, 256, 64)])
def test_sparse_pairs_uneven_lists(gpu, S, blk_k, blk_q):
    """Query blocks run in pairs (blocks 2p and 2p+1 share a workgroup and step through
    the longer of their two LUT lists; 64-row blocks with each group's waves split over
    the two key halves of a stage).  Random keep counts from 0 to all key blocks per row,
    so partners differ in length, some rows are empty (O = 0) and, with an odd block
    count, the last block has no partner."""
    rng = np.random.default_rng(7000 + S + blk_k + blk_q)
    q, k, v = (randn_bf16(rng, (1, 2, S, 128)) for _ in range(3))
    nq, nk = -(-S // blk_q), -(-S // blk_k)
    bmap = np.zeros((1, 2, nq, nk), np.uint8)
    for h in range(2):
        for i in range(nq):
            n = int(rng.integers(0, nk + 1)) if i % 3 else 0
            bmap[0, h, i, rng.choice(nk, size=n, replace=False)] = 1
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    o = h3attn.attn_fwd_blocksparse(*(to_dev_bf16(x, gpu) for x in (q, k, v)), lut, cnt, blk_q, blk_k)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk_q, blk_k=blk_k)
    assert_close_absmax(got, ref, what=f"sparse pairs S={S} blk_q={blk_q} blk_k={blk_k}")
    for h in range(2):
        for i in range(nq):
            if not bmap[0, h, i].any():
                assert not got[0, h, blk_q * i:blk_q * (i + 1)].any(), f"empty row h={h} block={i}"


@pytest.mark.parametrize("S,blk_k", [(1300, 128), (2000, 64), (640, 64)])
def test_sparse_split_tail_matches_unsplit(gpu, S, blk_k):
    """The split-tail path (h3a_attn_fwd_blocksparse_ws): each pair of 128-row query blocks
    in the last, partly filled round of workgroups is cut into ranges of both blocks'
    lists, and the combine kernel merges the partial results.  Uneven, empty and unpaired
    lists, so some pieces hold no stage of one block or of both.  Equal to the oracle and
    to the unsplit kernel at the attention tolerance; empty rows stay exactly 0."""
    rng = np.random.default_rng(9100 + S + blk_k)
    q, k, v = (randn_bf16(rng, (1, 2, S, 128)) for _ in range(3))
    nq, nk = -(-S // 128), -(-S // blk_k)
    bmap = np.zeros((1, 2, nq, nk), np.uint8)
    for h in range(2):
        for i in range(nq):
            n = int(rng.integers(0, nk + 1)) if i % 3 else 0
            bmap[0, h, i, rng.choice(nk, size=n, replace=False)] = 1
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    assert ops.sparse_workspace_bytes(1, 2, S, S, 128, blk_k, lut.shape[3]) > 0, "meant to split"
    qd, kd, vd = (to_dev_bf16(x, gpu) for x in (q, k, v))
    o_split = ops.attn_fwd_blocksparse(qd, kd, vd, lut, cnt, 128, blk_k)
    o_whole = ops.attn_fwd_blocksparse(qd, kd, vd, lut, cnt, 128, blk_k, split_tail=False)
    got = oracle.bf16_to_f32(from_dev_bf16(o_split)).reshape(o_split.shape)
    whole = oracle.bf16_to_f32(from_dev_bf16(o_whole)).reshape(o_whole.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=128, blk_k=blk_k)
    assert_close_absmax(got, ref, what=f"sparse split S={S} blk_k={blk_k} vs oracle")
    assert_close_absmax(whole, ref, what=f"sparse unsplit S={S} blk_k={blk_k} vs oracle")
    assert_close_absmax(got, whole, what="sparse split vs unsplit")
    for h in range(2):
        for i in range(nq):
            if not bmap[0, h, i].any():
                assert not got[0, h, 128 * i:128 * (i + 1)].any(), f"empty row h={h} block={i}"


@pytest.mark.parametrize("blk", [64, 128])
def test_sparse_wide_kv_stride(gpu, blk):
    """K and V as views with a sequence stride just below the 2^24-element limit, so
    a (b,h) slice spans 6.7 GB and stage addresses pass 2^32 bytes from the slice
    base: each stage's buffer resource is rebased on its first row with 64-bit
    arithmetic.  Same result as the masked oracle on the gathered rows."""
    rng = np.random.default_rng(4000 + blk)
    S, ss = 200, (1 << 24) - 8
    q, k, v = (randn_bf16(rng, (1, 1, S, 128)) for _ in range(3))
    nk = -(-S // blk)
    bmap = oracle.block_map(q, k, blk, blk, keep=max(1, nk // 2), force_diag=True)
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    n = (S - 1) * ss + 128

    def wide(bits):
        base = torch.empty(n, dtype=torch.bfloat16, device=gpu)
        view = base.as_strided((1, 1, S, 128), (n, n, ss, 1))
        view.copy_(to_dev_bf16(bits, gpu))
        return view

    kd, vd = wide(k), wide(v)
    o = h3attn.attn_fwd_blocksparse(to_dev_bf16(q, gpu), kd, vd, lut, cnt, blk, blk)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk, blk_k=blk)
    del kd, vd
    assert_close_absmax(got, ref, what=f"sparse blk={blk} wide K/V stride")


@pytest.mark.parametrize("blk_k", [64, 128])
def test_all_blocks_kept_equals_dense(gpu, blk_k):
    """A full block map visits the key stages in the dense order: bit-identical output
    to the unsplit dense kernel (h3a_attn_fwd), both without the split tail.  Holds for
    the default build, whose dense kernel also works in 64-key stages (a 128-key build
    sums in another order)."""
    rng = np.random.default_rng(21)
    S = 1000
    q, k, v = (to_dev_bf16(randn_bf16(rng, (1, 2, S, 128)), gpu) for _ in range(3))
    nq, nk = -(-S // 128), -(-S // blk_k)
    lut, cnt = h3attn.block_map_to_lut(torch.ones(1, 2, nq, nk, dtype=torch.uint8, device=gpu))
    o_s = h3attn.attn_fwd_blocksparse(q, k, v, lut, cnt, 128, blk_k, split_tail=False)
    o_d = h3attn.attn_fwd(q, k, v, split_tail=False)
    torch.cuda.synchronize()
    assert torch.equal(o_s, o_d)


@pytest.mark.parametrize("blk_k", [64, 128])
@pytest.mark.parametrize("S", [1, 20, 33, 64, 97, 300])
def test_sparse64_key_halves_vs_oracle(gpu, S, blk_k):
    """64-row query blocks run as 4-wave workgroups whose two key halves (keys 0-31
    and 32-63 of every 64-key stage) keep separate softmax state and are merged at
    the end.  Key counts that leave the second half empty (S <= 32), partly filled
    (33, 97) or exact (64), and a full block map at both key-block sizes, against
    the masked oracle."""
    rng = np.random.default_rng(900 + S + blk_k)
    q, k, v = (randn_bf16(rng, (1, 2, S, 128)) for _ in range(3))
    nq, nk = -(-S // 64), -(-S // blk_k)
    bmap = np.ones((1, 2, nq, nk), np.uint8)
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    o = h3attn.attn_fwd_blocksparse(*(to_dev_bf16(x, gpu) for x in (q, k, v)), lut, cnt, 64, blk_k)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=64, blk_k=blk_k)
    assert_close_absmax(got, ref, what=f"sparse64 S={S} blk_k={blk_k}")


def test_sparse64_key_half_maxima_differ(gpu):
    """Key 104 (key half 1 of the second stage) scores 22*22 = 484 above the rest
    (~62 log2 units after scaling; the other scores spread ~1.4 log2 units), so the
    merge scales key half 0's O and l by ~2^-62 against half 1's: the result is the
    masked oracle's, key 104's value row."""
    rng = np.random.default_rng(77)
    S = 256
    q, k, v = (randn_bf16(rng, (1, 1, S, 128)) for _ in range(3))
    qf = oracle.bf16_to_f32(q).reshape(q.shape).copy()
    kf = oracle.bf16_to_f32(k).reshape(k.shape).copy()
    qf[..., 0] = 22.0
    kf[..., 0] = 0.0
    kf[0, 0, 64 + 40, 0] = 22.0
    q, k = oracle.f32_to_bf16(qf).reshape(q.shape), oracle.f32_to_bf16(kf).reshape(k.shape)
    bmap = np.ones((1, 1, S // 64, S // 64), np.uint8)
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    o = h3attn.attn_fwd_blocksparse(*(to_dev_bf16(x, gpu) for x in (q, k, v)), lut, cnt, 64, 64)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=64, blk_k=64)
    assert_close_absmax(got, ref, what="sparse64 dominant key in key half 1")


@pytest.mark.parametrize("blk,slope", [(64, 0.4), (128, 0.4), (128, 0.0383)])
def test_sparse_running_max_rises(gpu, blk, slope):
    """Even rows see scores rising along the keys (~210 or ~20 log2 units per 64 keys),
    odd rows falling, over a random half of the key blocks plus the diagonal: the
    running max is refreshed along the LUT order at every stage or every few stages."""
    rng = np.random.default_rng(40 + blk)
    S = 1000
    q, k, v = ramp_case(rng, S, slope=slope, q0=64.0)
    nk = -(-S // blk)
    bmap = (rng.random((1, 2, nk, nk)) < 0.5).astype(np.uint8)
    for i in range(nk):
        bmap[:, :, i, i] = 1  # the diagonal block
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    o = h3attn.attn_fwd_blocksparse(*(to_dev_bf16(x, gpu) for x in (q, k, v)), lut, cnt, blk, blk)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    assert np.isfinite(got).all()
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk, blk_k=blk)
    assert_close_absmax(got, ref, what=f"sparse rising max blk={blk}")


def test_sparse_lone_dominant_key(gpu):
    """One kept key out-scores the rest by ~160 (log2 units): rows whose blocks include
    it return its value row."""
    rng = np.random.default_rng(42)
    S, blk = 777, 128
    q = rng.standard_normal((1, 1, S, 128)).astype(np.float32) * 0.1
    k = rng.standard_normal((1, 1, S, 128)).astype(np.float32) * 0.1
    v = rng.standard_normal((1, 1, S, 128)).astype(np.float32)
    q[..., 0] = 64.0
    k[:, :, 500, 0] = 20.0
    q, k, v = (oracle.f32_to_bf16(x) for x in (q, k, v))
    nk = -(-S // blk)
    bmap = np.ones((1, 1, nk, nk), np.uint8)
    bmap[0, 0, 0, 500 // blk] = 0  # the first query block does not see the key
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    o = h3attn.attn_fwd_blocksparse(*(to_dev_bf16(x, gpu) for x in (q, k, v)), lut, cnt, blk, blk)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk, blk_k=blk)
    assert_close_absmax(got, ref, what="sparse lone dominant key")
    vrow = oracle.bf16_to_f32(v).reshape(v.shape)[0, 0, 500]
    assert np.abs(got[0, 0, blk:] - vrow).max() <= 2.0 ** -8 * np.abs(vrow).max()


@pytest.mark.parametrize("blk", [128, 64])
@pytest.mark.parametrize("bad", [-1, 10**6, 2**24 + 5, 2**31 - 1, -2**31, 2**31 // 64])
def test_lut_leading_invalid_entry_changes_nothing(gpu, bad, blk):
    """A LUT row whose first entries name no key block (negative, or a block past the
    keys, up to 2^31 - 1, whose first key would overflow a 32-bit multiply) starts with
    fully masked stages.  The result equals the row without them, bit for bit: the first
    valid stage sets the reference max exactly either way.  Both sparse kernels (pairs
    of 128-row blocks, key-split 64-row blocks)."""
    rng = np.random.default_rng(43)
    S = 1000
    q, k, v = (to_dev_bf16(randn_bf16(rng, (1, 2, S, 128)), gpu) for _ in range(3))
    nq = nk = -(-S // blk)
    kept = [sorted(rng.choice(nk, size=3, replace=False).tolist()) for _ in range(2 * nq)]
    lut_a = torch.tensor([row + [-1, -1] for row in kept], dtype=torch.int32).view(1, 2, nq, 5)
    cnt_a = torch.full((1, 2, nq), 3, dtype=torch.int32)
    lut_b = torch.tensor([[bad, bad] + row for row in kept], dtype=torch.int32).view(1, 2, nq, 5)
    cnt_b = torch.full((1, 2, nq), 5, dtype=torch.int32)
    # unsplit: a split tail would cut the two lists (3 and 5 entries) at different places
    o_a = h3attn.attn_fwd_blocksparse(q, k, v, lut_a.to(gpu), cnt_a.to(gpu), blk, blk, split_tail=False)
    o_b = h3attn.attn_fwd_blocksparse(q, k, v, lut_b.to(gpu), cnt_b.to(gpu), blk, blk, split_tail=False)
    torch.cuda.synchronize()
    assert torch.equal(o_a, o_b)


@pytest.mark.parametrize("blk_q,blk_k,Sq,Skv", [(64, 64, 1, 973), (192, 128, 1, 973), (128, 128, 1, 300),
                                               (256, 64, 1, 500), (96, 96, 1, 700), (32, 48, 1, 333),
                                               (64, 64, 300, 1), (128, 128, 130, 1), (96, 32, 200, 1)])
def test_length_one_sequences(gpu, blk_q, blk_k, Sq, Skv):
    """One query row or one key, B=2, H=2, against the masked oracle, on the native kernels
    (64/128/192/256) and the tile path (other sizes).  A size-1 dimension's stride reaches the
    library as 0; the kernels step past the end of the sequence (whole O tiles, whole K/V
    stages) and those rows must still be dropped, not land on row 0."""
    rng = np.random.default_rng(blk_q + 7 * blk_k + Sq + Skv)
    B, H = 2, 2
    q = randn_bf16(rng, (B, H, Sq, 128))
    k = randn_bf16(rng, (B, H, Skv, 128))
    v = randn_bf16(rng, (B, H, Skv, 128), scale=4.0)
    nq, nk = -(-Sq // blk_q), -(-Skv // blk_k)
    bmap = (rng.random((B, H, nq, nk)) < 0.6).astype(np.uint8)
    bmap[..., 0] = 1
    qd, kd, vd = (to_dev_bf16(x, gpu) for x in (q, k, v))
    bt = torch.from_numpy(bmap).to(gpu)
    if blk_q in ops.NATIVE_BLOCKS and blk_k in ops.NATIVE_BLOCKS:
        lut, cnt = h3attn.block_map_to_lut(bt)
        o = h3attn.attn_fwd_blocksparse(qd, kd, vd, lut, cnt, blk_q, blk_k)
    else:
        tl, tc = ops.block_map_to_tile_lut(bt, blk_q, blk_k, Sq, Skv)
        o = ops.attn_fwd_blocksparse_tiles(qd, kd, vd, tl, tc)
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk_q, blk_k=blk_k)
    assert_close_absmax(got, ref, what=f"blk=({blk_q},{blk_k}) Sq={Sq} Skv={Skv}")


def test_empty_rows_give_zero(gpu):
    rng = np.random.default_rng(22)
    q, k, v = (to_dev_bf16(randn_bf16(rng, (1, 1, 256, 128)), gpu) for _ in range(3))
    bmap = torch.zeros(1, 1, 2, 2, dtype=torch.uint8, device=gpu)
    bmap[0, 0, 1, 1] = 1
    lut, cnt = h3attn.block_map_to_lut(bmap, 1)
    o = h3attn.attn_fwd_blocksparse(q, k, v, lut, cnt, 128, 128)
    torch.cuda.synchronize()
    assert torch.all(o[0, 0, :128] == 0)
    assert torch.all(torch.isfinite(o.float()))


def test_gpu_block_map_matches_oracle(gpu):
    """GPU block map (pool + select) vs the oracle: identical except at fp32-level score ties."""
    rng = np.random.default_rng(23)
    S, H, blk = 2000, 2, 128
    q, k = randn_bf16(rng, (1, H, S, 128)), randn_bf16(rng, (1, H, S, 128))
    nk = -(-S // blk)
    keep = sla.keep_count(0.25, nk)
    ref, scores = oracle.block_map(q, k, blk, blk, keep=keep, force_diag=True, return_scores=True)
    bmap, lut, cnt = sla.get_block_map(to_dev_bf16(q, gpu), to_dev_bf16(k, gpu), 0.25, blk, blk,
                                       force_diag=True, smooth_k=False)
    got = bmap.cpu().numpy()
    diff = np.argwhere(got != ref)
    for b, h, i, j in diff:  # any disagreement must sit at the selection threshold
        row = np.sort(scores[b, h, i])[::-1]
        thr = row[keep - 1]
        assert abs(scores[b, h, i, j] - thr) <= 1e-4 * max(1.0, abs(thr))
    assert np.array_equal(cnt.cpu().numpy(), got.sum(-1))


def test_block_pool_matches_means(gpu):
    """GPU block means over valid rows (partial last block), strided input."""
    rng = np.random.default_rng(24)
    S, H, blk = 1000, 3, 128
    x = randn_bf16(rng, (1, S, H, 128))                     # [B,S,H,D] memory
    xd = to_dev_bf16(x, gpu).transpose(1, 2)                 # [B,H,S,D] view
    got = ops.block_pool(xd, blk).cpu().numpy()
    xf = oracle.bf16_to_f32(x).reshape(x.shape).transpose(0, 2, 1, 3).astype(np.float64)
    nb = -(-S // blk)
    want = np.stack([xf[:, :, j * blk:min(S, (j + 1) * blk)].mean(2) for j in range(nb)], 2)
    assert np.abs(got - want).max() <= 1e-5


@pytest.mark.parametrize("blk,keep,diag", [(128, 3, True), (64, 5, False), (64, 1, True)])
def test_block_select_matches_oracle(gpu, blk, keep, diag):
    """Selection (rank by score, ties to the lower index, optional diagonal) vs the oracle."""
    rng = np.random.default_rng(25 + blk + keep)
    S, H = 1500, 2
    q, k = randn_bf16(rng, (1, H, S, 128)), randn_bf16(rng, (1, H, S, 128))
    ref, scores = oracle.block_map(q, k, blk, blk, keep=keep, force_diag=diag, return_scores=True)
    pq = ops.block_pool(to_dev_bf16(q, gpu), blk)
    pk = ops.block_pool(to_dev_bf16(k, gpu), blk)
    bmap, lut, cnt = ops.block_select(pq, pk, keep, blk, blk, force_diag=diag)
    got = bmap.cpu().numpy()
    for b, h, i, j in np.argwhere(got != ref):  # only fp32-vs-fp64 near-ties may differ
        thr = np.sort(scores[b, h, i])[::-1][keep - 1]
        assert abs(scores[b, h, i, j] - thr) <= 1e-4 * max(1.0, abs(thr))
    rl, rc = _lut_np(got, lut.shape[-1])
    assert np.array_equal(cnt.cpu().numpy(), rc)
    assert np.array_equal(lut.cpu().numpy(), rl)


def _select_ref(pq, pk, keep, blk_q, blk_k, diag, max_k):
    """Selection from exact scores: rank by (score desc, index asc), keep the first
    `keep` plus the diagonal, list them ascending, truncate to max_k."""
    B, H, nq, _ = pq.shape
    nk = pk.shape[2]
    sc = np.einsum("bhid,bhjd->bhij", pq.astype(np.float64), pk.astype(np.float64))
    bmap = np.zeros((B, H, nq, nk), np.uint8)
    lut = np.full((B, H, nq, max_k), -1, np.int32)
    cnt = np.zeros((B, H, nq), np.int32)
    for b, h, i in np.ndindex(B, H, nq):
        order = np.lexsort((np.arange(nk), -sc[b, h, i]))  # score desc, then index asc
        kept = set(order[:keep].tolist())
        if diag and i * blk_q // blk_k < nk:
            kept.add(i * blk_q // blk_k)
        kept = sorted(kept)
        bmap[b, h, i, kept] = 1
        cnt[b, h, i] = min(len(kept), max_k)
        lut[b, h, i, :cnt[b, h, i]] = kept[:max_k]
    return bmap, lut, cnt


@pytest.mark.parametrize("nq,nk,diag", [(40, 1025, True), (33, 2633, False), (17, 3072, True)])
def test_block_select_long_rows_real_scores(gpu, nq, nk, diag):
    """Rows of 1025-3072 key blocks (the 8- and 16-wave workgroups) on real-valued pooled vectors
    against a float64 selection: the kept set may differ only where a score is within
    fp32 rounding of the keep-th largest; the LUT and counts follow the map."""
    rng = np.random.default_rng(nq + nk)
    keep = nk // 4
    pq = rng.standard_normal((1, 2, nq, 128)).astype(np.float32)
    pk = rng.standard_normal((1, 2, nk, 128)).astype(np.float32)
    bmap, lut, cnt = ops.block_select(torch.from_numpy(pq).to(gpu), torch.from_numpy(pk).to(gpu), keep,
                                      16, 16, force_diag=diag)
    rmap, _, _ = _select_ref(pq, pk, keep, 16, 16, diag, lut.shape[-1])
    got = bmap.cpu().numpy()
    sc = np.einsum("bhid,bhjd->bhij", pq.astype(np.float64), pk.astype(np.float64))
    diff = np.argwhere(got != rmap)
    assert len(diff) <= 4 * nq, len(diff)
    for b, h, i, j in diff:
        thr = np.sort(sc[b, h, i])[::-1][keep - 1]
        assert abs(sc[b, h, i, j] - thr) <= 1e-4 * max(1.0, abs(thr)), (b, h, i, j)
    rl, rc = _lut_np(got, lut.shape[-1])
    assert np.array_equal(cnt.cpu().numpy(), rc)
    assert np.array_equal(lut.cpu().numpy(), rl)


@pytest.mark.parametrize("nq,nk,keep,diag,max_k", [
    (9, 700, 37, True, 38), (17, 65, 1, False, 1), (1, 64, 64, False, 64), (9, 1, 1, True, 1),
    (17, 700, 100, True, 50), (16, 200, 20, False, 20), (5, 384, 96, True, 97),
    (3, 769, 10, False, 10), (5, 1000, 150, True, 151), (17, 1024, 100, True, 101),
    (17, 1025, 60, False, 60), (9, 1536, 200, True, 201), (5, 1537, 30, False, 30),
    (33, 2000, 90, True, 91), (6, 2500, 300, True, 301), (4, 3072, 64, False, 64),
    (4, 3073, 10, True, 11), (3, 5000, 40, True, 41), (2, 7000, 100, False, 100)])
def test_block_select_exact_ties(gpu, nq, nk, keep, diag, max_k):
    """Integer pooled vectors make every score an exact fp32 integer, with many ties:
    the kept set, its order and the truncation to max_k_blocks must match exactly.
    Covers row groups of up to 16 query blocks per workgroup (fewer where the score
    rows fill LDS: 14 at nk 700, 13 at 1536 in the 8-wave form, 13 at 3072 in the 16-wave
    form, 3 at 3073, 2 at 5000, 1 at the 7000 maximum; the score MFMAs' rows past a
    group's end are computed and dropped), partial last groups (nq 17, 33), key tiles
    past nk (nk 65, 1, 769, 1000, 1025, 1537, 2500, 3073), and all four counting paths,
    each at its boundaries: keys held in registers, 4 rows per wave of a 4-wave
    workgroup in 6 (nk <= 384) or 12 (nk <= 768), 2 rows per wave of an 8-wave one in 24
    (nk 769-1536), 1 row per wave of a 16-wave one in 48 (nk 1537-3072), and re-read
    from LDS (3073 and above)."""
    rng = np.random.default_rng(50 + nq + nk)
    pq = rng.integers(-2, 3, (1, 2, nq, 128)).astype(np.float32)
    pk = rng.integers(-2, 3, (1, 2, nk, 128)).astype(np.float32)
    bmap, lut, cnt = ops.block_select(torch.from_numpy(pq).to(gpu), torch.from_numpy(pk).to(gpu), keep,
                                      128, 128, force_diag=diag, max_k_blocks=max_k)
    rmap, rlut, rcnt = _select_ref(pq, pk, keep, 128, 128, diag, max_k)
    assert np.array_equal(bmap.cpu().numpy(), rmap)
    assert np.array_equal(cnt.cpu().numpy(), rcnt)
    assert np.array_equal(lut.cpu().numpy(), rlut)


@pytest.mark.parametrize("blk", [128, 64])
def test_sparse_h56_s42120_full_shape(gpu, blk):
    """H=56, S=42120, top 25 % + diagonal: the H3 sparse workload at 128x128 tiles, and at
    the SLA default 64x64 (key-split workgroups, 164-165 key blocks per row).  Checked on
    2 heads, on the first, a middle and the last (partial) query block."""
    S, H = 42120, 56
    g = torch.Generator(device=gpu).manual_seed(5)
    q = torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    k = torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    v = torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) * 4
    bmap, lut, cnt = sla.get_block_map(q, k, 0.25, blk, blk, force_diag=True, smooth_k=False)
    nq = -(-S // blk)
    keep = int(0.25 * nq)
    assert keep <= int(cnt.min()) and int(cnt.max()) <= keep + 1
    o = h3attn.attn_fwd_blocksparse(q, k, v, lut, cnt, blk, blk)
    torch.cuda.synchronize()
    scale = 1.0 / math.sqrt(128)
    for h in (0, 55):
        kt = k[0, h].float().t().contiguous()
        vf = v[0, h].float()
        kept = bmap[0, h].bool()  # [nq, nk]
        for i0 in (0, 20480, (nq - 1) * blk):
            i1 = min(i0 + blk, S)
            qi = q[0, h, i0:i1].float()
            s = (qi @ kt) * scale
            mask = kept[i0 // blk].repeat_interleave(blk)[:S]
            s = s.masked_fill(~mask, float("-inf"))
            ref = torch.softmax(s, -1) @ vf
            assert_close_absmax(o[0, h, i0:i1].float().cpu().numpy(), ref.cpu().numpy(),
                                what=f"blk={blk} h={h} q0={i0}")


@pytest.mark.parametrize("blk", [128, 64, 256, 192])
def test_sparse_queued_matches_one_pair_per_workgroup(gpu, blk):
    """Four rounds of query-block pairs and more run on a persistent grid that takes pairs
    from per-XCD queues (h3a_attn_fwd_blocksparse_ws, 1 KiB of counters in the workspace).
    Without a split tail each pair's arithmetic is that of the one-pair-per-workgroup
    launch, so with uneven and empty lists the outputs are equal bit for bit."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rows = 128 if blk % 128 == 0 else 64  # query sub-block height of the kernel
    B, H, S = 4, max(cus // 4, 1), 8 * rows  # 4 pairs per head: 4 * CUs pairs, no remainder
    nq = nk = -(-S // blk)
    rng = np.random.default_rng(31 + blk)
    bmap = (rng.random((B, H, nq, nk)) < 0.5).astype(np.uint8)
    bmap[:, :, 0] = 0  # empty lists
    bmap[0, 0, -1] = 1  # a full one
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    assert ops.sparse_workspace_bytes(B, H, S, S, blk, blk, lut.shape[3]) == 1024
    g = torch.Generator(device=gpu).manual_seed(blk)
    q, k, v = (torch.randn(B, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    want = ops.attn_fwd_blocksparse(q, k, v, lut, cnt, blk, blk, split_tail=False)
    got = ops.attn_fwd_blocksparse(q, k, v, lut, cnt, blk, blk)
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"blk={blk}: queued dispatch differs from one pair per workgroup"
    assert not got[:, :, :blk].any(), "rows of empty lists must be 0"


# ----------------------------------------------------------------------------- tile LUTs (other block sizes)
TILE_SIZES = [16, 32, 48, 80, 96, 112, 144, 160, 176, 208, 224, 240]


def _tile_lut_np(bmap, blk_q, blk_k, Sq, Skv):
    """Restatement of the tile LUT on the CPU: per 64-row query sub-block, the ascending 32-key
    columns with a kept (query block, key block) pair, as column << 8 | mask with bit 2*i + j
    for rows 16i.. of the sub-block and keys 16j.. of the column."""
    B, H, nq, nk = bmap.shape
    nsub, ncol = -(-Sq // 64), -(-Skv // 32)
    rows = {}
    for b, h, qs in np.ndindex(B, H, nsub):
        ents = []
        for c in range(ncol):
            mask = 0
            for i in range(4):
                r = 64 * qs + 16 * i
                if r >= Sq:
                    continue
                for j in range(2):
                    key = 32 * c + 16 * j
                    if key < Skv and bmap[b, h, r // blk_q, key // blk_k]:
                        mask |= 1 << (2 * i + j)
            if mask:
                ents.append((c << 8) | mask)
        rows[(b, h, qs)] = ents
    return rows


def _check_tile_lut(tlut, tcnt, want):
    tl, tc = tlut.cpu().numpy(), tcnt.cpu().numpy()
    for idx, ents in want.items():
        n = len(ents)
        assert tc[idx] == n, (idx, tc[idx], n)
        assert list(tl[idx][:n]) == ents, idx
        assert (tl[idx][n:] == -1).all(), idx


@pytest.mark.parametrize("blk", TILE_SIZES)
def test_sparse_tile_sizes_vs_masked_oracle(gpu, blk):
    """Block sizes the native kernels do not take (the h3_sla node's other sizes,
    custom_nodes/h3_sla/__init__.py:315): the block map becomes a tile LUT, equal to the CPU
    restatement entry for entry, and the tile kernel's output equals the masked oracle."""
    rng = np.random.default_rng(300 + blk)
    S, H = 700 + blk, 2
    q, k, v = (randn_bf16(rng, (1, H, S, 128)) for _ in range(3))
    nk = -(-S // blk)
    bmap = oracle.block_map(q, k, blk, blk, keep=max(1, nk // 4), force_diag=True)
    tlut, tcnt = ops.block_map_to_tile_lut(torch.from_numpy(bmap).to(gpu), blk, blk, S, S)
    _check_tile_lut(tlut, tcnt, _tile_lut_np(bmap, blk, blk, S, S))
    o = ops.attn_fwd_blocksparse_tiles(*(to_dev_bf16(x, gpu) for x in (q, k, v)), tlut, tcnt)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk, blk_k=blk)
    assert_close_absmax(got, ref, what=f"tiles blk={blk}")


@pytest.mark.parametrize("blk_q,blk_k,Sq,Skv", [(32, 64, 640, 900), (64, 32, 900, 640), (96, 128, 1000, 1000),
                                                (48, 208, 777, 1300), (256, 16, 1111, 500), (16, 256, 500, 1111),
                                                (160, 224, 1500, 1501)])
def test_sparse_tile_mixed_sizes_from_lut(gpu, blk_q, blk_k, Sq, Skv):
    """attn_fwd_blocksparse with a block LUT at sizes outside the native ones, query and key blocks
    different and Sq != Skv: LUT -> block map -> tile LUT -> tile kernel, against the masked
    oracle; the map is also compared with the LUT it came from."""
    rng = np.random.default_rng(blk_q * 1000 + blk_k + Sq)
    H = 2
    q = randn_bf16(rng, (1, H, Sq, 128))
    k, v = (randn_bf16(rng, (1, H, Skv, 128)) for _ in range(2))
    nk = -(-Skv // blk_k)
    bmap = oracle.block_map(q, k, blk_q, blk_k, keep=max(1, nk // 3), force_diag=False)
    bmap[0, 1, 0] = 0  # a query block with no kept key block: its rows come out 0
    lut, cnt = h3attn.block_map_to_lut(torch.from_numpy(bmap).to(gpu))
    assert np.array_equal(ops.lut_to_block_map(lut, cnt, nk).cpu().numpy(), bmap)
    o = h3attn.attn_fwd_blocksparse(*(to_dev_bf16(x, gpu) for x in (q, k, v)), lut, cnt, blk_q, blk_k)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk_q, blk_k=blk_k)
    assert_close_absmax(got, ref, what=f"tiles blk_q={blk_q} blk_k={blk_k}")
    assert not got[0, 1, :blk_q].any()


@pytest.mark.parametrize("blk", [32, 96])
def test_sla_sparse_attention_at_tile_sizes(gpu, blk):
    """sla.sparse_attention end to end at a tile size (pool, select, tile LUT, tile kernel), with
    the block map checked against the oracle's pooled top-k at the same keep."""
    rng = np.random.default_rng(77 + blk)
    S, H, keep = 1200, 3, 0.25
    q, k, v = (randn_bf16(rng, (1, H, S, 128)) for _ in range(3))
    nk = -(-S // blk)
    bmap = oracle.block_map(q, k, blk, blk, keep=sla.keep_count(keep, nk), force_diag=False)
    qd, kd, vd = (to_dev_bf16(x, gpu) for x in (q, k, v))
    gmap, _, _ = sla.get_block_map(qd, kd, keep, blk, blk)
    assert np.array_equal(gmap.cpu().numpy(), bmap)
    o = sla.sparse_attention(qd, kd, vd, keep, blk)
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    ref = oracle.attn_fwd(q, k, v, block_map=bmap, blk_q=blk, blk_k=blk)
    assert_close_absmax(got, ref, what=f"sla blk={blk}")


@pytest.mark.parametrize("B,H,S,blk", [(1, 2, 1950, 96), (1, 3, 4100, 80), (1, 40, 8192, 112), (1, 1, 64, 48),
                                       (3, 2, 3000, 144)])
def test_sparse_tiles_pair_map(gpu, B, H, S, blk):
    """The workspace entry point pairs 64-row sub-blocks by stage count (tile_pair_map_kernel);
    the plain one pairs 2p and 2p+1.  Every row's arithmetic is the same either way, so the two
    outputs are equal bit for bit, over outputs pre-filled with different values so that a
    sub-block left out or run twice shows.  Block heights that put block boundaries inside
    some sub-blocks (80, 96, 112, 144: lists of unequal length), an odd sub-block count (1950:
    31, 64: 1), a static launch with the map and a queued one (H=40, S=8192), B=3, and the
    masked oracle on the first 192 rows of one head of the last batch."""
    rng = np.random.default_rng(90 + blk)
    g = torch.Generator(device=gpu).manual_seed(90 + blk)
    q, k, v = (torch.randn(B, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    nb = -(-S // blk)
    bmap_np = (rng.random((B, H, nb, nb)) < 0.25).astype(np.uint8)
    bmap_np[..., np.arange(nb), np.arange(nb)] = 1
    tlut, tcnt = ops.block_map_to_tile_lut(torch.from_numpy(bmap_np).to(gpu), blk, blk, S, S)
    nsub = -(-S // 64)
    assert ops.tiles_workspace_bytes(B, H, S, S, tlut.shape[3]) >= 8 * B * H * ((nsub + 1) // 2)
    a = torch.full_like(q, 1000.0)
    b = torch.full_like(q, -1000.0)
    ops.attn_fwd_blocksparse_tiles(q, k, v, tlut, tcnt, out=a, queues=True)
    ops.attn_fwd_blocksparse_tiles(q, k, v, tlut, tcnt, out=b, queues=False)
    assert torch.equal(a, b)
    bb, h, rows = B - 1, H - 1, min(192, S)
    nr = -(-rows // blk)
    qh = from_dev_bf16(q[bb:bb + 1, h:h + 1, :rows])
    kh, vh = (from_dev_bf16(t[bb:bb + 1, h:h + 1]) for t in (k, v))
    ref = oracle.attn_fwd(qh, kh, vh, block_map=bmap_np[bb:bb + 1, h:h + 1, :nr], blk_q=blk, blk_k=blk)
    got = oracle.bf16_to_f32(from_dev_bf16(a[bb:bb + 1, h:h + 1, :rows])).reshape(ref.shape)
    assert_close_absmax(got, ref, what=f"tiles pair map blk {blk}")


@pytest.mark.parametrize("extra", [0, 1])
def test_sparse_tiles_pair_map_limit(gpu, extra):
    """Up to 16384 sub-blocks per (b,h) the workspace holds the pair map (8 bytes a pair) and
    the queue counters; one more and the pairs stay consecutive (counters only).  At the
    limit (S = 64 * 16384, the sort over 16384 sub-blocks of random lengths) and just past
    it (S = 64 * 16384 + 1), the queued call equals the plain one bit for bit and fp32
    attention on rows of the first, a middle and the last sub-block.  Sub-block s lists
    its own diagonal column 2s with rows 0-31 admitted, and 0-3 more columns 2s+1 .. with
    no row admitted (they load and mask a whole column), so list lengths differ."""
    lim = 64 * 16384
    S = lim + extra
    nbytes = ops.tiles_workspace_bytes(1, 1, S, S, 4)
    if extra:
        assert 0 < nbytes < 8 * 8192
    else:
        assert nbytes >= 8 * 8192
    nsub = -(-S // 64)
    g = torch.Generator(device=gpu).manual_seed(17 + extra)
    q, k, v = (torch.randn(1, 1, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    sb = torch.arange(nsub, device=gpu, dtype=torch.int32).view(1, 1, nsub, 1)
    ncol = -(-S // 32)
    cols = torch.clamp(2 * sb + torch.arange(4, device=gpu, dtype=torch.int32).view(1, 1, 1, 4), max=ncol - 1)
    lut = (cols << 8).contiguous()
    lut[..., 0] |= 0xf  # the diagonal column: rows 0-31 of the sub-block against its 32 keys
    cnt = torch.randint(1, 5, (1, 1, nsub), generator=g, device=gpu, dtype=torch.int32)
    a = torch.full_like(q, 7.0)
    b = torch.full_like(q, -7.0)
    ops.attn_fwd_blocksparse_tiles(q, k, v, lut, cnt, out=a, queues=True)
    ops.attn_fwd_blocksparse_tiles(q, k, v, lut, cnt, out=b, queues=False)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    scale = 1.0 / math.sqrt(128)
    for s in (0, nsub // 2, nsub - 1):
        r0 = 64 * s
        rows = min(32, S - r0)
        kk, vv = k[0, 0, r0:r0 + 32].float(), v[0, 0, r0:r0 + 32].float()
        p = torch.softmax((q[0, 0, r0:r0 + rows].float() @ kk.t().contiguous()) * scale, -1)
        ref = p @ vv
        got = a[0, 0, r0:r0 + rows].float()
        assert (got - ref).abs().max().item() <= 2e-2 * ref.abs().max().item() + 1e-3, s
        if r0 + 32 < S:  # rows 32-63 see no key: O = 0
            assert torch.count_nonzero(a[0, 0, r0 + 32:r0 + 64]).item() == 0


def test_sparse_tiles_queued_matches_static(gpu):
    """The tile kernel through the per-XCD work queues (enough pairs for a persistent grid) equals
    the statically dispatched launch bit for bit, and the masked oracle on one head."""
    rng = np.random.default_rng(5)
    S, H, blk = 8192, 40, 32  # 2560 pairs of 64-row sub-blocks: four rounds or more on 256 CUs
    g = torch.Generator(device=gpu).manual_seed(5)
    q, k, v = (torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
    nk = S // blk
    bmap_np = (rng.random((1, H, nk, nk)) < 0.2).astype(np.uint8)
    tlut, tcnt = ops.block_map_to_tile_lut(torch.from_numpy(bmap_np).to(gpu), blk, blk, S, S)
    pairs = H * ((S // 64 + 1) // 2)
    assert ops.tiles_workspace_bytes(1, H, S, S, tlut.shape[3]) > 8 * pairs  # pair map + queue counters
    a = ops.attn_fwd_blocksparse_tiles(q, k, v, tlut, tcnt, queues=True)
    b = ops.attn_fwd_blocksparse_tiles(q, k, v, tlut, tcnt, queues=False)
    assert torch.equal(a, b)
    h, rows = 7, 128  # the oracle on the first 128 query rows of one head
    qh = from_dev_bf16(q[:, h:h + 1, :rows])
    kh, vh = (from_dev_bf16(t[:, h:h + 1]) for t in (k, v))
    ref = oracle.attn_fwd(qh, kh, vh, block_map=bmap_np[:, h:h + 1, :rows // blk], blk_q=blk, blk_k=blk)
    got = oracle.bf16_to_f32(from_dev_bf16(a[:, h:h + 1, :rows])).reshape(ref.shape)
    assert_close_absmax(got, ref, what="tiles queued")
