"""Pin the CPU oracle (oracle/h3_oracle.c) before it is trusted as the checker.

Each oracle function is checked against (a) the golden fixtures written by
tests/golden/make_golden.py from torch fp64 code paths independent of the
oracle, and (b) what the mathematics fixes: closed forms, special cases and
invariants chosen so that a dropped term, a wrong sign, a transposed operand
or an off-by-one block index fails.
"""
from __future__ import annotations

import glob
import math
import os

import numpy as np
import pytest

import oracle
from conftest import assert_close_absmax, randn_bf16

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def f32(bits):
    return oracle.bf16_to_f32(bits).reshape(bits.shape).astype(np.float64)


# ----------------------------------------------------------------------------- attention
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "attn_[0-9]*.npz"))))
def test_attn_matches_golden_sdpa(path):
    z = np.load(path)
    exact = oracle.attn_fwd(z["q"], z["k"], z["v"], round_p=False)
    assert np.abs(exact - z["o"]).max() <= 1e-6 * max(1.0, np.abs(z["o"]).max())
    rounded = oracle.attn_fwd(z["q"], z["k"], z["v"], round_p=True)
    assert_close_absmax(rounded, z["o"], what=os.path.basename(path))


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "attn_masked_*.npz"))))
def test_block_masked_attn_matches_golden(path):
    z = np.load(path)
    blk = int(z["blk"])
    o = oracle.attn_fwd(z["q"], z["k"], z["v"], round_p=False, block_map=z["block_map"], blk_q=blk, blk_k=blk)
    assert np.abs(o - z["o"]).max() <= 1e-6


def test_attn_two_keys_closed_form():
    """q.k1 and q.k2 set by hand; O = w1 v1 + w2 v2 with the exact softmax weights."""
    q = np.zeros((1, 1, 1, 128), np.float32)
    k = np.zeros((1, 1, 2, 128), np.float32)
    v = np.zeros((1, 1, 2, 128), np.float32)
    q[..., 0] = 2.0
    k[0, 0, 0, 0], k[0, 0, 1, 0] = 3.0, -1.0
    v[0, 0, 0, :] = 1.0
    v[0, 0, 1, :] = np.arange(128) / 64.0
    o = oracle.attn_fwd(*(oracle.f32_to_bf16(x) for x in (q, k, v)), round_p=False)
    s1, s2 = 6.0 / math.sqrt(128), -2.0 / math.sqrt(128)
    w1 = 1.0 / (1.0 + math.exp(s2 - s1))
    want = w1 * 1.0 + (1 - w1) * (np.arange(128) / 64.0)
    assert np.abs(o[0, 0, 0] - want).max() < 1e-6


def test_attn_scale_argument_is_used():
    rng = np.random.default_rng(3)
    q, k, v = (randn_bf16(rng, (1, 1, 5, 128)) for _ in range(3))
    a = oracle.attn_fwd(q, k, v, scale=0.0, round_p=False)  # scale 0 -> uniform weights -> mean of V
    assert np.abs(a - f32(v).mean(axis=2, keepdims=True)).max() < 1e-6


def test_attn_single_key_and_constant_value():
    rng = np.random.default_rng(4)
    q, k, v = randn_bf16(rng, (1, 2, 9, 128)), randn_bf16(rng, (1, 2, 1, 128)), randn_bf16(rng, (1, 2, 1, 128))
    o = oracle.attn_fwd(q, k, v)
    assert np.array_equal(o, np.broadcast_to(f32(v), o.shape).astype(np.float32))
    k2 = randn_bf16(rng, (1, 2, 40, 128))
    vc = oracle.f32_to_bf16(np.full((1, 2, 40, 128), -0.75, np.float32))
    assert np.abs(oracle.attn_fwd(q, k2, vc, round_p=False) + 0.75).max() < 1e-6


def test_attn_permutation_invariance():
    rng = np.random.default_rng(5)
    q, k, v = (randn_bf16(rng, (1, 1, 30, 128)) for _ in range(3))
    p = rng.permutation(30)
    a = oracle.attn_fwd(q, k, v, round_p=False)
    b = oracle.attn_fwd(q, k[:, :, p], v[:, :, p], round_p=False)
    assert np.abs(a - b).max() < 1e-6


def test_attn_strided_equals_contiguous():
    rng = np.random.default_rng(6)
    q, k, v = (randn_bf16(rng, (1, 11, 3, 128)) for _ in range(3))  # [B,S,H,D] memory
    tq, tk, tv = (x.transpose(0, 2, 1, 3) for x in (q, k, v))      # [B,H,S,D] views
    a = oracle.attn_fwd(tq, tk, tv)
    b = oracle.attn_fwd(np.ascontiguousarray(tq), np.ascontiguousarray(tk), np.ascontiguousarray(tv))
    assert np.array_equal(a, b)


def test_full_block_map_equals_dense_and_empty_row_is_zero():
    rng = np.random.default_rng(7)
    q, k, v = (randn_bf16(rng, (1, 1, 150, 128)) for _ in range(3))
    dense = oracle.attn_fwd(q, k, v)
    full = oracle.attn_fwd(q, k, v, block_map=np.ones((1, 1, 3, 3), np.uint8), blk_q=64, blk_k=64)
    assert np.array_equal(dense, full)
    bm = np.ones((1, 1, 3, 3), np.uint8)
    bm[0, 0, 1] = 0
    o = oracle.attn_fwd(q, k, v, block_map=bm, blk_q=64, blk_k=64)
    assert np.all(o[0, 0, 64:128] == 0)
    assert np.array_equal(o[0, 0, :64], dense[0, 0, :64])


def test_diagonal_only_map_is_local_attention():
    """Diagonal-only block map == attention restricted to each block (a brute-force restatement)."""
    rng = np.random.default_rng(8)
    S, blk = 200, 64
    q, k, v = (randn_bf16(rng, (1, 1, S, 128)) for _ in range(3))
    nb = -(-S // blk)
    bm = np.eye(nb, dtype=np.uint8)[None, None]
    o = oracle.attn_fwd(q, k, v, block_map=bm, blk_q=blk, blk_k=blk, round_p=False)
    for b0 in range(0, S, blk):
        sl = slice(b0, min(S, b0 + blk))
        loc = oracle.attn_fwd(q[:, :, sl], k[:, :, sl], v[:, :, sl], round_p=False)
        assert np.abs(o[:, :, sl] - loc).max() < 1e-6


# ----------------------------------------------------------------------------- prologue
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "prologue_*.npz"))))
def test_prologue_matches_golden(path):
    z = np.load(path)
    S, H = z["q"].shape[0], z["q"].shape[1]
    rot = int(z["rot"])
    rope = oracle.rope_table(S, rot, float(z["theta"])) if rot else None
    gq, gk = oracle.qk_rmsnorm_rope(z["q"][None], z["k"][None], rope, z["qw"], z["kw"],
                                    eps=float(z["eps"]), rot_dim=rot)
    for got, want in ((gq[0], z["q_out"]), (gk[0], z["k_out"])):
        g, w = f32(got), f32(want)
        assert np.all(np.abs(g - w) <= np.abs(w) * 2.0 ** -7 + 1e-30)  # <= 1 bf16 ulp
        assert np.mean(got == want) >= 0.99


def _unit_rows(S, H, rot):
    x = np.zeros((1, S, H, 128), np.float32)
    return x


def test_prologue_position_zero_is_plain_rmsnorm():
    rng = np.random.default_rng(9)
    x = randn_bf16(rng, (1, 1, 2, 128), scale=3.0)
    w = oracle.f32_to_bf16(np.ones(128, np.float32))
    rope = oracle.rope_table(1, 128)
    q, _ = oracle.qk_rmsnorm_rope(x, x, rope, w, w, eps=0.0)
    xf = f32(x)
    want = xf / np.sqrt((xf ** 2).mean(-1, keepdims=True))
    assert np.abs(f32(q) - want).max() <= 2.0 ** -7 * np.abs(want).max()


def test_prologue_split_half_pairing_and_sign():
    """A unit vector at dim i (< rot/2) rotates into dims i (cos) and i+rot/2 (+sin)."""
    S, rot, i = 3, 64, 5
    x = np.zeros((1, S, 1, 128), np.float32)
    x[..., i] = 1.0
    xb = oracle.f32_to_bf16(x)
    w = oracle.f32_to_bf16(np.ones(128, np.float32))
    q, _ = oracle.qk_rmsnorm_rope(xb, xb, oracle.rope_table(S, rot), w, w, eps=0.0, rot_dim=rot)
    qf = f32(q)[0, :, 0]
    nrm = math.sqrt(128.0)  # rmsnorm of a unit vector scales it by sqrt(D)
    for s in range(S):
        ang = s * 10000.0 ** (-2.0 * i / rot)
        assert abs(qf[s, i] - nrm * math.cos(ang)) <= 2 ** -7 * nrm
        assert abs(qf[s, i + rot // 2] - nrm * math.sin(ang)) <= 2 ** -7 * nrm
        others = np.delete(qf[s], [i, i + rot // 2])
        assert np.all(others == 0)


def test_prologue_rotation_preserves_pair_norms_and_relative_position():
    rng = np.random.default_rng(10)
    S, rot = 40, 128
    base = rng.standard_normal(128).astype(np.float32)
    x = oracle.f32_to_bf16(np.broadcast_to(base, (1, S, 1, 128)).copy())
    w = oracle.f32_to_bf16(np.ones(128, np.float32))
    q, _ = oracle.qk_rmsnorm_rope(x, x, oracle.rope_table(S, rot), w, w, eps=1e-6)
    qf = f32(q)[0, :, 0]
    h = rot // 2
    pair = qf[:, :h] ** 2 + qf[:, h:rot] ** 2
    assert np.abs(pair - pair[0]).max() <= 1e-2 * pair.max()
    # <rope(x, m), rope(x, n)> depends only on m - n
    d1 = qf[3] @ qf[10]
    d2 = qf[20] @ qf[27]
    assert abs(d1 - d2) <= 1e-2 * abs(qf[0] @ qf[0])


# ----------------------------------------------------------------------------- block map
@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "blockmap_*.npz"))))
def test_block_map_matches_golden(path):
    z = np.load(path)
    blk = int(z["blk"])
    m = oracle.block_map(z["q"], z["k"], blk, blk, keep=int(z["keep"]), force_diag=bool(z["force_diag"]))
    assert np.array_equal(m, z["block_map"])


def test_block_map_selects_the_top_scores():
    rng = np.random.default_rng(11)
    q, k = randn_bf16(rng, (1, 2, 500, 128)), randn_bf16(rng, (1, 2, 470, 128))
    keep = 3
    m, sc = oracle.block_map(q, k, 64, 64, keep=keep, force_diag=False, return_scores=True)
    assert np.all(m.sum(-1) == keep)
    kept = np.where(m == 1, sc, np.inf).min(-1)
    dropped = np.where(m == 0, sc, -np.inf).max(-1)
    assert np.all(kept >= dropped)
    # pooled score of block (i,j) is the mean over the valid rows (last blocks are partial)
    qf, kf = f32(q)[0, 1], f32(k)[0, 1]
    want = qf[448:500].mean(0) @ kf[448:470].mean(0)
    assert abs(sc[0, 1, 7, 7] - want) <= 1e-9 * max(1.0, abs(want))


def test_block_map_forced_diagonal_and_smoothing():
    rng = np.random.default_rng(12)
    q, k = randn_bf16(rng, (1, 1, 640, 128)), randn_bf16(rng, (1, 1, 640, 128))
    m = oracle.block_map(q, k, 128, 64, keep=1, force_diag=True)
    for i in range(m.shape[2]):
        assert m[0, 0, i, (i * 128) // 64] == 1
    # centring k shifts every score of a row by the same amount -> same selection
    m1, s1 = oracle.block_map(q, k, 64, 64, keep=2, force_diag=False, return_scores=True)
    m2, s2 = oracle.block_map(q, k, 64, 64, keep=2, force_diag=False, smooth_k=True, return_scores=True)
    assert np.array_equal(m1, m2)
    shift = s1 - s2
    assert np.abs(shift - shift[..., :1]).max() <= 1e-9 * np.abs(s1).max()
