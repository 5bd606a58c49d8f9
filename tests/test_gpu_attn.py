"""Parity of the dense gfx950 attention kernel (h3a_attn_fwd) with the oracle.

Reference behaviour: attn_sm80/fa3_sm80_h3.cu:252-458 (kernel), attn_sm80/bench_attn.py:22-33
(SDPA oracle + verify), attn_sm80/microtest.py:8-26 (fragment tests).
Tolerance (floating point): max|o-ref| <= 1e-2*absmax(ref), mean|o-ref| <= 1e-3*absmax(ref).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import h3attn
import oracle
from conftest import assert_close_absmax, from_dev_bf16, ramp_case, randn_bf16, to_dev_bf16

pytestmark = pytest.mark.gpu


def _run(q_bits, k_bits, v_bits, device):
    q, k, v = (to_dev_bf16(x, device) for x in (q_bits, k_bits, v_bits))
    o = h3attn.attn_fwd(q, k, v)
    torch.cuda.synchronize()
    return oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)


def test_version_and_attrs(gpu):
    assert h3attn.version().startswith("h3attn")
    regs, lds, blocks, clk, occ, threads = h3attn.kernel_attrs(0)
    assert threads in (256, 512) and regs > 0 and lds > 0 and blocks >= 1


def test_fragment_qk(gpu):
    """S = Q K^T on one wave (counterpart of test_qk, fa3_sm80_h3.cu:516-537)."""
    rng = np.random.default_rng(0)
    Q, K = randn_bf16(rng, (32, 128)), randn_bf16(rng, (64, 128))
    S = h3attn.test_qk(to_dev_bf16(Q, gpu), to_dev_bf16(K, gpu)).cpu().numpy()
    ref = oracle.bf16_to_f32(Q).reshape(32, 128).astype(np.float64) @ \
        oracle.bf16_to_f32(K).reshape(64, 128).astype(np.float64).T
    # bf16 x bf16 products are exact in fp32; only the fp32 summation order differs.
    assert np.abs(S - ref).max() <= 1e-5 * np.abs(ref).max()


def test_fragment_pv(gpu):
    """O = P V on one wave (counterpart of test_pv, fa3_sm80_h3.cu:539-560)."""
    rng = np.random.default_rng(1)
    P = oracle.f32_to_bf16(rng.random((32, 64)).astype(np.float32))
    V = randn_bf16(rng, (64, 128))
    O = h3attn.test_pv(to_dev_bf16(P, gpu), to_dev_bf16(V, gpu)).cpu().numpy()
    ref = oracle.bf16_to_f32(P).reshape(32, 64).astype(np.float64) @ \
        oracle.bf16_to_f32(V).reshape(64, 128).astype(np.float64)
    assert np.abs(O - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("B,H,Sq,Skv", [
    (1, 1, 1, 1), (1, 2, 7, 7), (1, 2, 64, 64), (1, 2, 65, 65), (1, 1, 129, 129),
    (1, 2, 200, 200), (2, 3, 128, 136), (1, 2, 64, 300), (1, 1, 300, 64), (1, 2, 1000, 1000),
    (1, 2, 1, 300), (2, 1, 1, 77), (2, 2, 300, 1),  # length-1 sequences (their stride reaches the ABI as 0)
])
def test_dense_vs_oracle(gpu, B, H, Sq, Skv):
    rng = np.random.default_rng(1000 + Sq * 7 + Skv)
    q = randn_bf16(rng, (B, H, Sq, 128))
    k = randn_bf16(rng, (B, H, Skv, 128))
    v = randn_bf16(rng, (B, H, Skv, 128))
    o = _run(q, k, v, gpu)
    assert_close_absmax(o, oracle.attn_fwd(q, k, v, round_p=True), what="vs oracle (bf16 P)")
    assert_close_absmax(o, oracle.attn_fwd(q, k, v, round_p=False), what="vs exact softmax")


def test_dense_h4_s2048_vs_oracle_and_sdpa(gpu):
    """B=1, H=4, S=2048, D=128, N(0,1) inputs, scale 1/sqrt(128) (the CPU-runnable case)."""
    rng = np.random.default_rng(2048)
    q, k, v = (randn_bf16(rng, (1, 4, 2048, 128)) for _ in range(3))
    o = _run(q, k, v, gpu)
    assert_close_absmax(o, oracle.attn_fwd(q, k, v), what="H=4 S=2048 vs oracle")
    qt, kt, vt = (to_dev_bf16(x, gpu).float() for x in (q, k, v))
    sd = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt).cpu().numpy()
    assert_close_absmax(o, sd, what="H=4 S=2048 vs fp32 SDPA")


@pytest.mark.parametrize("S", [1160, 4104])
def test_dense_tail_8_mod_128(gpu, S):
    """Sequence lengths = 8 (mod 128), as at S=42120: last query and key tiles hold 8 rows."""
    rng = np.random.default_rng(S)
    q, k = randn_bf16(rng, (1, 2, S, 128)), randn_bf16(rng, (1, 2, S, 128))
    v = randn_bf16(rng, (1, 2, S, 128), scale=4.0)
    o = _run(q, k, v, gpu)
    ref = oracle.attn_fwd(q, k, v)
    assert_close_absmax(o, ref, what=f"S={S}")
    assert_close_absmax(o[:, :, -8:], ref[:, :, -8:], what="tail rows")


def test_strided_fused_qkv_layout(gpu):
    """q,k,v read in place from a fused [S, 3*H*D] projection; O written as [1,S,H*D]."""
    S, H, D = 777, 4, 128
    g = torch.Generator(device="cpu").manual_seed(5)
    qkv = torch.randn(S, 3 * H * D, generator=g).to(torch.bfloat16).to(gpu)
    q, k, v = qkv.split(H * D, dim=-1)
    qv, kv, vv = (t.view(1, S, H, D).transpose(1, 2) for t in (q, k, v))
    out_shd = torch.empty(1, S, H, D, dtype=torch.bfloat16, device=gpu)
    o1 = h3attn.attn_fwd(qv, kv, vv, out=out_shd.transpose(1, 2))
    o2 = h3attn.attn_fwd(qv.contiguous(), kv.contiguous(), vv.contiguous())
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert torch.equal(out_shd.reshape(1, S, H * D), o2.transpose(1, 2).reshape(1, S, H * D))
    ref = oracle.attn_fwd(from_dev_bf16(qv), from_dev_bf16(kv), from_dev_bf16(vv))
    assert_close_absmax(o2.float().cpu().numpy(), ref, what="strided")


def test_single_key_returns_value(gpu):
    """One key: softmax weight is exactly 1, so O = V bit-for-bit."""
    rng = np.random.default_rng(7)
    q, k, v = randn_bf16(rng, (1, 3, 50, 128)), randn_bf16(rng, (1, 3, 1, 128)), randn_bf16(rng, (1, 3, 1, 128))
    o = h3attn.attn_fwd(*(to_dev_bf16(x, gpu) for x in (q, k, v)))
    ob = from_dev_bf16(o)
    assert np.array_equal(ob, np.broadcast_to(v, ob.shape))


def test_constant_value_rows(gpu):
    """V = c everywhere: O = c * sum(bf16(p)) / sum(p), within bf16 rounding of c."""
    rng = np.random.default_rng(8)
    q, k = randn_bf16(rng, (1, 2, 300, 128)), randn_bf16(rng, (1, 2, 300, 128))
    v = oracle.f32_to_bf16(np.full((1, 2, 300, 128), 1.5, np.float32))
    o = _run(q, k, v, gpu)
    assert np.abs(o - 1.5).max() <= 1.5 * 2.0 ** -7


@pytest.mark.parametrize("S,slope", [(300, 4 / 3), (1000, 0.4), (1000, 0.0383)])
def test_running_max_rises(gpu, S, slope):
    """Even query rows see scores rising steadily along the keys: 64*slope/sqrt(128)
    per key, i.e. ~700, ~210 and ~20 (log2 units) per 64-key stage for the three cases,
    ~3300 / ~3300 / ~310 in all.  exp2 against the first stage's max would overflow, so
    the running max is refreshed at every stage (all three: p may reach 2^16 between
    refreshes, and 20 log2 units per stage exceed that).  Odd rows fall and underflow
    to zero."""
    rng = np.random.default_rng(30)
    q, k, v = ramp_case(rng, S, slope=slope, q0=64.0)
    o = _run(q, k, v, gpu)
    assert np.isfinite(o).all()
    assert_close_absmax(o, oracle.attn_fwd(q, k, v, round_p=True), what="rising max")


@pytest.mark.parametrize("vscale,rise", [(1e16, 20.0), (1e28, 40.0), (1e30, 12.0)])
def test_large_values_with_rising_max(gpu, vscale, rise):
    """|v| far above activation scale while the running max rises `rise` log2 units per
    64-key stage (even rows; odd rows fall).  Between refreshes of the stale reference
    max p may reach 2^16, so O is bounded by 2^17 * ceil(S/64) * max|v| and stays finite
    for max|v| < 2^128 / (2^17 * ceil(S/64)), 8.1e31 at S = 2048 (the header's bound).
    A rise of 12 units per stage leaves p below the refresh limit for one stage and
    above it for the next, so both paths run at |v| = 1e30."""
    rng = np.random.default_rng(32)
    S = 2048
    q0 = 64.0
    slope = rise * math.sqrt(128) / (64 * q0 * math.log2(math.e))
    q, k, v = ramp_case(rng, S, slope=slope, q0=q0)
    v = oracle.f32_to_bf16(oracle.bf16_to_f32(v).reshape(v.shape) * np.float32(vscale))
    o = _run(q, k, v, gpu)
    assert np.isfinite(o).all(), "non-finite output"
    assert_close_absmax(o, oracle.attn_fwd(q, k, v, round_p=True), what=f"|v|~{vscale:g} rise {rise}")


def test_lone_dominant_key(gpu):
    """One key mid-sequence out-scores the rest by ~160 (log2 units): every row's output
    is that key's value row to bf16 rounding."""
    rng = np.random.default_rng(31)
    S = 777
    q = rng.standard_normal((1, 2, S, 128)).astype(np.float32) * 0.1
    k = rng.standard_normal((1, 2, S, 128)).astype(np.float32) * 0.1
    v = rng.standard_normal((1, 2, S, 128)).astype(np.float32)
    q[..., 0] = 64.0
    k[:, :, 500, 0] = 20.0
    q, k, v = (oracle.f32_to_bf16(x) for x in (q, k, v))
    o = _run(q, k, v, gpu)
    ref = oracle.attn_fwd(q, k, v, round_p=True)
    assert_close_absmax(o, ref, what="lone dominant key")
    vrow = oracle.bf16_to_f32(v).reshape(v.shape)[:, :, 500:501, :]
    assert np.abs(o - vrow).max() <= 2.0 ** -8 * np.abs(vrow).max()


def test_key_value_permutation_invariance(gpu):
    rng = np.random.default_rng(9)
    q, k, v = (randn_bf16(rng, (1, 2, 333, 128)) for _ in range(3))
    perm = rng.permutation(333)
    o1 = _run(q, k, v, gpu)
    o2 = _run(q, k[:, :, perm], v[:, :, perm], gpu)
    assert_close_absmax(o2, o1, what="permuted keys")


def test_value_power_of_two_scaling_is_exact(gpu):
    rng = np.random.default_rng(10)
    q, k, v = (randn_bf16(rng, (1, 2, 257, 128)) for _ in range(3))
    v2 = oracle.f32_to_bf16(oracle.bf16_to_f32(v).reshape(v.shape) * 2.0)
    o1 = _run(q, k, v, gpu)
    o2 = _run(q, k, v2, gpu)
    assert np.array_equal(o2, 2.0 * o1)


def test_batch_and_stream(gpu):
    """B > 1 is honoured (the reference ignored B) and work lands on the current stream."""
    rng = np.random.default_rng(11)
    q, k, v = (randn_bf16(rng, (3, 2, 150, 128)) for _ in range(3))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        qd, kd, vd = (to_dev_bf16(x, gpu) for x in (q, k, v))
        o = h3attn.attn_fwd(qd, kd, vd)
    s.synchronize()
    got = oracle.bf16_to_f32(from_dev_bf16(o)).reshape(o.shape)
    assert_close_absmax(got, oracle.attn_fwd(q, k, v), what="B=3 on side stream")


def _ref_fp32_heads(q, k, v, heads, scale, chunk=4096):
    """fp32 GPU reference softmax(q k^T * scale) v for selected heads, chunked over queries."""
    outs = []
    for h in heads:
        kt = k[0, h].float().t().contiguous()
        vf = v[0, h].float()
        rows = []
        for i0 in range(0, q.shape[2], chunk):
            s = (q[0, h, i0:i0 + chunk].float() @ kt) * scale
            rows.append(torch.softmax(s, dim=-1) @ vf)
        outs.append(torch.cat(rows, 0))
    return torch.stack(outs, 0)


@pytest.mark.parametrize("H", [56, 14])
def test_full_h3_shape(gpu, H):
    """H3 shape: B=1, S=42120 (512+256+2048+39304), D=128, H=56 and 14, q,k ~ N(0,1), v ~ 4 N(0,1)."""
    S = 42120
    g = torch.Generator(device=gpu).manual_seed(3)
    q = torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    k = torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    v = torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) * 4
    o = h3attn.attn_fwd(q, k, v)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all()
    heads = [0, H // 2, H - 1]
    ref = _ref_fp32_heads(q, k, v, heads, 1.0 / math.sqrt(128))
    got = o[0, heads].float()
    assert_close_absmax(got.cpu().numpy(), ref.cpu().numpy(), what=f"H={H} S={S}")
    assert_close_absmax(got[:, -8:].cpu().numpy(), ref[:, -8:].cpu().numpy(), what="tail tile")


def test_concurrent_host_threads_on_separate_streams(gpu):
    """Two host threads, each on its own stream, run queued dense and block-sparse
    launches at once (each call has its own workspace from torch's allocator on its
    stream, so its own queue counters, split partials and tile pair map).  Every result
    equals the same call made alone, bit for bit."""
    import threading

    from h3attn import ops, sla

    g = torch.Generator(device=gpu).manual_seed(21)
    H, S = 16, 16384  # 16 x 64 = 1024 dense tiles: a queued persistent launch
    inputs = [tuple(torch.randn(1, H, S, 128, generator=g, device=gpu, dtype=torch.bfloat16) for _ in range(3))
              for _ in range(2)]
    maps = [{blk: sla.get_block_map(q, k, 0.25, blk, blk, force_diag=True, want_map=False)[1:]
             for blk in (128, 64)} for q, k, _ in inputs]
    for i, (q, k, _) in enumerate(inputs):  # the tile path at 96x96 blocks
        bmap = sla.get_block_map(q, k, 0.25, 96, 96, force_diag=True, want_map=True)[0]
        maps[i][96] = ops.block_map_to_tile_lut(bmap, 96, 96, S, S)

    def calls(i):
        q, k, v = inputs[i]
        outs = [h3attn.attn_fwd(q, k, v)]
        for blk in (128, 64):
            lut, cnt = maps[i][blk]
            outs.append(h3attn.attn_fwd_blocksparse(q, k, v, lut, cnt, blk, blk))
        outs.append(ops.attn_fwd_blocksparse_tiles(q, k, v, *maps[i][96], queues=True))
        return outs

    alone = []
    for i in range(2):
        alone.append([o.clone() for o in calls(i)])
        torch.cuda.synchronize()

    results, errors = [None, None], []

    def worker(i):
        try:
            s = torch.cuda.Stream(device=gpu)
            with torch.cuda.stream(s):
                got = []
                for _ in range(3):
                    got.append(calls(i))
            s.synchronize()
            results[i] = got
        except Exception as e:  # surfaced in the main thread below
            errors.append(e)

    print("[threads] 2 host threads x 3 rounds of dense + sparse 128/64/96 at H=16 S=16384", flush=True)
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(2):
        for rnd in results[i]:
            for got, ref in zip(rnd, alone[i]):
                assert torch.equal(got, ref)
