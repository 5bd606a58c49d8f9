"""One H3 block's attention end to end at the fused-QKV layout: B=1, H=56, S=8192, D=128.

The workload: pre-norm q, k ~ N(0,1) scaled per token by U(0.5, 4); per-head RMSNorm
weights w ~ 1 + N(0, 0.05), eps 1e-6; 1-D RoPE with theta 10000 over the token index
(rot_dim 128); v ~ N(0,1).  As in the patched Attention.forward
(custom_nodes/h3_profiler/__init__.py:97-111, harness/sp_runtime.py:93-123):
rms_rope_split_half_ runs in place on the q/k views of the [S, 3*H*D] projection
output, then attention reads the transposed [1,H,S,D] views and writes O straight
into the [S, H*D] layout out_proj consumes.

Checks: the prologue output against the oracle's (one bf16 ulp); O on three heads
against the oracle's attention on the oracle's own prologue output (max error
<= 1e-2 * absmax, mean error <= 1e-3 * absmax); and every head against an fp32
torch reference on the kernel's prologue output.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import h3attn
import oracle
from conftest import assert_close_absmax, assert_prologue_close, from_dev_bf16, to_dev_bf16

pytestmark = pytest.mark.gpu


def test_fused_prologue_then_attention_h56_s8192(gpu):
    S, H, D = 8192, 56, 128
    HD = H * D
    rng = np.random.default_rng(20488192)
    print(f"[fused block] H={H} S={S}: generating inputs", flush=True)
    x = rng.standard_normal((S, 3 * HD), dtype=np.float32)
    x[:, :2 * HD] *= rng.uniform(0.5, 4.0, size=(S, 1)).astype(np.float32)  # q, k: per-token range
    w = (1.0 + 0.05 * rng.standard_normal((2, D))).astype(np.float32)
    xb, wb = oracle.f32_to_bf16(x), oracle.f32_to_bf16(w)
    rope = oracle.rope_table(S, D)

    qkv = to_dev_bf16(xb, gpu)  # [S, 3*H*D]
    q, k, v = qkv.split(HD, dim=-1)
    q4, k4 = q.view(1, S, H, D), k.view(1, S, H, D)
    rope_t = torch.from_numpy(rope).view(1, S, 1, D // 2, 2, 2).to(gpu)
    h3attn.rms_rope_split_half_(q4, k4, rope_t, to_dev_bf16(wb[0], gpu), to_dev_bf16(wb[1], gpu),
                                epsilon=1e-6, rot_dim=D)
    out = torch.empty(S, HD, dtype=torch.bfloat16, device=gpu)
    o = h3attn.attn_fwd(q4.transpose(1, 2), k4.transpose(1, 2), v.view(1, S, H, D).transpose(1, 2),
                        out=out.view(1, S, H, D).transpose(1, 2))
    torch.cuda.synchronize()
    assert o.data_ptr() == out.data_ptr()
    print("[fused block] kernels done; checking the prologue", flush=True)

    # 1) prologue vs the oracle's
    xq = xb[:, :HD].reshape(1, S, H, D)
    xk = xb[:, HD:2 * HD].reshape(1, S, H, D)
    rq, rk = oracle.qk_rmsnorm_rope(xq, xk, rope, wb[0], wb[1], eps=1e-6, rot_dim=D)
    gq, gk = from_dev_bf16(q4), from_dev_bf16(k4)
    assert_prologue_close(gq, rq, "q after the prologue")
    assert_prologue_close(gk, rk, "k after the prologue")
    assert np.array_equal(from_dev_bf16(v), xb[:, 2 * HD:]), "the prologue touched v"

    # 2) O on three heads vs the oracle's attention on the oracle's prologue output
    heads = [0, 27, 55]
    print(f"[fused block] oracle attention on heads {heads}", flush=True)
    vb = xb[:, 2 * HD:].reshape(S, H, D)
    qo = np.ascontiguousarray(rq[0][:, heads].transpose(1, 0, 2))[None]
    ko = np.ascontiguousarray(rk[0][:, heads].transpose(1, 0, 2))[None]
    vo = np.ascontiguousarray(vb[:, heads].transpose(1, 0, 2))[None]
    ref = oracle.attn_fwd(qo, ko, vo, round_p=False)[0]  # [3, S, D]
    got_all = oracle.bf16_to_f32(from_dev_bf16(out)).reshape(S, H, D)
    got = np.ascontiguousarray(got_all[:, heads].transpose(1, 0, 2))
    assert_close_absmax(got, ref, what="O vs oracle (3 heads)")

    # 3) every head vs fp32 torch on the kernel's own prologue output
    print("[fused block] fp32 reference on all heads", flush=True)
    scale = 1.0 / math.sqrt(D)
    qh, kh, vh = (t.view(S, H, D).transpose(0, 1) for t in (q, k, v))
    gout = out.view(S, H, D).transpose(0, 1)
    worst = 0.0
    for h in range(H):
        s = (qh[h].float() @ kh[h].float().t()) * scale
        r = torch.softmax(s, dim=-1) @ vh[h].float()
        mx, _, amax = assert_close_absmax(gout[h].float().cpu().numpy(), r.cpu().numpy(), what=f"head {h}")
        worst = max(worst, mx / amax)
    print(f"[fused block] worst max_err/absmax over heads: {worst:.3e}", flush=True)
