"""Write the golden fixtures of the attention path (tests/golden/*.npz).

The reference holds no usable golden vectors for this path (its fixtures are
gitignored .pt captures; microtest/bench use unsaved device-RNG inputs:
attn_sm80/microtest.py:8-23, attn_sm80/bench_attn.py:15-20), so the expected
outputs are computed here with torch on the CPU in float64 from seeded bf16
inputs, through code paths independent of the oracle:

  attn_*.npz     torch.nn.functional.scaled_dot_product_attention (fp64), the
                 reference's own oracle call (attn_sm80/bench_attn.py:22-24);
                 *_masked cases use SDPA's boolean attn_mask expanded from a
                 block map (the sparse path's definition, h3_sla:226-235).
  prologue_*.npz torch.nn.functional.rms_norm (fp64) and RoPE as a complex
                 rotation (x_i + i x_{i+rot/2}) * exp(i * pos * theta^(-2i/rot)),
                 rounded once to bf16.
  blockmap_*.npz mean pooling via reshape, scores in fp64, torch.topk.

Run: python tests/golden/make_golden.py   (deterministic; rewrites the files)
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16).to(torch.float64)


def attn_cases():
    cases = [(1, 1, 1, 1, 0), (1, 2, 7, 7, 1), (1, 1, 65, 65, 2), (2, 1, 33, 130, 3), (1, 2, 129, 64, 4)]
    for B, H, Sq, Skv, seed in cases:
        g = torch.Generator().manual_seed(seed)
        q = torch.randn(B, H, Sq, 128, generator=g)
        k = torch.randn(B, H, Skv, 128, generator=g)
        v = torch.randn(B, H, Skv, 128, generator=g)
        qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
        o = torch.nn.functional.scaled_dot_product_attention(from_bits(qb), from_bits(kb), from_bits(vb))
        np.savez_compressed(os.path.join(HERE, f"attn_{B}x{H}x{Sq}x{Skv}.npz"), q=qb, k=kb, v=vb,
                            o=o.numpy().astype(np.float64))


def attn_masked_cases():
    for (B, H, S, blk, seed) in [(1, 2, 200, 64, 10), (1, 1, 300, 128, 11)]:
        g = torch.Generator().manual_seed(seed)
        q, k, v = (torch.randn(B, H, S, 128, generator=g) for _ in range(3))
        nb = -(-S // blk)
        bmap = (torch.rand(B, H, nb, nb, generator=g) < 0.4).to(torch.uint8)
        bmap[..., 0] = 1  # at least one kept block per row
        qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
        mask = bmap.bool().repeat_interleave(blk, 2).repeat_interleave(blk, 3)[:, :, :S, :S]
        o = torch.nn.functional.scaled_dot_product_attention(from_bits(qb), from_bits(kb), from_bits(vb),
                                                             attn_mask=mask)
        np.savez_compressed(os.path.join(HERE, f"attn_masked_{S}_blk{blk}.npz"), q=qb, k=kb, v=vb,
                            block_map=bmap.numpy(), blk=blk, o=o.numpy())


def prologue_cases():
    for (S, H, rot, seed) in [(9, 2, 128, 20), (17, 3, 64, 21), (4, 1, 0, 22), (33, 2, 32, 23)]:
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(2, S, H, 128, generator=g) * (0.5 + 3.5 * torch.rand(2, S, 1, 1, generator=g))
        w = 1.0 + 0.05 * torch.randn(2, 128, generator=g)
        xb, wb = bf16_bits(x), bf16_bits(w)
        xf, wf = from_bits(xb), from_bits(wb)
        outs = []
        for t in range(2):
            y = torch.nn.functional.rms_norm(xf[t], (128,), weight=wf[t], eps=1e-6)
            if rot:
                half = rot // 2
                i = torch.arange(half, dtype=torch.float64)
                ang = torch.arange(S, dtype=torch.float64)[:, None] * (10000.0 ** (-2.0 * i / rot))[None, :]
                z = torch.complex(y[..., :half], y[..., half:rot]) * torch.exp(1j * ang)[:, None, :]
                y = torch.cat([z.real, z.imag, y[..., rot:]], dim=-1)
            outs.append(bf16_bits(y))
        np.savez_compressed(os.path.join(HERE, f"prologue_{S}x{H}_rot{rot}.npz"), q=xb[0], k=xb[1],
                            qw=wb[0], kw=wb[1], rot=rot, theta=10000.0, eps=1e-6,
                            q_out=outs[0], k_out=outs[1])


def blockmap_cases():
    for (S, H, blk, ratio, diag, seed) in [(700, 2, 64, 0.25, True, 30), (1000, 1, 128, 0.3, False, 31)]:
        g = torch.Generator().manual_seed(seed)
        q, k = (torch.randn(1, H, S, 128, generator=g) for _ in range(2))
        qb, kb = bf16_bits(q), bf16_bits(k)
        qf, kf = from_bits(qb), from_bits(kb)
        nb = -(-S // blk)
        pad = nb * blk - S

        def pool(x):
            xp = torch.nn.functional.pad(x, (0, 0, 0, pad))
            s = xp.reshape(1, H, nb, blk, 128).sum(3)
            cnt = torch.full((nb,), float(blk), dtype=torch.float64)
            cnt[-1] = blk - pad
            return s / cnt[None, None, :, None]

        scores = pool(qf) @ pool(kf).transpose(-1, -2)
        keep = max(1, int(ratio * nb))
        idx = torch.topk(scores, keep, dim=-1).indices
        bmap = torch.zeros(1, H, nb, nb, dtype=torch.uint8)
        bmap.scatter_(-1, idx, 1)
        if diag:
            ar = torch.arange(nb)
            bmap[:, :, ar, ar] = 1
        np.savez_compressed(os.path.join(HERE, f"blockmap_{S}_blk{blk}.npz"), q=qb, k=kb, blk=blk,
                            keep=keep, force_diag=diag, block_map=bmap.numpy())


if __name__ == "__main__":
    attn_cases()
    attn_masked_cases()
    prologue_cases()
    blockmap_cases()
    print("\n".join(sorted(f for f in os.listdir(HERE) if f.endswith(".npz"))))
